"""GPU parity of the fused qk-RMSNorm + rotary kernel (nva_qk_norm_rope) against
the CPU oracle (oracle/producer_oracle.py), through the C ABI.

Bar: the rotary-only path (no norm) is bit-exact.  With the norm, the kernel's sum
of squares runs in its own order, which can move the mean by an fp32 ulp and so a
normalised value x^ by one bf16 ulp before the rotation; an output may then differ
by at most what that ulp contributes, 2^-7 (|x^_i| + |x^_i+d/2|) (plus the output's
own rounding), and fewer than 1% of outputs may differ at all."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from _helpers import bits16, f32
from oracle import producer_oracle as PO

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def dev():
    assert torch.cuda.is_available(), "GPU tests need an MI355X"
    from nanovllm_amd import _capi
    _capi.load()
    return torch.device("cuda:0")


def _normed(case):
    """The oracle's normalised q and k (before the rotation), or the inputs without norm."""
    q, k = f32(case.q), f32(case.k)
    if case.q_norm_weight is None:
        return q, k
    return (PO.rms_norm_bf16(q, f32(case.q_norm_weight), case.eps),
            PO.rms_norm_bf16(k, f32(case.k_norm_weight), case.eps))


def _oracle(case, positions=None):
    pos = (case.positions if positions is None else positions).cpu().numpy()
    cs = case.cos_sin_cache.cpu().numpy()
    wq = None if case.q_norm_weight is None else f32(case.q_norm_weight)
    wk = None if case.k_norm_weight is None else f32(case.k_norm_weight)
    return PO.qk_norm_rope(f32(case.q), f32(case.k), pos, cs, wq, wk, case.eps)


def _run(case, inplace=False):
    from nanovllm_amd.layers.qk_norm_rope import qk_norm_rope
    q, k = qk_norm_rope(case.positions, case.q, case.k, case.cos_sin_cache, case.num_heads, case.num_kv_heads,
                        case.head_dim, case.q_norm_weight, case.k_norm_weight, case.eps, inplace=inplace)
    torch.cuda.synchronize()
    return q, k


def _ulps(got: torch.Tensor, ref: np.ndarray) -> np.ndarray:
    g = bits16(got).astype(np.int32)
    r = PO.f32_to_bf16_bits(ref.astype(np.float32)).astype(np.int32)
    return np.abs(g - r)


def _assert_close(got, ref, what, exact=False, xhat=None):
    u = _ulps(got, ref)
    frac = float((u > 0).mean())
    if exact:
        assert u.max() == 0, f"{what}: {int((u > 0).sum())} outputs differ (max {u.max()} ulp)"
        return frac
    g = f32(got).reshape(ref.shape)
    d = ref.shape[-1]
    pair = np.abs(xhat[..., : d // 2]) + np.abs(xhat[..., d // 2:])
    bound = 2.0 ** -7 * np.concatenate([pair, pair], axis=-1) + 2.0 ** -8 * np.abs(ref)
    err = np.abs(g - ref)
    assert (err <= bound).all() and frac < 0.01, \
        f"{what}: {int((err > bound).sum())} outside the one-ulp-of-x^ bound, {frac:.4%} differ"
    return frac


@pytest.mark.parametrize("nh,nkv", [(16, 8), (32, 8), (64, 8)])
def test_qwen3_shapes(dev, nh, nkv):
    from nanovllm_amd import workloads as W
    case = W.make_producer_case(333, nh, nkv, seed=nh, device=dev)
    q, k = _run(case)
    rq, rk = _oracle(case)
    xq, xk = _normed(case)
    fq = _assert_close(q, rq, f"q nh={nh}", xhat=xq)
    fk = _assert_close(k, rk, f"k nkv={nkv}", xhat=xk)
    print(f"nh={nh} nkv={nkv}: q differs {fq:.4%}, k {fk:.4%}")


def test_qwen2_rotary_only_head_dim_64(dev):
    from nanovllm_amd import workloads as W
    case = W.make_producer_case(257, 14, 2, head_dim=64, max_position=32768, rope_theta=1_000_000.0, norm=False,
                                seed=5, device=dev)
    q, k = _run(case)
    rq, rk = _oracle(case)
    _assert_close(q, rq, "q d=64", exact=True)
    _assert_close(k, rk, "k d=64", exact=True)


def test_head_dim_64_with_norm(dev):
    from nanovllm_amd import workloads as W
    case = W.make_producer_case(100, 8, 2, head_dim=64, seed=6, device=dev)
    q, k = _run(case)
    rq, rk = _oracle(case)
    xq, xk = _normed(case)
    _assert_close(q, rq, "q d=64 norm", xhat=xq)
    _assert_close(k, rk, "k d=64 norm", xhat=xk)


def test_inplace_matches_out_of_place(dev):
    from nanovllm_amd import workloads as W
    case = W.make_producer_case(64, 16, 8, seed=7, device=dev)
    q0, k0 = _run(case)
    q1, k1 = _run(case, inplace=True)
    assert q1.data_ptr() == case.q.data_ptr()
    assert torch.equal(q0, q1) and torch.equal(k0, k1)
    # v, which shares the qkv rows, is untouched
    nh, nkv, d = 16, 8, 128
    v_before = W.make_producer_case(64, 16, 8, seed=7, device=dev).qkv[:, (nh + nkv) * d:]
    assert torch.equal(case.qkv[:, (nh + nkv) * d:], v_before)


def test_token_counts_and_positions(dev):
    """Row counts that leave partial wavefronts, one token, and the position range ends."""
    from nanovllm_amd import workloads as W
    for T in (1, 2, 3, 5, 17):
        case = W.make_producer_case(T, 4, 1, seed=10 + T, device=dev)
        q, k = _run(case)
        rq, rk = _oracle(case)
        xq, xk = _normed(case)
        _assert_close(q, rq, f"T={T} q", xhat=xq)
        _assert_close(k, rk, f"T={T} k", xhat=xk)
    case = W.make_producer_case(4, 16, 8, max_position=128, positions=[0, 1, 126, 127], seed=3, device=dev)
    q, k = _run(case)
    rq, _ = _oracle(case)
    _assert_close(q, rq, "edge positions", xhat=_normed(case)[0])


def test_out_of_range_positions_are_clamped(dev):
    from nanovllm_amd import workloads as W
    case = W.make_producer_case(3, 16, 8, max_position=64, positions=[-5, 64, 1000], seed=4, device=dev)
    q, k = _run(case)
    rq, rk = _oracle(case, positions=torch.tensor([0, 63, 63]))
    xq, xk = _normed(case)
    _assert_close(q, rq, "clamped q", xhat=xq)
    _assert_close(k, rk, "clamped k", xhat=xk)


def test_config4_producer(dev):
    """The full config-4 token set (8813 tokens, heads 32/8) against the oracle."""
    from nanovllm_amd import workloads as W
    case = W.producer_config4(dev)
    q, k = _run(case)
    rq, rk = _oracle(case)
    xq, xk = _normed(case)
    fq = _assert_close(q, rq, "cfg4 q", xhat=xq)
    fk = _assert_close(k, rk, "cfg4 k", xhat=xk)
    print(f"cfg4 producer: q differs {fq:.4%}, k {fk:.4%}")


def test_graph_capture_replay(dev):
    from nanovllm_amd import workloads as W
    from nanovllm_amd.layers.qk_norm_rope import qk_norm_rope
    case = W.make_producer_case(48, 16, 8, seed=9, device=dev)
    q_out = torch.empty_like(case.q)
    k_out = torch.empty_like(case.k)
    eager_q, eager_k = _run(case)
    g = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        with torch.cuda.graph(g, stream=s):
            a, b = qk_norm_rope(case.positions, case.q, case.k, case.cos_sin_cache, 16, 8, 128,
                                case.q_norm_weight, case.k_norm_weight, case.eps)
            q_out.copy_(a)
            k_out.copy_(b)
    torch.cuda.current_stream().wait_stream(s)
    for _ in range(3):
        q_out.zero_()
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(q_out, eager_q) and torch.equal(k_out, eager_k)
