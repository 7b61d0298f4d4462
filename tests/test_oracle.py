"""Pins the CPU oracle (oracle/attention_oracle.py) before it is trusted as the checker.

The reference ships no golden vectors for this path, so every oracle function is
checked against an independent statement of the same mathematics:
  * brute-force pure-Python float64 loops on tiny inputs;
  * torch.nn.functional.scaled_dot_product_attention (a library routine) with an
    explicit bottom-right mask;
  * closed forms: one visible key gives v0; q = 0 gives the mean of the visible V
    rows, which pins the causal alignment row by row;
  * invariants: decode == last prefill row, prefix prefill == tail of the full
    prefill, GQA == MHA with repeated K/V, page-permutation invariance;
  * formats: the e4m3fn table and encoder against torch.float8_e4m3fn, bf16
    rounding against torch, the store against index_copy_.
Then mistakes are planted in copies of the oracle's source (mask alignment, GQA
index, dropped scale or normaliser, transposed operand, store/encoder/slot
formula slips) and each must fail at least one of those checks.
"""
from __future__ import annotations

import importlib.util
import inspect
import math
import types

import numpy as np
import pytest
import torch

from oracle import attention_oracle as O

RNG = np.random.default_rng(1234)


# ----------------------------------------------------------------------------
# independent statements
# ----------------------------------------------------------------------------

def brute_attention(q, k, v, scale):
    Lq, nh, d = q.shape
    Lk, nkv, _ = k.shape
    grp = nh // nkv
    out = np.zeros((Lq, nh, d))
    for i in range(Lq):
        for h in range(nh):
            kh = h // grp
            lim = i + Lk - Lq
            idx = [j for j in range(Lk) if j <= lim]
            if not idx:
                continue
            sc = [sum(float(q[i, h, x]) * float(k[j, kh, x]) for x in range(d)) * scale for j in idx]
            m = max(sc)
            w = [math.exp(s - m) for s in sc]
            tot = sum(w)
            for x in range(d):
                out[i, h, x] = sum(w[t] * float(v[idx[t], kh, x]) for t in range(len(idx))) / tot
    return out


def sdpa_attention(q, k, v, scale):
    qt = torch.from_numpy(np.ascontiguousarray(q, dtype=np.float64)).permute(1, 0, 2)[None]
    kt = torch.from_numpy(np.ascontiguousarray(k, dtype=np.float64)).permute(1, 0, 2)[None]
    vt = torch.from_numpy(np.ascontiguousarray(v, dtype=np.float64)).permute(1, 0, 2)[None]
    Lq, Lk = q.shape[0], k.shape[0]
    mask = torch.ones(Lq, Lk, dtype=torch.bool).tril(diagonal=Lk - Lq)
    o = torch.nn.functional.scaled_dot_product_attention(qt, kt, vt, attn_mask=mask, scale=scale,
                                                         enable_gqa=True)
    return o[0].permute(1, 0, 2).numpy()


def rand(*shape):
    return RNG.standard_normal(shape)


# ----------------------------------------------------------------------------
# checks: each takes an oracle module and raises AssertionError on mismatch
# ----------------------------------------------------------------------------

def check_bruteforce(mod):
    for (Lq, Lk, nh, nkv, d) in [(3, 3, 2, 1, 4), (2, 5, 4, 2, 3), (4, 7, 4, 1, 5), (1, 6, 2, 2, 4)]:
        q, k, v = rand(Lq, nh, d), rand(Lk, nkv, d), rand(Lk, nkv, d)
        scale = 0.37
        got = mod.attention(q, k, v, scale, True, np.float64)
        np.testing.assert_allclose(got, brute_attention(q, k, v, scale), rtol=1e-10, atol=1e-12)


def check_sdpa(mod):
    for (Lq, Lk, nh, nkv, d) in [(17, 17, 8, 2, 16), (9, 40, 4, 4, 8), (33, 70, 16, 8, 32)]:
        q, k, v = rand(Lq, nh, d), rand(Lk, nkv, d), rand(Lk, nkv, d)
        scale = d ** -0.5
        got = mod.attention(q, k, v, scale, True, np.float64)
        np.testing.assert_allclose(got, sdpa_attention(q, k, v, scale), rtol=1e-9, atol=1e-11)


def check_closed_forms(mod):
    # one key: every row sees exactly v0
    k, v = rand(1, 2, 8), rand(1, 2, 8)
    q = rand(1, 4, 8)
    got = mod.attention(q, k, v, 0.5, True, np.float64)
    np.testing.assert_allclose(got, np.repeat(v, 2, axis=1), rtol=1e-12)
    # q = 0: uniform weights over the visible keys, bottom-right aligned
    Lq, Lk = 5, 12
    k, v = rand(Lk, 1, 6), rand(Lk, 1, 6)
    got = mod.attention(np.zeros((Lq, 2, 6)), k, v, 0.3, True, np.float64)
    for i in range(Lq):
        expect = v[: i + Lk - Lq + 1, 0].mean(axis=0)
        np.testing.assert_allclose(got[i, 0], expect, rtol=1e-12)
        np.testing.assert_allclose(got[i, 1], expect, rtol=1e-12)


def check_gqa_mha(mod):
    Lq, Lk, nh, nkv, d = 6, 9, 8, 2, 8
    q, k, v = rand(Lq, nh, d), rand(Lk, nkv, d), rand(Lk, nkv, d)
    grp = nh // nkv
    gqa = mod.attention(q, k, v, 0.25, True, np.float64)
    mha = mod.attention(q, np.repeat(k, grp, axis=1), np.repeat(v, grp, axis=1), 0.25, True, np.float64)
    np.testing.assert_allclose(gqa, mha, rtol=1e-12)


def _paged(rng, L, nkv, d, bs, npool):
    """Random paged layout holding K/V rows (L, nkv, d) at pages of a permutation."""
    k, v = rng.standard_normal((L, nkv, d)), rng.standard_normal((L, nkv, d))
    pages = math.ceil(L / bs)
    perm = rng.permutation(npool)[:pages]
    kc = rng.standard_normal((npool, bs, nkv, d))
    vc = rng.standard_normal((npool, bs, nkv, d))
    for j in range(L):
        kc[perm[j // bs], j % bs] = k[j]
        vc[perm[j // bs], j % bs] = v[j]
    bt = np.full(pages + 2, -1, dtype=np.int32)
    bt[:pages] = perm
    return k, v, kc, vc, bt


def check_decode_vs_prefill(mod):
    rng = np.random.default_rng(7)
    B, nh, nkv, d, bs = 3, 4, 2, 8, 4
    lens = [5, 9, 1]
    q = rng.standard_normal((B, nh, d))
    kcs, vcs, bts, full = [], [], [], []
    npool = 12
    kc = rng.standard_normal((npool, bs, nkv, d))
    vc = rng.standard_normal((npool, bs, nkv, d))
    perm = rng.permutation(npool)
    bt = np.full((B, 4), -1, dtype=np.int32)
    at = 0
    for b, L in enumerate(lens):
        n = math.ceil(L / bs)
        bt[b, :n] = perm[at:at + n]
        at += n
    out = mod.decode_attention(q, kc, vc, np.array(lens), bt, 0.4, dtype=np.float64)
    for b, L in enumerate(lens):
        ks = np.concatenate([kc[bt[b, j // bs], j % bs][None] for j in range(L)])
        vs = np.concatenate([vc[bt[b, j // bs], j % bs][None] for j in range(L)])
        # a prefill over L tokens whose last row is the decode query
        qq = rng.standard_normal((L, nh, d))
        qq[-1] = q[b]
        pre = brute_attention(qq, ks, vs, 0.4)
        np.testing.assert_allclose(out[b], pre[-1], rtol=1e-10, atol=1e-12)


def check_prefix_tail(mod):
    rng = np.random.default_rng(11)
    nh, nkv, d, bs = 4, 2, 8, 4
    prefix, Lq = 8, 6
    L = prefix + Lq
    k, v, kc, vc, bt = _paged(rng, L, nkv, d, bs, 10)
    q = rng.standard_normal((L, nh, d))
    full = mod.prefill_attention(q, k, v, [0, L], [0, L], 0.3, dtype=np.float64)
    tail = mod.prefill_attention(q[prefix:], kc, vc, [0, Lq], [0, L], 0.3, block_table=bt[None],
                                 dtype=np.float64)
    np.testing.assert_allclose(tail, full[prefix:], rtol=1e-10, atol=1e-12)
    np.testing.assert_allclose(full, brute_attention(q, k, v, 0.3), rtol=1e-10, atol=1e-12)


def check_page_invariance(mod):
    rng = np.random.default_rng(5)
    nh, nkv, d, bs, L = 2, 1, 4, 4, 11
    k, v, kc, vc, bt = _paged(rng, L, nkv, d, bs, 9)
    q = rng.standard_normal((1, nh, d))
    a = mod.decode_attention(q, kc, vc, np.array([L]), bt[None], 0.5, dtype=np.float64)
    b = brute_attention(q, k, v, 0.5)
    np.testing.assert_allclose(a[0], b[0], rtol=1e-10, atol=1e-12)
    # relabel pages: same answer
    perm = rng.permutation(kc.shape[0])
    inv = np.argsort(perm)
    bt2 = bt.copy()
    bt2[bt2 >= 0] = inv[bt2[bt2 >= 0]]
    a2 = mod.decode_attention(q, kc[perm], vc[perm], np.array([L]), bt2[None], 0.5, dtype=np.float64)
    np.testing.assert_allclose(a2, a, rtol=1e-12)


def check_store(mod):
    rng = np.random.default_rng(3)
    T, nkv, d, nb, bs = 9, 2, 4, 5, 4
    key = rng.integers(0, 65535, (T, nkv, d), dtype=np.uint16)
    val = rng.integers(0, 65535, (T, nkv, d), dtype=np.uint16)
    slots = rng.permutation(nb * bs)[:T].astype(np.int32)
    slots[2] = -1
    kc = np.full((nb, bs, nkv, d), 0xABCD, dtype=np.uint16)
    vc = np.full((nb, bs, nkv, d), 0x1234, dtype=np.uint16)
    mod.store_kvcache(key, val, kc, vc, slots)
    kt = torch.full((nb * bs, nkv * d), 0xABCD, dtype=torch.int32)
    vt = torch.full((nb * bs, nkv * d), 0x1234, dtype=torch.int32)
    keep = slots >= 0
    idx = torch.from_numpy(slots[keep].astype(np.int64))
    kt.index_copy_(0, idx, torch.from_numpy(key[keep].reshape(-1, nkv * d).astype(np.int32)))
    vt.index_copy_(0, idx, torch.from_numpy(val[keep].reshape(-1, nkv * d).astype(np.int32)))
    assert np.array_equal(kc.reshape(nb * bs, -1).astype(np.int32), kt.numpy())
    assert np.array_equal(vc.reshape(nb * bs, -1).astype(np.int32), vt.numpy())


def _fp8_probe_values():
    tab = O.e4m3fn_table()
    fin = tab[np.isfinite(tab)]
    fin = np.unique(fin)
    mids = (fin[1:] + fin[:-1]) / 2  # exact ties
    vals = np.concatenate([fin, mids, np.nextafter(mids, 0), np.nextafter(mids, 1e9),
                           [448, 460, 463.99, 464, 464.01, 479, 480, 500, 1e30, np.inf, -np.inf, np.nan,
                            2.0 ** -10, 2.0 ** -9 * 0.5, 2.0 ** -9 * 1.5, 1e-45, 0.0],
                           RNG.standard_normal(4000) * 100, RNG.standard_normal(4000) * 1e-2])
    vals = np.concatenate([vals, -vals]).astype(np.float32)
    return vals


def check_fp8(mod):
    tab = mod.e4m3fn_table()
    ref = torch.arange(256, dtype=torch.uint8).view(torch.float8_e4m3fn).to(torch.float64).numpy()
    both_nan = np.isnan(tab) & np.isnan(ref)
    assert np.array_equal(tab[~both_nan], ref[~both_nan]) and np.array_equal(np.isnan(tab), np.isnan(ref))
    vals = _fp8_probe_values()
    ours = mod.f32_to_e4m3fn(vals)
    theirs = torch.from_numpy(vals).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    assert np.array_equal(ours, theirs), np.flatnonzero(ours != theirs)[:10]


def check_bf16(mod):
    x = np.concatenate([RNG.standard_normal(10000).astype(np.float32) * 10,
                        np.array([np.inf, -np.inf, 0.0, -0.0, 3.0e38, 1e-40], dtype=np.float32)])
    ours = mod.f32_to_bf16_bits(x)
    theirs = torch.from_numpy(x).to(torch.bfloat16).view(torch.uint16).numpy() if hasattr(torch, "uint16") \
        else torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().astype(np.uint16)
    assert np.array_equal(ours, theirs)
    back = mod.bf16_bits_to_f32(ours)
    assert np.array_equal(back, torch.from_numpy(x).to(torch.bfloat16).float().numpy())


def check_slots(mod):
    # model_runner.py:180-188 with 3 cached pages of 4, seqlen 15 -> pages 3 (partial)
    row = [7, 2, 9, 4]
    assert mod.prefill_slots(row, 12, 15, 4) == [16, 17, 18]
    assert mod.prefill_slots(row, 0, 6, 4) == [28, 29, 30, 31, 8, 9]
    # model_runner.py:227-229: newest token of a 6-token sequence in pages [7, 2]
    assert mod.decode_slot(row, 6, 4) == 2 * 4 + 1
    assert mod.decode_slot(row, 8, 4) == 2 * 4 + 3
    assert mod.decode_slot(row, 9, 4) == 9 * 4 + 0


def check_flops(mod):
    lq, lk = [3, 5, 0], [3, 9, 4]
    cu_q = np.concatenate([[0], np.cumsum(lq)])
    cu_k = np.concatenate([[0], np.cumsum(lk)])
    pairs = sum(1 for a, b in zip(lq, lk) for i in range(a) for j in range(b) if j <= i + b - a)
    assert mod.prefill_flops(cu_q, cu_k, 2, 8) == 4 * 8 * 2 * pairs


CHECKS = [check_bruteforce, check_sdpa, check_closed_forms, check_gqa_mha, check_decode_vs_prefill,
          check_prefix_tail, check_page_invariance, check_store, check_fp8, check_bf16, check_slots,
          check_flops]


@pytest.mark.parametrize("check", CHECKS, ids=[c.__name__ for c in CHECKS])
def test_oracle_passes(check):
    check(O)


# ----------------------------------------------------------------------------
# planted mistakes: each mutant of the oracle's source must fail some check
# ----------------------------------------------------------------------------

MUTANTS = {
    "top_left_mask": ("visible = j <= i + (Lk - Lq)", "visible = j <= i"),
    "no_mask": ("visible = j <= i + (Lk - Lq)", "visible = j >= 0"),
    "gqa_mod_index": ("h = kh * grp + hg", "h = hg * nkv + kh"),
    "dropped_scale": ("s = (q[:, h, :] @ kk.T) * dtype(scale)", "s = (q[:, h, :] @ kk.T)"),
    "pv_uses_k": ("o = (p @ vv)", "o = (p @ kk)"),
    "no_normaliser": ("o = (p @ vv) / np.where(l > 0, l, 1)", "o = (p @ vv)"),
    "keys_reversed": ("kk = k[:, kh, :]  # (Lk, d)", "kk = k[::-1, kh, :]"),
    "values_of_other_head": ("vv = v[:, kh, :]", "vv = v[:, (kh + 1) % nkv, :]"),
    "gather_wrong_offset": ("return g[:length]", "return g[-length:] if length else g[:0]"),
    "store_swaps_kv": ("kf[s] = key[i].reshape(D)", "kf[s] = value[i].reshape(D)"),
    "store_no_skip": ("if 0 <= s < kf.shape[0]:", "if True:"),
    "fp8_floor_subnormal": ("q_sub = np.rint(a * 2.0 ** 9)", "q_sub = np.floor(a * 2.0 ** 9)"),
    "fp8_bias": ("normal_code = ((e + 7)", "normal_code = ((e + 8)"),
    "fp8_saturate": ("codes = np.where(overflow, 0x7F, codes)", "codes = np.where(overflow, 0x7E, codes)"),
    "decode_slot_off_by_one": ("return int(block_table_row[nblocks - 1]) * block_size + last - 1",
                               "return int(block_table_row[nblocks - 1]) * block_size + last"),
    "flops_square": ("pairs = lq * (lk - lq) + lq * (lq + 1) // 2", "pairs = lq * lk"),
    "bf16_truncate": ("rounded = (u + 0x7FFF + ((u >> 16) & 1)) >> 16", "rounded = u >> 16"),
}


def _mutant(old, new):
    src = inspect.getsource(O)
    assert src.count(old) >= 1, f"mutation anchor not found: {old!r}"
    src = src.replace(old, new)
    mod = types.ModuleType("oracle_mutant")
    exec(compile(src, "oracle_mutant", "exec"), mod.__dict__)
    return mod


@pytest.mark.parametrize("name", sorted(MUTANTS))
def test_planted_mistake_is_caught(name):
    mod = _mutant(*MUTANTS[name])
    caught = []
    for check in CHECKS:
        try:
            check(mod)
        except (AssertionError, ValueError, IndexError):
            caught.append(check.__name__)
    assert caught, f"mutant {name} passed every check"
