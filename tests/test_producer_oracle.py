"""Pins the producer oracle (oracle/producer_oracle.py: per-head RMSNorm and the
rotary embedding of qwen3.py:91-105) before it is trusted as the checker.

Independent statements:
  * the rotation as numpy complex multiplication (x1 + i x2) * exp(i p f) in float64;
  * every (x_i, x_{i+d/2}) pair keeps its norm; position 0 is the identity;
    rotating by p1 then p2 equals rotating by p1 + p2 (float64 cache);
  * RMSNorm: a unit-weight normalised row has RMS 1; a constant row maps to
    sign * weight; torch float32 ops and torch.nn.functional.rms_norm agree;
  * the cache against torch's own construction (the product's builder).
Planted mistakes (halves swapped, sin sign flipped, mean over the wrong axis,
eps dropped, weight skipped, wrong cache half) must each fail a check.
"""
from __future__ import annotations

import inspect
import types

import numpy as np
import pytest
import torch

from oracle import producer_oracle as P
from oracle.attention_oracle import bf16_bits_to_f32, f32_to_bf16_bits

RNG = np.random.default_rng(77)


def bf16_vals(*shape, scale=1.0):
    x = (RNG.standard_normal(shape) * scale).astype(np.float32)
    return bf16_bits_to_f32(f32_to_bf16_bits(x))


def cache64(d, n, base=10000.0):
    inv = 1.0 / (base ** (np.arange(0, d, 2, dtype=np.float64) / d))
    f = np.arange(n, dtype=np.float64)[:, None] * inv[None, :]
    return np.concatenate([np.cos(f), np.sin(f)], axis=-1)


def check_rope_complex(mod):
    d, T, H = 16, 7, 3
    x = bf16_vals(T, H, d)
    pos = RNG.integers(0, 50, T)
    cs = mod.rope_cos_sin(d, 64, 10000.0)
    got = mod.rope_bf16(x, pos, cs)
    z = x[..., : d // 2].astype(np.float64) + 1j * x[..., d // 2:].astype(np.float64)
    rot = np.exp(1j * np.angle(cs[pos, None, : d // 2] + 1j * cs[pos, None, d // 2:]).astype(np.float64))
    w = z * rot
    ref = np.concatenate([w.real, w.imag], axis=-1)
    assert np.abs(got - ref).max() <= 2.0 ** -7 * np.abs(ref).max() + 1e-6


def check_rope_invariants(mod):
    d, T = 32, 5
    x = bf16_vals(T, 2, d)
    cs = mod.rope_cos_sin(d, 128, 10000.0)
    # position 0: identity (cos 1, sin 0), so bf16 in -> same bf16 out
    assert np.array_equal(mod.rope_bf16(x, np.zeros(T, np.int64), cs), x)
    # pair norms preserved (up to the bf16 rounding of the outputs)
    y = mod.rope_bf16(x, np.arange(T), cs)
    n0 = np.hypot(x[..., : d // 2], x[..., d // 2:])
    n1 = np.hypot(y[..., : d // 2], y[..., d // 2:])
    assert np.abs(n0 - n1).max() <= 2.0 ** -7 * n0.max()
    # composition with a float64 cache: rotate(p1) o rotate(p2) == rotate(p1 + p2)
    c64 = cache64(d, 128).astype(np.float32)
    a = mod.rope_bf16(mod.rope_bf16(x, np.full(T, 3), c64), np.full(T, 4), c64)
    b = mod.rope_bf16(x, np.full(T, 7), c64)
    assert np.abs(a - b).max() <= 2.0 ** -6 * np.abs(b).max()


def check_cache(mod):
    cs = mod.rope_cos_sin(64, 512, 1_000_000.0)
    t_inv = 1.0 / (1_000_000.0 ** (torch.arange(0, 64, 2, dtype=torch.float) / 64))
    f = torch.einsum("i,j -> ij", torch.arange(512, dtype=torch.float), t_inv)
    ref = torch.cat((f.cos(), f.sin()), dim=-1).numpy()
    assert cs.shape == (512, 64)
    assert np.abs(cs - ref).max() < 1e-4


def check_rms(mod):
    d = 64
    x = bf16_vals(6, 3, d, scale=3.0)
    w = bf16_vals(d)
    got = mod.rms_norm_bf16(x, w, 1e-6)
    # torch float32 statement of layernorm.py:21-27
    xt = torch.from_numpy(x)
    var = xt.pow(2).mean(dim=-1, keepdim=True)
    ref = (xt * torch.rsqrt(var + 1e-6)).to(torch.bfloat16) * torch.from_numpy(w).to(torch.bfloat16)
    ref = ref.float().numpy()
    diff = np.abs(got - ref)
    assert diff.max() <= 2.0 ** -7 * np.abs(ref).max()
    assert (diff > 0).mean() < 0.02
    # library routine, no intermediate rounding: close, not bit-equal
    lib = torch.nn.functional.rms_norm(xt, (d,), torch.from_numpy(w), 1e-6).numpy()
    assert np.abs(got - lib).max() <= 2.0 ** -6 * np.abs(lib).max()
    # unit weight: RMS of each row is 1 (bf16 rounding aside)
    one = mod.rms_norm_bf16(x, np.ones(d, np.float32), 1e-6)
    rms = np.sqrt((one.astype(np.float64) ** 2).mean(-1))
    assert np.abs(rms - 1).max() < 1e-2
    # constant row c -> sign(c) * weight (eps negligible)
    c = np.full((1, 1, d), -2.5, np.float32)
    assert np.array_equal(mod.rms_norm_bf16(c, w, 1e-6)[0, 0], bf16_vals_like(-w))


def bf16_vals_like(x):
    return bf16_bits_to_f32(f32_to_bf16_bits(np.asarray(x, np.float32)))


def check_eps(mod):
    d = 16
    x = np.full((1, 1, d), 1e-4, np.float32)
    x = bf16_vals_like(x)
    w = np.ones(d, np.float32)
    got = mod.rms_norm_bf16(x, w, 1e-2)        # eps dominates: x / sqrt(1e-8 + 1e-2)
    ref = bf16_vals_like(x / np.sqrt(np.float32(np.mean(x * x)) + np.float32(1e-2)))
    assert np.array_equal(got, ref)


def check_fused(mod):
    T, nh, nkv, d = 4, 4, 2, 32
    q, k = bf16_vals(T, nh, d), bf16_vals(T, nkv, d)
    wq, wk = bf16_vals(d), bf16_vals(d)
    pos = np.array([0, 5, 17, 3])
    cs = mod.rope_cos_sin(d, 32, 10000.0)
    q2, k2 = mod.qk_norm_rope(q, k, pos, cs, wq, wk, 1e-6)
    assert np.array_equal(q2, mod.rope_bf16(mod.rms_norm_bf16(q, wq, 1e-6), pos, cs))
    assert np.array_equal(k2, mod.rope_bf16(mod.rms_norm_bf16(k, wk, 1e-6), pos, cs))
    q3, _ = mod.qk_norm_rope(q, k, pos, cs)   # no weights: rotary embedding alone
    assert np.array_equal(q3, mod.rope_bf16(q, pos, cs))
    # the q and k norms use their own weights
    assert not np.array_equal(q2, mod.qk_norm_rope(q, k, pos, cs, wk, wk, 1e-6)[0])
    assert mod.producer_bytes(10, 4, 2, 32) == 10 * 6 * 32 * 4 + 10 * (32 * 4 + 8) + 2 * 32 * 2


CHECKS = [check_rope_complex, check_rope_invariants, check_cache, check_rms, check_eps, check_fused]


@pytest.mark.parametrize("check", CHECKS, ids=[c.__name__ for c in CHECKS])
def test_producer_oracle_passes(check):
    check(P)


MUTANTS = {
    "halves_swapped": ("x1, x2 = x[..., : d // 2], x[..., d // 2:]", "x2, x1 = x[..., : d // 2], x[..., d // 2:]"),
    "sin_sign": ("y1 = (x1 * cos).astype(np.float32) - (x2 * sin).astype(np.float32)",
                 "y1 = (x1 * cos).astype(np.float32) + (x2 * sin).astype(np.float32)"),
    "cos_sin_halves": ("cos = cs[:, None, : d // 2]", "cos = cs[:, None, d // 2:]"),
    "mean_wrong_axis": ("var = np.mean(x * x, axis=-1, keepdims=True, dtype=np.float32)",
                        "var = np.mean(x * x, axis=-2, keepdims=True, dtype=np.float32)"),
    "eps_dropped": ("np.sqrt(var + np.float32(eps))", "np.sqrt(var)"),
    "weight_skipped": ("return bf16_round(y * np.asarray(weight_bf16, dtype=np.float32))", "return y"),
    "k_uses_q_weight": ("k = rms_norm_bf16(k, k_weight, eps)", "k = rms_norm_bf16(k, q_weight, eps)"),
    "freq_exponent": ("(np.arange(0, head_dim, 2, dtype=np.float64) / head_dim)",
                      "(np.arange(0, head_dim, 1, dtype=np.float64)[: head_dim // 2] / head_dim)"),
    "bytes_no_write": ("rows * head_dim * 2 * 2", "rows * head_dim * 2"),
}


def _mutant(old, new):
    src = inspect.getsource(P)
    assert src.count(old) >= 1, f"mutation anchor not found: {old!r}"
    mod = types.ModuleType("producer_mutant")
    exec(compile(src.replace(old, new), "producer_mutant", "exec"), mod.__dict__)
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
