"""Host replay of the index arithmetic of the balanced split-K decode
(paged_decode_balanced_kernel + decode_merge_kernel in csrc/paged_decode.hip)
for the exact launches of the two shapes that faulted on the GPU -- fp8 at
head_dim 64 with 8-wave workgroups (heads 16/8), and the 2-wave workgroup at
heads 14/2 -- and for the shapes launched today.  Every shared-memory index
(s_wsum per WAVES, s_seg per scan chunk), every global address (q rows,
block-table entries, K/V cache bytes, the step prefix, partial slots b + r,
the merge's reads, output rows) is formed the way the kernel forms it and
checked against the allocation it falls in; the step partition must cover every
32-key step of every sequence exactly once, and the merge may read only partial
slots written in the same launch.  CPU only: nothing here launches a kernel.

The replay restates the kernel's integer math (plan_decode, used_ranges,
range_start, the two scans, decode_segment's loads and writes, the merge's slot
range); it pins that arithmetic against its own invariants, not against the
reference (the decode outputs are pinned by the GPU parity tests)."""
from __future__ import annotations

import math

import pytest
import torch

from nanovllm_amd import workloads as W

K_TARGET_WAVES = {False: 1024, True: 2048}
K_WAVES = {False: 4, True: 8}
K_MIN_RANGE_STEPS = 4


def waves_per_group(nkv, fp8, allow_two):
    w = K_WAVES[fp8]
    while w > 1 and w // 2 >= nkv:
        w //= 2
    return 1 if (w == 2 and not allow_two) else w


def plan(batch, nkv, max_blocks, block_size, fp8, allow_two):
    w = waves_per_group(nkv, fp8, allow_two)
    groups = -(-nkv // w)
    P = K_TARGET_WAVES[fp8] // (w * groups)
    max_steps = batch * ((max_blocks * block_size + 31) // 32)
    P = max(1, min(P, max_steps))
    return w, groups, P


def used_ranges(P, T):
    cap = T // K_MIN_RANGE_STEPS
    return 1 if cap < 1 else min(P, cap)


def range_start(r, T, P):
    return r * T // P


def replay(case, fp8, D, allow_two):
    B = case.batch
    nh, nkv = case.num_heads, case.num_kv_heads
    G = nh // nkv
    bt = case.block_tables.numpy()
    bs = case.block_size
    max_blocks = bt.shape[1]
    num_blocks = case.k_cache.shape[0] if case.k_cache is not None else int(bt.max()) + 1
    EB = 1 if fp8 else 2
    cache_bytes = num_blocks * bs * nkv * D * EB
    lane_offsets(fp8, D)
    w_, groups, Pplan = plan(B, nkv, max_blocks, bs, fp8, allow_two)
    WAVES = w_
    CH = 64 * WAVES
    lens = [max(0, min(L, max_blocks * bs)) for L in case.context_lens.tolist()]
    steps = [(L + 31) >> 5 for L in lens]
    rows = (B + Pplan) * nh  # workspace rows (nva_decode_workspace_bytes)
    ws_o_len, ws_ml_len, prefix_len = rows * D, rows * 2, B + 1
    written_slots = set()
    covered = [[0] * s for s in steps]
    direct = set()

    # pass 1 (every workgroup): chunked scan; workgroup (0, 0) writes the prefix
    prefix = [0] * (B + 1)
    T = 0
    for c0 in range(0, B, CH):
        for tid in range(CH):
            assert tid >> 6 < WAVES  # s_wsum[wave]
        chunk = [steps[b] if b < B else 0 for b in range(c0, c0 + CH)]
        acc = 0
        for i, st in enumerate(chunk):
            acc += st
            b = c0 + i
            if b < B:
                assert 0 <= b < prefix_len
                prefix[b] = T + acc - st
        T += acc
    prefix[B] = T
    P = used_ranges(Pplan, T)
    assert P <= Pplan  # grid.x = Pplan workgroups, ranges >= P return
    for kvg in range(groups):
        for r in range(Pplan):
            if r >= P:
                continue
            start, end = range_start(r, T, P), range_start(r + 1, T, P)
            if start >= end:
                continue
            carry = 0
            c0 = 0
            while c0 < B and carry < end:
                segs = []
                incl = 0
                for tid in range(CH):
                    b = c0 + tid
                    st = steps[b] if b < B else 0
                    incl += st
                    s0, s1 = carry + incl - st, carry + incl
                    if b < B and st > 0 and s0 < end and s1 > start:
                        segs.append((b, max(start, s0) - s0, min(end, s1) - s0))
                for pos in range(len(segs)):
                    assert 0 <= 3 * pos + 2 < 3 * CH  # s_seg
                for wave in range(WAVES):
                    kvh = kvg * WAVES + wave
                    if kvh >= nkv:
                        continue
                    for (sb, lo, hi) in segs:
                        whole = lo == 0 and hi == steps[sb]
                        k_begin, k_end = 32 * lo, min(32 * hi, lens[sb])
                        if kvh == 0:
                            for i in range(lo, hi):
                                covered[sb][i] += 1
                        segment(case, fp8, D, kvh, sb, k_begin, k_end, bt, bs, num_blocks, cache_bytes, G)
                        if whole:
                            direct.add(sb)
                        else:
                            slot = sb + r
                            assert slot < B + Pplan
                            for n in range(min(16, G)):
                                idx = slot * nh + kvh * G + n
                                assert 0 <= idx * D and idx * D + D <= ws_o_len
                                assert idx * 2 + 2 <= ws_ml_len
                            written_slots.add(slot)
                carry += incl
                c0 += CH
    # every step of every sequence in exactly one range
    for b in range(B):
        assert covered[b] == [1] * steps[b], f"sequence {b}: step coverage {covered[b]}"
    # merge: per (b, h) the slot range it reads, all written in this launch
    for b in range(B):
        s0, s1 = prefix[b], prefix[b + 1]
        if s1 <= s0:
            continue
        rf = ((s0 + 1) * P - 1) // T
        rl = (s1 * P - 1) // T
        if rf == rl:
            assert b in direct
            continue
        assert b not in direct
        for s in range(rl - rf + 1):
            rr = rf + s
            if range_start(rr, T, P) == range_start(rr + 1, T, P):
                continue
            slot = b + rf + s
            assert slot in written_slots, f"merge of sequence {b} reads unwritten slot {slot}"
            assert (slot * nh + nh - 1) * D + D <= ws_o_len
    return WAVES, P


def lane_offsets(fp8, D):
    """In-row byte offsets (and widths) every lane reads from a K and a V row,
    and the Q dims: the same for every step, so formed once."""
    EB = 1 if fp8 else 2
    k, v, q = [], [], []
    for lane in range(64):
        n, g = lane & 15, lane >> 4
        krow0 = 8 * (n >> 2) + (n & 3)
        for t in range(2):
            if fp8:
                k += [(krow0 + 4 * t, 64 * u + 16 * g, 16) for u in range(D // 64)]
            else:
                k += [(krow0 + 4 * t, (32 * s + 8 * g) * 2, 16) for s in range(D // 32)]
        if D == 128 or n < D // 8:
            width = 8 if fp8 else 16
            v += [(8 * g + r, width * n, width) for r in range(8)]
        for s in range(D // 32):
            q.append((n, (64 * (s >> 1) + 16 * g + 8 * (s & 1)) if fp8 else 32 * s + 8 * g))
    for (row, off, width) in k + v:
        assert 0 <= row < 32 and off + width <= D * EB  # inside the kv head's row of one key of the step
    for (_, dim) in q:
        assert dim + 8 <= D
    return k, v, q


def segment(case, fp8, D, kvh, b, k_begin, k_end, bt, bs, num_blocks, cache_bytes, G):
    """decode_segment's loads: the per-lane offsets inside a step are checked by
    lane_offsets; here each step's page, first row and 32-row span."""
    EB = 1 if fp8 else 2
    slot_bytes = case.num_kv_heads * D * EB
    kbase = kvh * D * EB
    assert (b * case.num_heads + kvh * G + min(16, G) - 1) * D + D <= case.batch * case.num_heads * D  # q rows
    nsteps = (k_end - k_begin + 31) >> 5
    for i in range(nsteps):
        key0 = k_begin + 32 * i
        blk = key0 // bs
        assert blk < bt.shape[1]  # block-table read
        page = int(bt[b, blk])
        ok = 0 <= page < num_blocks
        row0 = (page if ok else 0) * bs + (key0 - blk * bs)
        assert key0 - blk * bs + 31 < bs  # a step never straddles two pages
        assert kbase + row0 * slot_bytes >= 0 and kbase + (row0 + 31) * slot_bytes + D * EB <= cache_bytes


CASES = [
    # (nh, nkv, d, fp8, allow_two_waves): the faulted launches first
    (16, 8, 64, True, False),   # fp8, 8 waves, head_dim 64
    (14, 2, 64, True, True),    # the 2-wave workgroup, fp8
    (14, 2, 64, False, True),   # the 2-wave workgroup, bf16
    (14, 2, 128, False, True),
    (14, 2, 64, False, False),  # what serves 14/2 today: one wave per workgroup
    (16, 8, 128, True, False),
    (16, 8, 128, False, False),
    (64, 8, 64, False, False),
]


@pytest.mark.parametrize("nh,nkv,d,fp8,two", CASES)
def test_balanced_decode_indices_in_bounds(nh, nkv, d, fp8, two):
    lengths = [1, 2, 31, 33, 256, 257, 700, 1025, 0, 3000]  # the faulted tests' lengths and table
    case = W.make_decode_case(len(lengths), nh, nkv, 0, 0, 40, fp8=fp8, seed=640, head_dim=d, bulk_device=None,
                              lengths=lengths, table_width=12)
    case.k_cache = torch.empty((40, 256, nkv, d), dtype=torch.uint8 if fp8 else torch.bfloat16, device="meta")
    waves, P = replay(case, fp8, d, two)
    if two:
        assert waves == 2
    assert P >= 1


@pytest.mark.parametrize("B,lo,hi", [(1300, 0, 300), (64, 16384, 32768), (256, 100, 2048), (3, 0, 40)])
def test_balanced_decode_indices_many_shapes(B, lo, hi):
    """Scan chunks (B above 64 * WAVES), the config-5 and config-3 shapes, tiny batches."""
    for fp8, d, nh, nkv, two in ((False, 128, 16, 8, False), (True, 128, 64, 8, False), (True, 64, 16, 8, False),
                                 (False, 64, 14, 2, True)):
        g = torch.Generator().manual_seed(B + d)
        lengths = torch.randint(lo, hi + 1, (B,), generator=g).tolist()
        width = max(1, -(-max(lengths) // 256))
        pool = sum(-(-L // 256) for L in lengths) + 1
        case = W.make_decode_case(B, nh, nkv, 0, 0, pool, seed=B, head_dim=d, bulk_device=None, lengths=lengths,
                                  table_width=width)
        case.k_cache = torch.empty((pool, 256, nkv, d), dtype=torch.uint8, device="meta")
        replay(case, fp8, d, two)


# ---------------------------------------------------------------------------
# Spread mode (paged_decode_spread_kernel, plan_decode's small-batch branch).
K_SPREAD_MAX_PAIRS, K_SPREAD_TARGET, K_MAX_BLOCKS, K_SPREAD_MAX_SHARES = 256, 1024, 64, 16


def spread_plan(batch, nkv, max_blocks, block_size):
    pairs = batch * nkv
    if pairs > K_SPREAD_MAX_PAIRS or max_blocks > K_MAX_BLOCKS:
        return None
    table_steps = (max_blocks * block_size + 31) // 32
    return max(1, min(K_SPREAD_TARGET // pairs, table_steps, K_SPREAD_MAX_SHARES))


def replay_spread(lengths, nh, nkv, D, max_blocks, block_size):
    B = len(lengths)
    S = spread_plan(B, nkv, max_blocks, block_size)
    assert S is not None
    G = nh // nkv
    rows = B * S * nh if S > 1 else 0  # workspace rows: partial_slots * nh
    for b, L in enumerate(lengths):
        ctx = max(0, min(L, max_blocks * block_size))
        steps = (ctx + 31) >> 5
        per = (steps + S - 1) // S if steps > 0 else 1
        shares = (steps + per - 1) // per
        direct = shares <= 1
        covered = []
        for kvh in range(nkv):
            for r in range(S):  # grid.x
                if r >= (1 if direct else shares):
                    continue
                k0, k1 = min(ctx, 32 * per * r), min(ctx, 32 * per * (r + 1))
                assert direct or k1 > k0, "a counted share must hold keys"
                if kvh == 0:
                    covered += list(range(k0, k1))
                for key0 in range(k0, k1, 32):
                    assert key0 // block_size < max_blocks <= 64  # readlane of the hoisted row
                if not direct:
                    slot = b * S + r
                    for n in range(G):
                        idx = slot * nh + kvh * G + n
                        assert (idx + 1) * D <= rows * D and (idx + 1) * 2 <= rows * 2
            if not direct:  # decode_merge_kernel reads shares 0 .. shares-1
                for s in range(shares):
                    assert (b * S + s + 1) * nh * D <= rows * D
        assert covered == list(range(ctx)), f"sequence {b}: keys covered once, in order"
    return S


@pytest.mark.parametrize("nh,nkv,d", [(16, 8, 128), (14, 2, 64), (8, 1, 128), (128, 8, 128)])
def test_spread_decode_indices(nh, nkv, d):
    for B in (1, 3, 256 // nkv):
        g = torch.Generator().manual_seed(B * 31 + nh)
        for bs, width in ((256, 16), (64, 64), (32, 5), (256, 64)):
            lengths = torch.randint(0, width * bs + 40, (B,), generator=g).tolist()
            lengths[0] = width * bs
            if B > 2:
                lengths[1], lengths[2] = 0, 1
            replay_spread(lengths, nh, nkv, d, width, bs)
