"""The streaming scoring kernel's selection scheme, restated on the CPU and
checked against the oracle's stable top-k.

pkm_score_topk's streaming kernel (modelos_amd/csrc/score_topk.hip, namespace
stream) selects each token's per-half top-knn of bfloat16 scores without
sorting a row: each token's keys are split between two lanes, each with a
sorted running list T of 32 unique keys, a threshold bound shared by the two
lanes and a final merge of their lists; an admission test of every score
against a float threshold, LDS slots for the
admitted scores, merges of 32-slot chunks through Batcher's odd-even merge
sort and a half-cleaner cascade, decided for 256 tokens at a time. The GPU
tests check the kernel's outputs; this file checks the scheme itself, on many
more inputs than a GPU run covers (tie-heavy rows, +0 / -0, every knn, key
orders that fill the slots fastest), so that an error in the scheme (a key
map that misorders two values, a threshold that rejects a key that belongs
in the list, a network that does not sort, a slot budget that overflows) fails
here without a GPU:

  * the key map (raw_key) orders raw words as (value desc, index asc), with
    -0 equal to +0, and key_to_okey16 gives the bf16 order key;
  * the threshold (raw_floor) admits every key >= theta, on all bf16 values;
  * the two networks sort (0-1 principle, exhaustively for the merge step);
  * the whole per-token stream, with the kernel's block order, pipelining,
    workgroup-wide merge decisions, slot budget and final drain, returns the
    oracle's per-half top-knn (values and indices, ties by index).

The restatement follows the kernel's code line by line (its constants are
read from its source, so a change there is seen here); the oracle is
oracle/pkm.py's topk_stable.
"""
from __future__ import annotations

import os
import re

import numpy as np
import pytest
import torch

from oracle import pkm as ref
from tests.helpers import gen

SRC = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "modelos_amd", "csrc",
                   "score_topk.hip")


def _const(name: str) -> int:
    """A constant of the kernel's namespace, read from its source."""
    with open(SRC) as f:
        src = f.read()
    body = src[src.index("namespace stream {"):src.index("}  // namespace stream")]
    m = re.search(r"constexpr int %s = (\d+)( \* kWaves)?;" % name, body)
    assert m, name
    return int(m.group(1)) * (_const("kWaves") if m.group(2) else 1)


K_BUF, K_TRIGGER, K_KB, K_TOK, K_NET = (_const(x) for x in ("kBuf", "kTrigger", "kKB", "kTok", "kNet"))
U32 = np.uint32
M32 = 0xFFFFFFFF


# --- key map -----------------------------------------------------------------

def raw_words(bits: np.ndarray, idx: np.ndarray) -> np.ndarray:
    """Slot word of a score: bf16 bits << 16 | (0xFFFF - index)."""
    return ((bits.astype(np.int64) << 16) | (0xFFFF - idx.astype(np.int64))).astype(U32)


def raw_key(r: np.ndarray) -> np.ndarray:
    r = r.astype(np.int64)
    sgn = np.where(r >> 31, 0xFFFFFFFF, 0)
    return (((r ^ ((sgn & 0x7FFF0000) | 0x80000000)) + ((r >> 31) << 16)) & M32).astype(U32)


def key_to_okey16(k: np.ndarray) -> np.ndarray:
    k = k.astype(np.int64)
    return (k - np.where(k < 0x80000000, 0x10000, 0)).astype(U32)


def raw_floor(th: np.ndarray) -> np.ndarray:
    th = np.asarray(th).astype(np.int64)
    ok = th >> 16
    b = np.where(ok > 0x8000, ok - 0x8000, 0x10000 - ok) & 0xFFFF
    w = (b << 16) | np.where(b & 0x8000, 0xFFFF, 0)
    w = np.where(ok == 0, 0xFFFFFFFF, w)
    return w.astype(U32).view(np.float32)


def bf16_order_key(bits: np.ndarray) -> np.ndarray:
    """The usual order-preserving map of bf16 bits (okey16): sign set ->
    inverted bits, else bits | 0x8000."""
    bits = bits.astype(np.int64)
    return np.where(bits & 0x8000, 0xFFFF - bits, bits | 0x8000)


def all_finite_bf16() -> np.ndarray:
    b = np.arange(0x10000, dtype=np.int64)
    exp = (b >> 7) & 0xFF
    return b[exp != 0xFF]


def test_raw_key_orders_value_then_index():
    bits = all_finite_bf16()
    vals = torch.from_numpy(bits.astype(np.int16)).view(torch.bfloat16).float().numpy()
    rng = np.random.default_rng(1)
    i = rng.integers(0, 2048, size=bits.size)
    k = raw_key(raw_words(bits, i)).astype(np.int64)
    # the high half is the value's rank, equal for equal values (+0 and -0 included)
    hi = k >> 16
    order = np.argsort(vals, kind="stable")
    v_s, h_s = vals[order], hi[order]
    assert np.all(np.diff(h_s)[np.diff(v_s) > 0] > 0)
    assert np.all(np.diff(h_s)[np.diff(v_s) == 0] == 0)
    assert hi.min() >= 1, "0 is no value's key (T starts at 0)"
    # the low half orders equal values by index, smaller first
    assert np.array_equal(k & 0xFFFF, 0xFFFF - i)
    # okey16 of every value but -0, which leaves as +0
    ok = key_to_okey16(k.astype(U32)).astype(np.int64) >> 16
    want = bf16_order_key(np.where(bits == 0x8000, 0, bits))
    assert np.array_equal(ok, want)


def test_raw_floor_admits_every_key_at_or_above_theta():
    bits = all_finite_bf16()
    rng = np.random.default_rng(2)
    # every finite value as theta, against words of every finite value
    th = raw_key(raw_words(bits, rng.integers(0, 2048, size=bits.size)))
    tau = raw_floor(th)
    for shift in range(0, bits.size, 4099):
        cand_bits = np.roll(bits, shift)
        cand_idx = rng.integers(0, 2048, size=bits.size)
        r = raw_words(cand_bits, cand_idx)
        k = raw_key(r)
        passed = ~(r.view(np.float32) < tau)
        assert np.all(passed[k >= th]), "a key >= theta was rejected"
        # only equal-valued keys below theta may pass: different values are cut
        assert not np.any(passed & (k < th) & ((k >> 16) != (th >> 16)))
    # theta = 0 (fewer than knn merged): NaN, every word passes
    r = raw_words(bits, rng.integers(0, 2048, size=bits.size))
    assert np.all(~(r.view(np.float32) < raw_floor(np.zeros(1, dtype=np.int64))))


# --- networks ----------------------------------------------------------------

def oem_net(N):
    net = []
    p = 1
    while p < N:
        k = p
        while k >= 1:
            j = k % p
            while j + k < N:
                for i in range(k):
                    if i + j + k >= N:
                        break
                    if (i + j) // (2 * p) == (i + j + k) // (2 * p):
                        net.append((i + j, i + j + k))
                j += 2 * k
            k >>= 1
        p <<= 1
    return net


def clean_net(N):
    net = []
    j = N // 2
    while j >= 1:
        net += [(i, i + j) for i in range(N) if not (i & j)]
        j >>= 1
    return net


SORT32, SORT16, CLEAN32 = oem_net(32), oem_net(16), clean_net(32)


def run_net(x: np.ndarray, net) -> np.ndarray:
    """Descending compare-exchanges on columns of x [rows, 32]."""
    x = x.copy()
    for a, b in net:
        hi, lo = np.maximum(x[:, a], x[:, b]), np.minimum(x[:, a], x[:, b])
        x[:, a], x[:, b] = hi, lo
    return x


def test_network_sizes_match_the_kernel():
    with open(SRC) as f:
        src = f.read()
    assert "kSort32.n == %d && kSort16.n == %d && kClean32.n == %d" % (len(SORT32), len(SORT16), len(CLEAN32)) in src
    assert (len(SORT32), len(SORT16), len(CLEAN32)) == (191, 63, 80)


def test_sort32_sorts():
    rng = np.random.default_rng(3)
    # 0-1 inputs: all with <= 2 ones or <= 2 zeros, and random ones
    rows = []
    for a in range(32):
        for b in range(a, 32):
            z = np.zeros(32, dtype=np.int64)
            z[[a, b]] = 1
            rows += [z, 1 - z]
    rows = np.stack(rows + list(rng.integers(0, 2, size=(60000, 32))))
    assert np.array_equal(run_net(rows, SORT32), -np.sort(-rows, axis=1))
    # keys with ties
    x = rng.integers(0, 8, size=(20000, 32))
    assert np.array_equal(run_net(x, SORT32), -np.sort(-x, axis=1))


def test_sort16_sorts():
    # 0-1 principle, exhaustive over the 2^16 inputs
    rows = (np.arange(1 << 16)[:, None] >> np.arange(16)[None, :]) & 1
    assert np.array_equal(run_net(rows, SORT16), -np.sort(-rows, axis=1))


def test_merge16_step_keeps_the_best_32_sorted():
    # 0-1 principle, exhaustive: T = 1^a 0^(32-a), C = 1^b 0^(16-b); C reversed
    # meets T[16 .. 32) only
    T = np.array([[1] * a + [0] * (32 - a) for a in range(33) for _ in range(17)])
    C = np.array([[1] * b + [0] * (16 - b) for _ in range(33) for b in range(17)])
    M = T.copy()
    M[:, 16:] = np.maximum(M[:, 16:], C[:, ::-1])
    M = run_net(M, CLEAN32)
    want = -np.sort(-np.concatenate([T, C], axis=1), axis=1)[:, :32]
    assert np.array_equal(M, want)


def test_merge_step_keeps_the_best_32_sorted():
    # 0-1 principle, exhaustive: T = 1^a 0^(32-a), C = 1^b 0^(32-b), both sorted desc
    T = np.array([[1] * a + [0] * (32 - a) for a in range(33) for _ in range(33)])
    C = np.array([[1] * b + [0] * (32 - b) for _ in range(33) for b in range(33)])
    M = run_net(np.maximum(T, C[:, ::-1]), CLEAN32)
    want = -np.sort(-np.concatenate([T, C], axis=1), axis=1)[:, :32]
    assert np.array_equal(M, want)


# --- the per-token stream ------------------------------------------------------

def word_key(w: int) -> int:
    return 32 * (w >> 3) + 8 * ((w & 7) >> 1) + 2 * (w & 1)


K_WPB = K_KB // 4  # words per block and lane
K_SPLITS = (12, 16, 20)
# a block's keys of each lane of a token (lane half hl = lane / 32), in append
# order: words in order, each its two keys; the raw words carry index' = key - 4 hl
BLOCK_KEYS = [[word_key(w) + 4 * hl + v for w in range(K_WPB) for v in range(2)] for hl in (0, 1)]


def stream_select(bits: np.ndarray, knn: int, stats: dict | None = None) -> np.ndarray:
    """The kernel's selection for the tokens of one workgroup (rows of bits
    [tokens <= 256, n], bf16 scores of one half): returns the okey16-form
    lists [tokens, knn] (okey16 << 16 | 0xFFFF - index). Lane t * 2 + hl here
    is lane t % 32 + 32 hl of wave t // 32 in the kernel."""
    L, n = bits.shape
    assert L <= K_TOK and n % K_KB == 0
    assert sorted(BLOCK_KEYS[0] + BLOCK_KEYS[1]) == list(range(K_KB))
    nb = n // K_KB
    NL = 2 * L
    hl = np.arange(NL) % 2
    tok = np.arange(NL) // 2
    T = np.zeros((NL, K_NET), dtype=U32)
    buf = np.zeros((NL, K_BUF), dtype=U32)
    cnt = np.zeros(NL, dtype=np.int64)
    lanes = np.arange(NL)
    tau = np.full(NL, np.inf, dtype=np.float32)

    def merge_chunk(j0, rows, width_rule):
        C = np.zeros((NL, 32), dtype=U32)
        hi = min(j0 + 32, K_BUF)
        C[:, :hi - j0] = raw_key(buf[:, j0:hi])
        C = np.where(np.arange(j0, j0 + 32)[None, :] < cnt[:, None], C, U32(0)).astype(U32)
        for w0 in range(0, NL, 64):  # each wave picks its chunk width
            r = np.intersect1d(np.arange(w0, min(w0 + 64, NL)), rows)
            if r.size == 0:
                continue
            if width_rule(r):
                T[r] = run_net(np.maximum(T[r], run_net(C[r], SORT32)[:, ::-1]), CLEAN32)
            else:  # 16 wide: slots j0 + 16 .. are past every count of the wave (or the buffer)
                assert np.all(cnt[r] <= j0 + 16)
                C16 = run_net(C[r, :16], SORT16)
                M = T[r].copy()
                M[:, 16:] = np.maximum(M[:, 16:], C16[:, ::-1])
                T[r] = run_net(M, CLEAN32)
            if stats is not None:
                key = "w32" if width_rule(r) else "w16"
                stats[key] = stats.get(key, 0) + 1

    def tau_of():
        th = T[:, K_NET - 1].astype(np.int64)
        lo, hi_ = T[0::2].astype(np.int64), T[1::2].astype(np.int64)  # the token's two lanes
        bound = np.max(np.stack([np.minimum(lo[:, a - 1], hi_[:, 31 - a]) for a in K_SPLITS]), axis=0)
        th = np.maximum(th, np.repeat(bound, 2))
        return raw_floor(th)

    def merge(rows):
        # every slot: [0, 32), then [32, kBuf) in the waves where a lane holds more than 32
        merge_chunk(0, rows, lambda r: np.any(cnt[r] > 16))
        second = np.array([w for w in rows if np.any(cnt[(w // 64) * 64:(w // 64) * 64 + 64] > 32)], dtype=np.int64)
        if second.size:
            merge_chunk(32, second, lambda r: False)
        cnt[rows] = 0

    tau_first = None
    for j in range(nb + 1):
        if j == 0:
            # the first block's 32 scores of a lane, sorted, are T
            keys = np.array(BLOCK_KEYS[0])  # index' of the lane's append positions
            tk = keys[None, :] + 4 * hl[:, None]
            r = raw_words(bits[tok[:, None], tk], np.broadcast_to(keys, tk.shape))
            T[:] = run_net(raw_key(r), SORT32)
            tau_first = tau_of()
        if j >= 1:
            # the appends of block j - 1's words, during block j (or the drain)
            for q in range(K_WPB):
                k0 = (j - 1) * K_KB + word_key(q)  # index' of the word's first score
                # a word's two scores: slot cnt takes the first if it passes,
                # else the second; slot cnt + 1 takes the second (both are
                # written whether or not they count)
                # (block 0's words are zeroed once sorted into T)
                w0_ = np.zeros(NL, np.int64) if j == 1 else bits[tok, k0 + 4 * hl]
                w1_ = np.zeros(NL, np.int64) if j == 1 else bits[tok, k0 + 4 * hl + 1]
                r0 = raw_words(w0_, np.full(NL, k0))
                r1 = raw_words(w1_, np.full(NL, k0 + 1))
                p0 = ~(r0.view(np.float32) < tau)
                p1 = ~(r1.view(np.float32) < tau)
                assert cnt.max() + 2 <= K_BUF, "both slots of a word inside the buffer"
                buf[lanes, cnt] = np.where(p0, r0, r1)
                buf[lanes, cnt + 1] = r1
                cnt += p0.astype(np.int64) + p1.astype(np.int64)
                if stats is not None:
                    stats["max_cnt"] = max(stats.get("max_cnt", 0), int(cnt.max()))
        if j == 1:
            tau[:] = tau_first  # block 0's words (in T, then zeroed) were appended against +inf
        if j < nb:
            if np.any(cnt >= K_TRIGGER):  # the workgroup merges together
                merge(lanes)
                tau[:] = tau_of()
            assert cnt.max() <= K_TRIGGER - 1, "slot budget: a block starts with <= kTrigger - 1 slots"
        else:
            for w0 in range(0, NL, 64):  # each wave drains its own slots
                rows = lanes[w0:w0 + 64]
                if np.any(cnt[rows] > 0):
                    merge(rows)
            assert cnt.max() == 0
    # the token's list: true indices (0xFFFF - index is 4 lower in the upper
    # lane), then the pair merge max(T_lo[i], T_hi[31 - i]) and the cleaner
    Tt = np.where((hl[:, None] == 1) & (T != 0), T.astype(np.int64) - 4, T.astype(np.int64)).astype(U32)
    lo, hi_ = Tt[0::2], Tt[1::2]
    M = run_net(np.maximum(lo, hi_[:, ::-1]), CLEAN32)
    return key_to_okey16(M[:, :knn])


def check_rows(bits: np.ndarray, knn: int):
    lists = stream_select(bits, knn)
    vals = torch.from_numpy(bits.astype(np.int16)).view(torch.bfloat16)
    e_v, e_i = ref.topk_stable(vals, knn)
    got_i = 0xFFFF - (lists.astype(np.int64) & 0xFFFF)
    got_ok = lists.astype(np.int64) >> 16
    assert np.array_equal(got_i, e_i.numpy())
    e_bits = e_v.view(torch.int16).numpy().astype(np.int64) & 0xFFFF
    assert np.array_equal(got_ok, bf16_order_key(np.where(e_bits == 0x8000, 0, e_bits)))


def bf16_bits(x: torch.Tensor) -> np.ndarray:
    return x.to(torch.bfloat16).view(torch.int16).numpy().astype(np.int64) & 0xFFFF


@pytest.mark.parametrize("knn", [1, 2, 7, 16, 31, 32])
def test_stream_random_scores(knn):
    g = gen(10 + knn)
    for L, n in ((256, 1024), (37, 2048), (64, 64)):
        check_rows(bf16_bits(torch.randn(L, n, generator=g)), knn)


def test_stream_uses_both_chunk_widths():
    g = gen(77)
    bits = bf16_bits(torch.randn(256, 1024, generator=g))
    stats = {}
    lists = stream_select(bits, 32, stats)
    assert stats.get("w16", 0) > 0 and stats.get("w32", 0) > 0, stats
    check_rows(bits, 32)
    assert np.array_equal(lists, stream_select(bits, 32))


def test_stream_tie_heavy_and_signed_zeros():
    g = gen(20)
    for knn in (1, 5, 32):
        # few distinct values: long equal runs everywhere
        check_rows(bf16_bits(torch.randint(-3, 4, (256, 512), generator=g).float()), knn)
        # ... and all negative: theta negative, where the threshold's rounding
        # interval runs the other way
        check_rows(bf16_bits(-torch.randint(1, 4, (256, 512), generator=g).float()), knn)
        # +0 and -0 mixed with a few positives and negatives
        x = torch.randint(-1, 2, (128, 256), generator=g).float() * 0.0
        x[torch.rand(128, 256, generator=g) < 0.5] = -0.0
        x[:, ::17] = torch.randn(128, 256 // 17 + 1, generator=g)
        check_rows(bf16_bits(x), knn)
        # all equal
        check_rows(bf16_bits(torch.full((64, 320), 0.25)), knn)


def test_stream_key_orders_that_fill_slots_fastest():
    # increasing scores: every key beats every earlier one, so every block
    # appends all of its scores; decreasing: only the blocks before the first
    # merge do
    n = 2048
    inc = torch.linspace(-4.0, 4.0, n)
    for row in (inc, inc.flip(0), -inc.abs(), inc * 0.0 + torch.arange(n) % 3):
        for knn in (1, 32):
            check_rows(bf16_bits(row.expand(256, n).contiguous()), knn)


def test_stream_slot_budget_worst_case():
    # Lanes that reach kTrigger - 1 unmerged slots at the start of a block
    # (too few for a merge) and then append a whole block: the most slots a
    # lane can hold. Scores are bf16 bits: 0x3F80 + 2 rank + lane half is an
    # increasing run of positive values over both lanes of a token, so a
    # passing position's score is above every earlier score of the token and
    # passes whatever theta is; 0xBF80 (-1.0) is below everything, so once a
    # merge has set theta it never passes (before the first merge every score
    # passes).
    per_blk = 2 * K_WPB  # scores of a block per lane
    first = -(-K_TRIGGER // per_blk)  # blocks of all-passing scores until the first merge
    assert first * per_blk >= K_TRIGGER
    fill = []  # passing counts of the following blocks up to kTrigger - 1 slots
    while sum(fill) < K_TRIGGER - 1:
        fill.append(min(per_blk, K_TRIGGER - 1 - sum(fill)))
    nblk = first + len(fill) + 4
    n, L = K_KB * nblk, 256
    rng = np.random.default_rng(40)
    for knn in (1, 32):
        bits = np.full((L, n), 0xBF80, dtype=np.int64)
        for t in range(L):
            rank = 0
            for b in range(nblk):
                if b < first or b >= first + len(fill):
                    cnt_b = per_blk if (b < first + len(fill) + 1 or t % 2 == 0) else 0
                else:
                    cnt_b = fill[b - first]
                pos = np.sort(rng.choice(per_blk, cnt_b, replace=False))
                for p_ in pos:
                    for h in (0, 1):
                        bits[t, b * K_KB + BLOCK_KEYS[h][p_]] = 0x3F80 + 2 * (rank + p_) + h
                rank += per_blk
        stats = {}
        lists = stream_select(bits, knn, stats)
        assert stats["max_cnt"] == K_TRIGGER - 1 + per_blk <= K_BUF, stats
        check_rows(bits, knn)
        assert lists.shape == (L, knn)


def test_stream_extremes():
    g = gen(30)
    x = torch.randn(256, 1024, generator=g) * 1e38
    x[:, ::5] = torch.randn(256, 205, generator=g) * 1e-38  # subnormal bf16s
    check_rows(bf16_bits(x), 32)
