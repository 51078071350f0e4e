"""CPU replay of the value-backward row kernel's work schedule
(eb_bwd_rows_dyn_kernel, list_long_rows_kernel and launch_rows_dyn in
modelos_amd/csrc/eb_bwd.hip).

Rows are cut into blocks of `blk` rows; block k belongs to group k % 8, and
each group hands out chunks of 4 rows through 4 ticket counters (counter s
serves chunks s, s + 4, ... of every block of its group). A wave takes three
tickets up front and one per trip, and leaves when the chunk after the current
one is past its counter's end. This test replays that arithmetic for many
table sizes and checks that every row is reduced by exactly one chunk, that
every index the kernel forms (row offsets, metadata slots, lanes read by
readlane) is in bounds, that the workgroup count gives every counter a
workgroup, that interleaved waves on one counter reduce each chunk once and
drop none, and that the long-row listing covers every row once.
"""
import random

import pytest

RC, GROUPS, SUB, HEAVY_T, META_PAD = 4, 8, 4, 256, 16  # kDynRC, kDynGroups, kDynSub, kHeavyT, kMetaPad


def cdiv(a, b):
    return (a + b - 1) // b


def launch_params(K):
    blk = 1024 if K >= GROUPS * 8 * 1024 else RC * SUB
    wgs = min(cdiv(K, 64), 1280)
    wgs = cdiv(wgs, GROUPS * SUB) * GROUPS * SUB
    return blk, wgs


def counter_chunks(K, blk, grp, sub):
    """row0 of tickets 0.. of counter (grp, sub); the kernel's fetch_offs."""
    nblk = cdiv(K, blk)
    grp_blocks = cdiv(nblk - grp, GROUPS) if nblk > grp else 0
    cpb = blk // (RC * SUB)
    nchunks = grp_blocks * cpb
    return [(grp + GROUPS * (t // cpb)) * blk + ((t % cpb) * SUB + sub) * RC for t in range(nchunks)]


SIZES = [1, 3, 4, 15, 16, 17, 63, 64, 65, 100, 1000, 1023, 4096, 65535, 65536, 65537, 262144, 100003,
         (1 << 20) - 1, 1 << 20, (1 << 20) + 5, 3 * (1 << 20) + 777]


@pytest.mark.parametrize("K", SIZES)
def test_every_row_once(K):
    blk, wgs = launch_params(K)
    assert blk % (RC * SUB) == 0
    assert wgs % (GROUPS * SUB) == 0 and wgs >= GROUPS * SUB  # every (group, counter) has workgroups
    seen = bytearray(K)
    for grp in range(GROUPS):
        for sub in range(SUB):
            chunks = counter_chunks(K, blk, grp, sub)
            # row0 grows with the ticket, so a wave that meets a chunk starting
            # past the table (only in the last, partial block) has no rows after it
            assert chunks == sorted(chunks)
            for row0 in chunks:
                assert row0 < K or row0 // blk == (K - 1) // blk
                for i in range(RC):
                    r = row0 + i
                    if r < K:
                        assert seen[r] == 0
                        seen[r] = 1
    assert all(seen)


def _chunk_reads(offs, K, row0, U):
    """Indices the kernel reads for one chunk; returns the lanes get_meta reads."""
    N = offs[K]
    # fetch_offs: lane i -> offs[min(row0 + min(i, RC), K)]
    off = [offs[min(row0 + min(lane, RC), K)] for lane in range(64)]
    # fetch_meta: lane l reads meta[beg of row (l / U) & 3 + l % U]
    for lane in range(64):
        ri = (lane // U) & (RC - 1)
        assert 0 <= off[ri] + lane % U < N + META_PAD
    # get_meta: rows i < 4 read lanes i, i + 1 of off and i * U + u of the metadata
    for i in range(RC):
        assert i + 1 < 64 and i * U + U - 1 < 64
        beg, end = off[i], off[i + 1]
        assert beg <= end
        cnt = end - beg
        nh = cnt if cnt <= U else 0
        for u in range(nh):  # the slots a row reduces are its own occurrences, loaded by lane i * U + u
            lane = i * U + u
            assert (lane // U) & (RC - 1) == i and off[i] + lane % U == beg + u < end
    return off


@pytest.mark.parametrize("U", [8, 4, 2, 1])
@pytest.mark.parametrize("K", [5, 64, 1000, 70000])
def test_chunk_indices_in_bounds(K, U):
    rng = random.Random(K * 10 + U)
    counts = [rng.choice([0, 0, 1, 2, 3, 4, 5, 8, 9, 12, 300]) for _ in range(K)]
    offs = [0]
    for c in counts:
        offs.append(offs[-1] + c)
    blk, _ = launch_params(K)
    for grp in range(GROUPS):
        for sub in range(SUB):
            for row0 in counter_chunks(K, blk, grp, sub):
                _chunk_reads(offs, K, row0, U)
    # a ticket past the end gives row0 = K: every lane reads offs[K]
    _chunk_reads(offs, K, K, U)


def _run_waves(n_tickets, n_waves, rng):
    """Interleaves waves on one counter as the kernel's loop does; returns the
    tickets whose chunks were reduced."""
    counter = [0]

    def take():
        t = counter[0]
        counter[0] += 1
        return t

    done = []
    # each wave: a generator yielding at every atomic, reducing chunks in between
    def wave():
        t0 = take(); yield
        t1 = take(); yield
        tk = take(); yield
        if t0 >= n_tickets:
            return
        cur, nxt = t0, t1
        while True:
            nn = tk  # fetch_offs(tk, nn)
            tk = take(); yield
            done.append(cur)  # the chunk's 4 rows
            if not nxt < n_tickets:
                break
            cur, nxt = nxt, nn

    live = [wave() for _ in range(n_waves)]
    while live:
        w = rng.choice(live)
        try:
            next(w)
        except StopIteration:
            live.remove(w)
    return done


@pytest.mark.parametrize("n_tickets,n_waves", [(0, 4), (1, 4), (2, 1), (3, 1), (7, 3), (64, 40), (1000, 64), (5, 64)])
def test_interleaved_waves_reduce_each_chunk_once(n_tickets, n_waves):
    for seed in range(20):
        done = _run_waves(n_tickets, n_waves, random.Random(seed))
        assert sorted(done) == list(range(n_tickets))


@pytest.mark.parametrize("K", [1, 63, 1000, 1024, 5000, 262144, 1 << 20, (1 << 20) + 3])
def test_long_row_listing_covers_rows(K):
    # launch_rows_dyn: lwg workgroups of rows_per_wg rows (a multiple of 256)
    lwg = min(cdiv(K, 1024), 256)
    rows_per_wg = cdiv(cdiv(K, lwg), 256) * 256
    assert lwg * rows_per_wg >= K
    seen = bytearray(K)
    for w in range(lwg):
        r_beg = w * rows_per_wg
        r_end = min(r_beg + rows_per_wg, K)
        for wv in range(4):
            r0 = r_beg + wv * 64
            while r0 < r_end:  # the wave's rows r0 + lane, those < r_end counted
                for lane in range(64):
                    if r0 + lane < r_end:
                        assert seen[r0 + lane] == 0
                        seen[r0 + lane] = 1
                r0 += 256
    assert all(seen)
