"""CPU check of the value-backward row kernel's metadata window
(eb_bwd_rows64_kernel in modelos_amd/csrc/eb_bwd.hip).

A wave walks its 64 rows two rows ahead of the reduction: get_meta(i + 2)
may move the LDS window of occurrence metadata before row i is reduced, so
everything a row needs from the window (its bags and weights) is read inside
get_meta. Rows longer than the prefetch and at most kHeavyT long are reduced
after the main loop, each with the window moved to its start. This test
replays the kernel's order of window loads and reads for random row layouts
(empty, light, long and heavy rows, partial last waves) and checks every
index, including the padded reads of the metadata array. It also checks that
a read of a row's window entries at reduction time could fall outside the
window.
"""
import random

import pytest

META_CHUNK, HEAVY_T = 256, 256  # kMetaChunk, kHeavyT


def _replay(offs, K, U, r0, read_at_process=False):
    N = offs[-1]
    nmeta = N + META_CHUNK + 16  # padded metadata array
    nrows = min(64, K - r0)
    tail = offs[r0 + nrows]
    beg_l = [offs[r0 + l] if l < nrows else tail for l in range(64)]
    end_l = [offs[r0 + l + 1] if l < nrows else tail for l in range(64)]
    st = {"cbase": 0}

    def load_chunk(start):
        assert start + META_CHUNK <= nmeta
        st["cbase"] = start

    load_chunk(beg_l[0])

    deferred = []

    def get_meta(i):
        beg, end = (beg_l[i], end_l[i]) if i < 64 else (tail, tail)
        cnt = end - beg
        longrow = U < cnt <= HEAVY_T
        if longrow:
            deferred.append(i)
        nh = 0 if (cnt > HEAVY_T or longrow) else cnt
        if beg + U > st["cbase"] + META_CHUNK:
            load_chunk(beg)
        for lane in range(max(U, 1)):
            assert 0 <= beg - st["cbase"] + lane < META_CHUNK
        for lane in range(nh):
            assert beg <= st["cbase"] + (beg - st["cbase"] + lane) < end
        return beg, end, nh

    def process(m):
        beg, end, nh = m
        if read_at_process:
            for lane in range(nh):
                assert 0 <= beg - st["cbase"] + lane < META_CHUNK, "stale window"
        assert nh <= U

    ma, mb = get_meta(0), get_meta(1)
    for i in range(0, 64, 2):
        process(ma)
        ma = get_meta(i + 2)
        process(mb)
        mb = get_meta(i + 3)

    # deferred long rows, in row order: window at the row's start, U at a time
    assert deferred == sorted(set(deferred))
    for i in deferred:
        beg, end = beg_l[i], end_l[i]
        assert U < end - beg <= HEAVY_T
        load_chunk(beg)
        for s in range(beg, end, U):
            nh = min(end - s, U)
            for u in range(U):
                at = s - st["cbase"] + u
                idx = at if at < META_CHUNK else 0  # the kernel clamps the unused slots' reads
                assert 0 <= idx < META_CHUNK
                if u < nh:
                    assert at < META_CHUNK and beg <= st["cbase"] + at < end


def _layouts(seed, n):
    rnd = random.Random(seed)
    for _ in range(n):
        K = rnd.choice([1, 5, 63, 64, 65, 200, 700])
        pick = rnd.choice([[0, 0, 1, 2, 3, 9, 300], list(range(13)), [0, 4, 5, 8, 17, 255, 256, 257, 1000]])
        offs = [0]
        for _ in range(K):
            offs.append(offs[-1] + rnd.choice(pick))
        yield K, offs


def test_window_indices_in_range():
    for K, offs in _layouts(1, 600):
        for U in (1, 2, 4, 8):
            for r0 in range(0, K, 64):
                _replay(offs, K, U, r0)


def test_reading_at_reduction_would_leave_the_window():
    with pytest.raises(AssertionError, match="stale window"):
        for K, offs in _layouts(2, 600):
            for r0 in range(0, K, 64):
                _replay(offs, K, 8, r0, read_at_process=True)
