"""CPU model of the record-stream GEMM kernel's addressing (moat_amd/csrc/gemm.hip,
``rec_slots`` / ``RecReads`` / X slice loads), checked against the record
format itself and against the buffer bounds, for every tile and round of the
benchmark shapes and of small edge shapes.

The model replays the kernel's integer arithmetic: which 16-byte chunk each
lane copies into the per-round LDS stage, and where each lane then reads the
payload and scale of its rows.  It checks that

* every copied chunk lies inside the record stream (and every X chunk inside X);
* for every row of a round and every group of a 256-column tile that is inside
  the matrix, the 16 payload bytes and the fp16 scale the compute lanes read
  from the stage are the bytes the format puts there (group g of row k at
  144*(g'/8) + 16 + 16*(g'%8) and 144*(g'/8) + 2*(g'%8), g' = k*M/32 + g);
* the X chunk each MFMA lane reads back is X[row j][8q .. 8q+7] of the round.
"""

import numpy as np
import pytest

SLOTS_PER_ROW = 11
ROW_BYTES = 176
WEIGHT_LOADS = 6


def rec_slots(lane, tile, m, groups):
    """Absolute source offsets (round 0) of a lane's weight slots: the tile's
    base 144*tile (scalar in the kernel) plus the lane's offset from the full
    or the 128-column set (``rec_slots``: ``full`` / ``half``)."""
    offs = []
    halves_per_row = m >> 7
    for i in range(WEIGHT_LOADS):
        slot = 64 * i + lane
        row = min(slot // SLOTS_PER_ROW, 31)
        c = slot % SLOTS_PER_ROW if slot < 32 * SLOTS_PER_ROW else SLOTS_PER_ROW - 1
        halves = row * halves_per_row
        head = (halves >> 1) * 144
        shifted = halves & 1
        pay = 16 * c + (64 if shifted else 0)
        last = (9 if shifted else 8) if groups == 8 else 4
        offs.append(144 * tile + head + (pay if 1 <= c <= last else 0))
    return offs


def reads(j, shift):
    g = j >> 1
    pay0 = 16 + 16 * g + 8 * (j & 1)
    sc0 = 2 * g
    if shift:
        pay1 = (32 if g >= 4 else 16) + 16 * g + 8 * (j & 1)
        sc1 = (8 if g < 4 else 72) + 2 * g
    else:
        pay1, sc1 = pay0, sc0
    return (pay0, pay1), (sc0, sc1)


def check_shape(K, M, n=32, tiles_to_check=None):
    assert M % 128 == 0 and K % 32 == 0
    S = K * M // 256
    total = 144 * S
    # record stream with a recognisable byte at every position
    stream = (np.arange(total, dtype=np.int64) * 2654435761 % 251).astype(np.uint8)
    tiles = (M + 255) // 256
    shift = (M % 256) != 0
    rounds = K // 32
    tile_list = range(tiles) if tiles_to_check is None else tiles_to_check
    for tile in tile_list:
        groups = min(8, (M - 256 * tile) >> 5)
        lane_offs = [rec_slots(l, tile, M, groups) for l in range(64)]
        for r in {0, rounds // 2, rounds - 1}:
            base = r * 18 * M
            stage = np.zeros(1024 * WEIGHT_LOADS, dtype=np.uint8)
            for lane in range(64):
                for i, off in enumerate(lane_offs[lane]):
                    a = base + off
                    assert 0 <= a and a + 16 <= total, (K, M, tile, r, lane, i, a)
                    stage[1024 * i + 16 * lane:1024 * i + 16 * lane + 16] = stream[a:a + 16]
            for j in range(16):
                (p0, p1), (s0, s1) = reads(j, shift)
                g = j >> 1
                if g >= groups:
                    continue
                for t in range(32):
                    k = 32 * r + t
                    gg = k * (M // 32) + 8 * tile + g
                    pay = 144 * (gg >> 3) + 16 + 16 * (gg & 7) + 8 * (j & 1)
                    sca = 144 * (gg >> 3) + 2 * (gg & 7)
                    po = p1 if (t & 1) else p0
                    so = s1 if (t & 1) else s0
                    got = stage[ROW_BYTES * t + po:ROW_BYTES * t + po + 8]
                    assert np.array_equal(got, stream[pay:pay + 8]), (K, M, tile, r, t, j)
                    got_s = stage[ROW_BYTES * t + so:ROW_BYTES * t + so + 2]
                    assert np.array_equal(got_s, stream[sca:sca + 2]), (K, M, tile, r, t, j, "scale")
    # X slices: lane l copies row min(16nt + l/4, n-1), chunk (l&3)^((l>>2)&3)^((l>>4)&3)
    xbytes = 2 * n * K
    for nt in range(2 if n > 16 else 1):
        pos = {}
        for lane in range(64):
            row = min(16 * nt + (lane >> 2), n - 1)
            chunk = (lane & 3) ^ ((lane >> 2) & 3) ^ ((lane >> 4) & 3)
            for r in (0, rounds - 1):
                a = 2 * (row * K + 8 * chunk) + 64 * r
                assert 0 <= a and a + 16 <= xbytes
            pos[16 * lane] = (row, chunk)
        for q in range(4):
            for j in range(16):
                rx = 64 * j + 16 * (q ^ (j & 3) ^ ((j >> 2) & 3))
                row, chunk = pos[rx]
                assert chunk == q and row == min(16 * nt + j, n - 1)


@pytest.mark.parametrize("K,M,n", [(2048, 5504, 32), (3072, 8192, 1), (2048, 2048, 8), (5632, 2048, 16),
                                   (2048, 5632, 16), (32, 128, 1), (64, 384, 17), (96, 640, 3), (32, 256, 32)])
def test_record_stream_addressing(K, M, n):
    check_shape(K, M, n)


def test_record_stream_addressing_large():
    K, M = 8192, 28672
    check_shape(K, M, 32, tiles_to_check=[0, 1, 55, 110, 111])


def streamk_plan(T, R, P):
    """Segments of the record-stream kernel's stream-K split (gemm.hip:
    streamk_range / streamk_owner / the segment loop / streamk_fixup_kernel)."""
    items = T * R
    base, rem = divmod(items, P)

    def rng(p):
        lo = p * base + min(p, rem)
        return lo, lo + base + (1 if p < rem else 0)

    def owner(i):
        big = rem * (base + 1)
        return i // (base + 1) if i < big else rem + (i - big) // base

    writes = {}  # tile -> list of (p, r0, r1, slot or None)
    for p in range(P):
        lo, hi = rng(p)
        seg = lo
        while seg < hi:
            tile = seg // R
            r0 = seg - tile * R
            seg_hi = min(hi, (tile + 1) * R)
            r1 = seg_hi - tile * R
            whole = r0 == 0 and r1 == R
            slot = None if whole else 2 * p + (0 if seg == lo else 1)
            writes.setdefault(tile, []).append((p, r0, r1, slot))
            seg = seg_hi
    return rng, owner, writes


@pytest.mark.parametrize("T,R,P", [(22, 64, 176), (22, 64, 512), (32, 96, 384), (112, 256, 512), (8, 64, 128),
                                   (22, 64, 22), (22, 64, 44), (1, 1, 1), (3, 5, 7), (5, 3, 15), (112, 256, 224),
                                   (6, 64, 174), (28, 256, 504), (11, 64, 44)])
def test_streamk_partition(T, R, P):
    """T counts tile groups (1, 2 or 4 tiles each): the partition, owners and
    partial slots are per group; a group's tiles share its slots by offset."""
    rng, owner, writes = streamk_plan(T, R, P)
    for p in range(P):
        lo, hi = rng(p)
        assert hi > lo  # every workgroup has work (P <= items)
        assert owner(lo) == p and owner(hi - 1) == p
    slots_used = set()
    for t in range(T):
        segs = sorted(writes[t])
        # the segments of a tile cover its rounds exactly once, in workgroup order
        assert [s[1] for s in segs][0] == 0 and segs[-1][2] == R
        for a, b in zip(segs, segs[1:]):
            assert a[2] == b[1] and a[0] < b[0]
        p0, p1 = owner(t * R), owner(t * R + R - 1)
        if p0 == p1:
            assert len(segs) == 1 and segs[0][3] is None  # written straight to Y
        else:
            assert [s[0] for s in segs] == list(range(p0, p1 + 1))
            for s in segs:
                lo_p = rng(s[0])[0]
                # the slot the fix-up kernel reads is the one the segment wrote
                assert s[3] == 2 * s[0] + (1 if lo_p < t * R else 0)
                assert s[3] not in slots_used
                slots_used.add(s[3])
