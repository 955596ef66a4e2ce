"""CPU model of the INT8 int8-P V kernel's LDS layout (fa_fwd_int8.hip, D = 64).

K and V tiles (64 rows of 64 int8 bytes) arrive in LDS by DMA: lane i of
DMA block j writes bytes [1024 j + 16 i, +16), and the kernel chooses each
lane's source so that LDS chunk position P holds row P / 4, logical chunk
(P % 4) ^ swz(row), swz(r) = (r >> 2) & 3.  The model replays that placement
and both operand reads element by element:

* the K (and Q) operand of v_mfma_i32_32x32x32_i8, a ds_read_b128 by lane l
  at row l % 32 (+ 32 kt), chunk 2 st + l / 32, must hold K[row][32 st + 16 g
  .. +15];
* the V^T operand, two ds_read_b64_tr_b8 per MFMA, must hold in byte s of
  lane l (column d = 32 dt + l % 32, reduction group g = l / 32) the value
  V[32 kt + 8 (s / 4) + 4 g + s % 4][d], the key order of the S^T
  accumulator that supplies P^T.  The transpose read is modelled as the probe
  on the GPU measured it: within a 16-lane group, lane i receives as byte k
  the byte i % 8 of the word that lane 2k + i / 8 addresses.

It also checks that the swizzle spreads each read pattern over distinct
banks (64 banks of 4 bytes).
"""
import numpy as np

D = 64
CH = D // 16


def swz(r):
    return (r >> 2) & 3


def lds_tile(rows):
    lds = np.full(64 * D, -999, dtype=np.int64)
    for j in range(64 * D // 1024):
        for lane in range(64):
            p = 64 * j + lane
            r, c = p // CH, (p % CH) ^ swz(p // CH)
            lds[1024 * j + 16 * lane:1024 * j + 16 * lane + 16] = rows[r, 16 * c:16 * c + 16]
    assert (lds != -999).all()
    return lds


def k_offset(lane, st, kt):
    l32, g = lane & 31, lane >> 5
    return l32 * D + 16 * ((2 * st + g) ^ swz(l32)) + kt * 32 * D


def v_offset(lane, dt, kt, r):
    g, k8 = lane >> 5, (lane & 15) >> 1
    kb = 8 * (k8 >> 2) + 4 * g + (k8 & 3)
    return kb * D + 16 * ((2 * dt + ((lane >> 4) & 1)) ^ swz(kb)) + 8 * (lane & 1) + kt * 32 * D + 16 * D * r


def test_k_operand_reads():
    rng = np.random.default_rng(1)
    k = rng.integers(-128, 128, size=(64, D))
    lds = lds_tile(k)
    for lane in range(64):
        l32, g = lane & 31, lane >> 5
        for st in range(D // 32):
            for kt in range(2):
                off = k_offset(lane, st, kt)
                assert (lds[off:off + 16] == k[32 * kt + l32, 32 * st + 16 * g:32 * st + 16 * g + 16]).all()


def test_vt_transpose_reads():
    rng = np.random.default_rng(2)
    v = rng.integers(-128, 128, size=(64, D))
    lds = lds_tile(v)
    for dt in range(D // 32):
        for kt in range(2):
            for r in range(2):
                addr = [v_offset(lane, dt, kt, r) for lane in range(64)]
                for lane in range(64):
                    base, i, g = lane & ~15, lane & 15, lane >> 5
                    for k in range(8):
                        got = lds[addr[base + 2 * k + i // 8] + i % 8]
                        s = 8 * r + k
                        key = 32 * kt + 8 * (s // 4) + 4 * g + s % 4
                        assert got == v[key, 32 * dt + (lane & 31)]


def _banks(byte_offsets, width):
    out = []
    for off in byte_offsets:
        out += [((off + 4 * w) // 4) % 64 for w in range(width // 4)]
    return out


def test_reads_use_distinct_banks():
    # ds_read_b128: 16 lanes (256 bytes) at a time
    for st in range(D // 32):
        for lo in (0, 16, 32, 48):
            banks = _banks([k_offset(lane, st, 0) for lane in range(lo, lo + 16)], 16)
            assert len(set(banks)) == 64, (st, lo)
    # ds_read_b64_tr_b8: 32 lanes (256 bytes) at a time
    for dt in range(D // 32):
        for r in range(2):
            for lo in (0, 32):
                banks = _banks([v_offset(lane, dt, 0, r) for lane in range(lo, lo + 32)], 8)
                assert len(set(banks)) == 64, (dt, r, lo)
