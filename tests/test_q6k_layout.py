"""The Q6_K device layout without a GPU: the host re-layout is a bijection,
and the kernel's register-level decode of a tiled tile-block -- masks, shifts,
the biased-scale byte permute and one fp16 fused multiply-add per pair --
reproduces the oracle's (q - 32) * sc for every element, in the B-operand
order of v_mfma_f32_16x16x32_f16 that the decode pack's A fragments use
(element 64g + 32 (fs / 4) + 8 (fs % 4) + h for lane group g, MFMA fs,
half h)."""
import numpy as np
import pytest

from q4k_ref import TYPE_Q6_K, make_q6k

TILE_BLOCK = 3360


def test_relayout_roundtrip_and_permutation(q4k):
    rng = np.random.default_rng(11)
    n, k = 48, 768
    w = make_q6k(rng, n, k)
    tiled = q4k.relayout_host(w, n, k, TYPE_Q6_K)
    assert tiled.nbytes == w.nbytes
    back = q4k.unrelayout_host(tiled, n, k, TYPE_Q6_K)
    np.testing.assert_array_equal(back, w.reshape(-1))
    # Popcount is preserved except for the scale bias (one flipped bit per scale byte).
    ones = lambda a: int(np.unpackbits(np.ascontiguousarray(a, np.uint8).reshape(-1)).sum())  # noqa: E731
    nblk = n * (k // 256)
    flips = ones(w.reshape(nblk, 210)[:, 192:208] ^ 0x80) - ones(w.reshape(nblk, 210)[:, 192:208])
    assert ones(tiled) == ones(w) + flips


def _and_or(a, mask, bits):
    return (a & mask) | bits


def _fma_h2(o, mul, add):
    """v_pk_fma_f16 on two halves: fp16(o_h * mul_h + add_h), one rounding
    (the exact product-sum of fp16 inputs is representable in float64)."""
    h = np.array([o & 0xFFFF, o >> 16], np.uint16).view(np.float16).astype(np.float64)
    return (h * mul + add).astype(np.float16)


def decode_tile_block(tb):
    """[64 lanes, 8 MFMAs, 8 halves] B-operand values of one tile-block, as
    the kernel computes them (q6_triple and the scale constants)."""
    u32 = np.frombuffer(tb[:3072].tobytes(), np.uint32).reshape(3, 64, 4)
    scw = np.frombuffer(tb[3072:3328].tobytes(), np.uint32)
    out = np.zeros((64, 8, 8), np.float64)
    m6, m4, m2, magic = 0x03F003F0, 0x00F000F0, 0x03000300, 0x64006400
    for lane in range(64):
        wd = [int(u32[s, lane, j]) for s in range(3) for j in range(4)]
        sw = int(scw[lane])
        for tr in range(4):
            u = (sw >> (8 * tr)) & 0xFF
            p = np.float16(np.uint16(0x6400 | u).view(np.float16))
            mul = np.float16(np.float64(p) * 0.0625 - 72.0)
            add = np.float16(np.float64(mul) * -1536.0)
            A, B, C = wd[3 * tr:3 * tr + 3]
            os_ = [_and_or(A, m6, magic), _and_or(A >> 6, m6, magic), _and_or(B, m6, magic), _and_or(B >> 6, m6, magic),
                   _and_or(C, m6, magic), _and_or(C >> 6, m6, magic),
                   _and_or((A << 4) & 0xFFFFFFFF, m4, _and_or((B << 8) & 0xFFFFFFFF, m2, magic)),
                   _and_or((C << 4) & 0xFFFFFFFF, m4, _and_or((B << 6) & 0xFFFFFFFF, m2, magic))]
            for r, o in enumerate(os_):
                fs, t = 2 * tr + r // 4, r % 4
                out[lane, fs, 2 * t:2 * t + 2] = _fma_h2(o, float(mul), float(add))
    return out


@pytest.mark.parametrize("seed", [12, 13])
def test_kernel_decode_matches_oracle(q4k, oracle, seed):
    rng = np.random.default_rng(seed)
    n, k = 16, 512
    w = make_q6k(rng, n, k)
    if seed == 13:  # extreme scales and quants: sc in {-128, 127}, q in {0, 63}
        blk = w.reshape(n, 2, 210)
        blk[:, :, 192:208] = rng.choice(np.array([0x80, 0x7F], np.uint8), size=(n, 2, 16))
        blk[:, :, :192] = rng.choice(np.array([0x00, 0xFF], np.uint8), size=(n, 2, 192))
    tiled = q4k.relayout_host(w, n, k, TYPE_Q6_K)
    for b in range(k // 256):
        got = decode_tile_block(tiled[b * TILE_BLOCK:(b + 1) * TILE_BLOCK])
        d = np.frombuffer(tiled[b * TILE_BLOCK + 3328:(b + 1) * TILE_BLOCK].tobytes(), np.float16)
        for lane in range(64):
            g, i = lane >> 4, lane & 15
            q, sc = oracle.q6_fields(w[i, b * 210:(b + 1) * 210])
            for fs in range(8):
                for h in range(8):
                    e = 64 * g + 32 * (fs // 4) + 8 * (fs % 4) + h
                    exact = (q[e] - 32) * sc[e]
                    # fp16 holds |v| <= 2048 exactly; above that, the nearest even integer.
                    assert got[lane, fs, h] == float(np.float16(exact)), (lane, fs, h)
                    assert abs(got[lane, fs, h] - exact) <= (1 if abs(exact) > 2048 else 0)
        assert np.array_equal(d, w.reshape(n, 2, 210)[:, b, 208:210].copy().view(np.float16).reshape(-1))


def test_typed_validation_before_hip(q4k):
    buf = np.zeros(16 * 210, np.uint8)
    with pytest.raises(q4k.Q4KError) as e:
        q4k.Weight(buf, 16, 256, ggml_type=10)
    assert e.value.code == -2
    with pytest.raises(q4k.Q4KError) as e:
        q4k.Weight(buf[:-1], 16, 256, ggml_type=TYPE_Q6_K)
    assert e.value.code == -3
    assert q4k.q4k_nbytes(16, 512, TYPE_Q6_K) == 16 * 2 * 210
    with pytest.raises(q4k.Q4KError):
        q4k.relayout_host(np.zeros(16 * 210, np.uint8), 16, 256, 10)
