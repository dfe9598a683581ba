"""Pins of the CPU oracle (oracle/sm24_oracle.py) against the reference's golden
vectors, truth tables, closed forms and brute force.  CPU only."""
import itertools

import numpy as np
import pytest

from oracle import sm24_oracle as o

GOLD = np.load(__import__("pathlib").Path(__file__).parent / "golden" / "semi_structured.npz")


# ---------------------------------------------------------------- permutations

def test_perm_is_bijection():
    perm, scale_perm, scale_perm_single = o.get_perms_2_4()
    assert sorted(perm.tolist()) == list(range(1024))
    assert sorted(scale_perm.tolist()) == list(range(64))
    assert scale_perm_single.tolist() == list(range(64))


def test_perm_matches_kernel_view_closed_form():
    """Two derivations of the weight layout: the pack() permutation (MRL:242-271) and
    the coordinates the kernel's fragments consume (NM:389-410, MMA:57-96, 130-150)."""
    perm, _, _ = o.get_perms_2_4()
    kc, n = o.word_coords(32, 64)  # one k-block row, one 64-column block
    x = perm.reshape(128, 8)
    assert np.array_equal((x // 256) * 16 + x % 16, n[0])
    assert np.array_equal((x % 256) // 16, kc[0])


@pytest.mark.parametrize("K,N", [(64, 64), (128, 256), (256, 512)])
def test_word_coords_bijection(K, N):
    kc, n = o.word_coords(K, N)
    flat = (kc * N + n).ravel()
    assert np.array_equal(np.sort(flat), np.arange(K // 2 * N))


def test_scale_perm_closed_form():
    """Packed slot 8a+b holds column 8a + {0,4,1,5,2,6,3,7}[b] (MRL:262-264)."""
    _, sp, _ = o.get_perms_2_4()
    for a in range(8):
        for b in range(8):
            assert sp[8 * a + b] == 8 * a + [0, 4, 1, 5, 2, 6, 3, 7][b]


# ---------------------------------------------------------------- metadata

def test_meta_table_two_flag_rows_are_positions():
    """For exactly two nonzeros the nibble must name their positions (idx0 < idx1)."""
    for flags, code in o.META_TABLE.items():
        idx0, idx1 = code & 3, code >> 2
        assert idx0 < idx1
        if sum(flags) == 2:
            assert [i for i in range(4) if flags[i]] == [idx0, idx1]
    assert len(o.META_TABLE) == 16


@pytest.mark.parametrize("tag", ["a", "b", "c", "d"])
def test_compress_matches_reference_vectors(tag):
    dense = GOLD[f"conv_{tag}_dense"]
    sparse, meta = o.compress(dense)
    assert np.array_equal(sparse, GOLD[f"conv_{tag}_sparse"])
    assert np.array_equal(meta, GOLD[f"conv_{tag}_meta"])
    assert np.array_equal(o.decompress(GOLD[f"conv_{tag}_sparse"], GOLD[f"conv_{tag}_meta"]), GOLD[f"conv_{tag}_back"])


def test_compress_half_matches_reference_vectors():
    sparse, meta = o.compress(GOLD["conv_h_dense"])
    assert np.array_equal(sparse, GOLD["conv_h_sparse"])
    assert np.array_equal(meta, GOLD["conv_h_meta"])


@pytest.mark.parametrize("key", [k for k in GOLD.files if k.startswith("offsets_")])
def test_meta_offsets_match_reference_vectors(key):
    rows, cols = map(int, key[len("offsets_"):].split("x"))
    off = o.meta_offsets(rows, cols)
    assert np.array_equal(off.ravel(), GOLD[key])
    assert np.array_equal(np.sort(off.ravel()), np.arange(rows * cols))


def test_decompress_inverts_compress_on_2_4_input():
    rng = np.random.default_rng(3)
    dense = rng.integers(1, 16, size=(128, 64)).astype(np.int32)
    keep = o.mask_2_4(rng.standard_normal((128, 64)), axis=-1)
    dense = dense * keep
    sparse, meta = o.compress(dense)
    assert np.array_equal(o.decompress(sparse, meta), dense)


# ---------------------------------------------------------------- mask

def test_mask_brute_force_with_ties():
    vals = [0.0, 1.0, -1.0, 2.0]
    for quad in itertools.product(vals, repeat=4):
        x = np.array(quad)
        keep = o.mask_2_4(x[None, :], axis=-1)[0]
        assert keep.sum() == 2
        a = np.abs(x)
        assert a[keep].min() >= a[~keep].max()
        # ties keep the lower index: among equal magnitudes a kept index precedes a dropped one
        for i in np.where(keep)[0]:
            for j in np.where(~keep)[0]:
                if a[i] == a[j]:
                    assert i < j


def test_mask_matches_reference_on_tie_free_vectors():
    assert np.array_equal(o.mask_2_4(GOLD["mask_x"], axis=-1), GOLD["mask_ref"].astype(bool))


# ---------------------------------------------------------------- quantizer / pack

def test_quantizer_closed_form():
    rng = np.random.default_rng(5)
    w = (rng.standard_normal((256, 64)) * 0.02).astype(np.float16)
    q, s, ref = o.quantize(w, 128)
    assert q.min() >= 0 and q.max() <= 15
    smax = np.abs(w.reshape(2, 128, 64)).max(axis=1)
    assert np.array_equal(s, (smax.astype(np.float32) * np.float32(2 / 15)).astype(np.float16))
    # reconstruction error at most half a quantization step (plus fp16 rounding)
    err = np.abs(ref.astype(np.float64) - w.astype(np.float64)).reshape(2, 128, 64)
    # (s is rounded to fp16, so max|w| / s may exceed 7.5 by ~2^-10 relative; the +7.5 side clamps)
    assert (err <= s[:, None, :].astype(np.float64) * 0.51 + 1e-7).all()


def test_quantizer_group_extremes():
    """+max|w| is 7.5 steps: rounds to 8 and clamps to code 15 (value 7s); -max|w|
    rounds half-to-even to -8, code 0 (value -8s)."""
    rng = np.random.default_rng(6)
    w = (rng.standard_normal((128, 2)) * 0.01).astype(np.float16)
    w[3, 0] = np.float16(0.05)
    w[7, 1] = np.float16(-0.05)
    q, s, ref = o.quantize(w, 128)
    assert q[3, 0] == 15 and q[7, 1] == 0
    assert ref[3, 0] == np.float16(np.float32(7) * np.float32(s[0, 0]))
    assert ref[7, 1] == np.float16(np.float32(-8) * np.float32(s[0, 1]))


@pytest.mark.parametrize("K,N,g", [(128, 64, 128), (256, 128, -1), (512, 256, 128)])
def test_pack_unpack_round_trip(K, N, g):
    rng = np.random.default_rng(K + N)
    w = (rng.standard_normal((K, N)) * 0.02).astype(np.float16)
    mask = o.mask_2_4(w, axis=0)
    w = np.where(mask, w, np.float16(0))
    q, s, ref = o.quantize(w, g)
    B, sp, meta = o.pack(w, s, g, mask=mask)
    codes, kept = o.unpack_codes(B, meta, K, N)
    assert np.array_equal(kept, mask)
    assert np.array_equal(np.where(mask, codes, 0), np.where(mask, q, 0))
    assert np.array_equal(o.unpack_scales(sp, K, N, g), s)
    W = o.dequant(B, meta, sp, K, N, g)
    assert np.array_equal(W, np.where(mask, ref, np.float16(0)))


def test_pack_reference_rule_keeps_largest_codes():
    rng = np.random.default_rng(9)
    w = (rng.standard_normal((128, 64)) * 0.02).astype(np.float16)
    q, s, ref = o.quantize(w, 128)
    B, sp, meta = o.pack(ref, s, 128)
    codes, kept = o.unpack_codes(B, meta, 128, 64)
    assert np.array_equal(kept, o.mask_2_4(q, axis=0) & (q != 0) | (kept & (q == 0)))
    assert (kept.reshape(32, 4, 64).sum(axis=1) == 2).all()


def test_planted_layout_mistake_is_caught(monkeypatch):
    """A transposed sub-block (BLK swapped) must break the round trip pin."""
    rng = np.random.default_rng(11)
    w = (rng.standard_normal((128, 64)) * 0.02).astype(np.float16)
    mask = o.mask_2_4(w, axis=0)
    w = np.where(mask, w, np.float16(0))
    q, s, ref = o.quantize(w, 128)
    B, sp, meta = o.pack(w, s, 128, mask=mask)
    monkeypatch.setattr(o, "_BLK", np.array([1, 1, 0, 0, 1, 1, 0, 0]))
    W = o.dequant(B, meta, sp, 128, 64, 128)
    assert not np.array_equal(W, np.where(mask, ref, np.float16(0)))


def test_gemm_brute_force():
    rng = np.random.default_rng(12)
    A = rng.standard_normal((3, 8)).astype(np.float16)
    W = rng.standard_normal((8, 5)).astype(np.float16)
    C = o.gemm(A, W)
    for i in range(3):
        for j in range(5):
            ref = sum(np.float64(A[i, k]) * np.float64(W[k, j]) for k in range(8))
            assert abs(C[i, j] - ref) < 1e-5


# ---------------------------------------------------------------- 3-bit codecs

def test_meta3_tables_are_inverse():
    valid = [4, 8, 9, 12, 13, 14]
    for enc, dec in ((o.ENC_HIGH, o.DEC_HIGH), (o.ENC_LOW, o.DEC_LOW)):
        assert sorted(enc) == valid
        assert sorted(enc.values()) == sorted(set(enc.values()))
        for nib, code in enc.items():
            assert dec[code] == nib


def _random_valid_meta(n_int16, seed):
    rng = np.random.default_rng(seed)
    valid = np.array([4, 8, 9, 12, 13, 14], dtype=np.uint16)
    nib = valid[rng.integers(0, 6, size=(n_int16, 4))]
    return (nib[:, 0] | nib[:, 1] << 4 | nib[:, 2] << 8 | nib[:, 3] << 12).astype(np.uint16).view(np.int16)


def test_meta3_round_trip_bit_exact():
    meta = _random_valid_meta(128 * 40, 1)
    packed, bad = o.meta3_pack(meta)
    assert bad == 0
    assert packed.size == meta.size * 3 // 8
    assert np.array_equal(o.meta3_unpack(packed), meta)


def test_meta3_counts_invalid_nibbles():
    meta = _random_valid_meta(128, 2).view(np.uint16).copy()
    meta[5] = (meta[5] & 0xFFF0) | 0x3   # nibble 3 is not a 2:4 pattern
    meta[70] = (meta[70] & 0x0FFF) | 0xF000
    _, bad = o.meta3_pack(meta.view(np.int16))
    assert bad == 2


def test_meta3_layout_positions():
    """first/second 48-bit fields land where CODEC:21-23 puts them."""
    meta = np.full(128, 0x4444, dtype=np.uint16).view(np.int16)  # every nibble = 4
    words = meta.view(np.uint32).copy()
    words[0] = 0xEEEEEEEE  # a[0] -> code 0 in the high table
    packed, _ = o.meta3_pack(words.view(np.int16))
    # a[p] (p<16) high-encoded in bits 0..23 of out[p]; nibble 4 -> code 5 everywhere else
    assert packed[0] & 0xFFFFFF == 0
    c5 = sum(5 << (3 * i) for i in range(8))
    assert packed[1] & 0xFFFFFF == c5
    c6 = sum(6 << (3 * i) for i in range(8))  # nibble 4 -> code 6 in the low table (a[32..63])
    assert (packed[0] >> 24) | ((packed[16] & 0xFFFF) << 8) == c6


def test_expand3_truth_table():
    assert o.EXPAND3_TABLE == [4, 4, 9, 8, 14, 14, 13, 12]
    for x in range(8):
        assert 3 ^ (x | (7 + (x >> 1))) == o.EXPAND3_TABLE[x]


def test_expand3_exhaustive_against_closed_form():
    """All 2^24 packed 8-code inputs: table decode == nibble-parallel closed form."""
    x = np.arange(1 << 24, dtype=np.uint32)
    stream = np.stack([x & 255, (x >> 8) & 255, (x >> 16) & 255], axis=-1).astype(np.uint8).ravel()
    got = o.expand3(stream)
    s = ((x & 0x00FFF000) << 4) | (x & 0x00000FFF)
    s = ((s & 0x0FC00FC0) << 2) | (s & 0x003F003F)
    s = ((s & 0x38383838) << 1) | (s & 0x07070707)
    ref = (s | (((s >> 1) & 0x33333333) + 0x77777777)) ^ 0x33333333
    assert np.array_equal(got, ref.astype(np.uint32))


def test_values3_bit_positions_and_round_trip():
    for i in range(16):
        codes = np.zeros(16, dtype=np.int64)
        codes[i] = 5
        b = o.pack_values3(codes)
        bits = np.unpackbits(b, bitorder="little")
        assert list(np.nonzero(bits)[0]) == [3 * i, 3 * i + 2]
    rng = np.random.default_rng(4)
    codes = rng.integers(0, 8, size=1024)
    assert np.array_equal(o.unpack_values3(o.pack_values3(codes), 1024), codes)


# ---------------------------------------------------------------- native layout

def _packed(K, N, g, seed):
    rng = np.random.default_rng(seed)
    w = (rng.standard_normal((K, N)) * 0.02).astype(np.float16)
    mask = o.mask_2_4(w.T).T
    gg = K if g == -1 else g
    s = (np.abs(w * mask).reshape(K // gg, gg, N).max(1) * 2 / 15).astype(np.float16)
    return o.pack(w, s, g, mask=mask)


@pytest.mark.parametrize("K,N,g", [(256, 64, 128), (512, 128, -1), (768, 192, 128)])
def test_native_round_trip_and_meaning(K, N, g):
    """The lane-native layout is a bijection of the reference layout's bytes, and its
    fields, read on their own terms (native_dequant), carry the same weight."""
    B, sp, meta = _packed(K, N, g, K + N)
    Wn, Xn, Sn = o.native_pack(B, meta, sp, K, N, g)
    assert Wn.shape == (N // 16, K // 256, 64, 4) and Xn.shape == Wn.shape
    B2, meta2, sp2 = o.native_unpack(Wn, Xn, Sn, K, N, g)
    assert np.array_equal(B, B2)
    assert np.array_equal(np.asarray(meta).view(np.uint16), np.asarray(meta2).view(np.uint16))
    assert np.array_equal(np.asarray(sp, np.float16).view(np.uint16), np.asarray(sp2, np.float16).view(np.uint16))
    W = o.dequant(B, meta, sp, K, N, g)
    assert np.array_equal(W.view(np.uint16), o.native_dequant(Wn, Xn, Sn, K, N, g).view(np.uint16))


def test_native_lane_word_positions():
    """A single nonzero code lands in the lane word, nibble and halfword the layout
    states: column n = 16 c16 + rho, compressed value kc = 32 (4q + j) + 8h + e at
    nibble NATIVE_NIBBLE[e] of word j of lane 16h + rho of quad q."""
    K, N = 512, 64
    sparse = np.zeros((N, K // 2), dtype=np.uint32)
    n, kc = 37, 32 * (4 * 1 + 3) + 8 * 2 + 5   # c16 2, rho 5; q 1, j 3, h 2, e 5
    sparse[n, kc] = 9
    kcs, ns = o.word_coords(K, N)
    codes = sparse[ns, kcs]
    words = np.zeros(codes.shape[:2], dtype=np.uint32)
    for p in range(8):
        words |= codes[..., p] << np.uint32(4 * p)
    meta = np.zeros((N, K // 16), dtype=np.int16)
    sp = np.ones((K // 128, N), dtype=np.float16)
    Wn, Xn, Sn = o.native_pack(words.view(np.int32), meta, sp, K, N, 128)
    nz = np.argwhere(Wn)
    assert nz.tolist() == [[2, 1, 16 * 2 + 5, 3]]
    assert Wn[2, 1, 37, 3] == 9 << (4 * int(o.NATIVE_NIBBLE[5]))
    assert o.NATIVE_NIBBLE.tolist() == [0, 4, 1, 5, 2, 6, 3, 7]


# ---- dense Marlin layout (MRL:78-99, 177-226) ----


def test_dense_perm_is_bijection_and_matches_closed_form():
    """Two derivations of the dense layout agree: the restated construction steps of
    ``_get_perms`` and the closed form ``dense_word_coords``."""
    perm, scale_perm, scale_perm_single = o.get_perms_dense()
    assert sorted(perm.tolist()) == list(range(1024))
    assert sorted(scale_perm.tolist()) == list(range(64))
    assert sorted(scale_perm_single.tolist()) == list(range(32))
    d = np.arange(1024)
    tile, kk, nn = perm // 256, (perm % 256) // 16, perm % 16
    k, n = o.dense_word_coords(16, 64)
    assert np.array_equal(k[0, d // 8, d % 8], kk)
    assert np.array_equal(n[0, d // 8, d % 8], 16 * tile + nn)


@pytest.mark.parametrize("K,N", [(16, 64), (64, 128), (256, 512)])
def test_dense_word_coords_bijection(K, N):
    k, n = o.dense_word_coords(K, N)
    flat = (k * N + n).ravel()
    assert np.array_equal(np.sort(flat), np.arange(K * N))


def test_dense_word_meaning_known_answer():
    """Word 16 ci + 4 rq + jt of row r: columns 16 jt + ci (byte 0, 2) and + 8 (bytes
    1, 3); low nibbles k = 2rq (bytes 0, 1) and 2rq + 1 (bytes 2, 3), high nibbles
    2rq + 8 and 2rq + 9 (the A-fragment rows of the reference's m16n8k16 MMA)."""
    K, N = 32, 128
    q = np.zeros((K, N), dtype=np.int64)
    # plant distinct codes at the eight positions of word (r=1, c=1, ci=5, rq=2, jt=3)
    r, c, ci, rq, jt = 1, 1, 5, 2, 3
    planted = {}
    for t, (dk, db) in enumerate(zip([0, 8, 0, 8, 1, 9, 1, 9], [0, 0, 1, 1, 0, 0, 1, 1])):
        kk, nn = 16 * r + 2 * rq + dk, 64 * c + 16 * jt + ci + 8 * db
        q[kk, nn] = t + 3
        planted[t] = t + 3
    s = np.ones((1, N), np.float16)
    W = ((q - 8) * 1.0).astype(np.float16)
    B, _ = o.dense_pack(W, s, -1)
    word = B.view(np.uint32).reshape(K // 16, 2 * N)[r, 128 * c + 16 * ci + 4 * rq + jt]
    for t, code in planted.items():
        assert (int(word) >> (4 * t)) & 15 == code
    assert np.array_equal(o.dense_unpack_codes(B, K, N), q)


@pytest.mark.parametrize("K,N,g", [(128, 256, 128), (256, 64, -1), (512, 512, 128)])
def test_dense_pack_round_trip(K, N, g):
    """unpack(pack(W)) gives W's codes and scales exactly for on-grid weights."""
    rng = np.random.default_rng(K + N)
    w = (rng.standard_normal((K, N)) * 0.02).astype(np.float16)
    q, s, ref = o.quantize(w, g)
    B, sp = o.dense_pack(ref, s, g)
    assert np.array_equal(o.dense_unpack_codes(B, K, N), q)
    assert np.array_equal(o.dense_unpack_scales(sp, K, N, g).view(np.int16), s.view(np.int16))
    assert np.array_equal(o.dense_dequant(B, sp, K, N, g).view(np.int16), ref.view(np.int16))


def test_dense_planted_layout_mistake_is_caught():
    """A swapped pair of nibble rows in the closed form breaks agreement with the
    restated permutation (the check above is not vacuous)."""
    perm, _, _ = o.get_perms_dense()
    bad = np.array([0, 8, 0, 8, 9, 1, 1, 9])
    w = np.arange(128)[:, None]
    t = np.arange(8)[None, :]
    k_bad = 2 * ((w // 4) % 4) + bad[t]
    d = np.arange(1024)
    assert not np.array_equal(k_bad[d // 8, d % 8], (perm % 256) // 16)
