"""CPU oracle for the Sparse-Marlin 2:4 INT4 x FP16 GEMM path.

TEST INFRASTRUCTURE ONLY.  Nothing in ``csed499ii_amd`` imports this module;
only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` use it, and only as the checker.  It is written with numpy (no
torch), element-wise from the reference's semantics, so that it shares no code
with the product path it checks.

Reference files restated here (paths relative to the reference checkout):

* ``kernel_experiments/sparse_marlin/src/marlin/__init__.py`` (``MRL``)
* ``kernel_experiments/sparse_marlin/src/marlin/_semi_structured_conversions.py`` (``SEMI``)
* ``kernel_experiments/sparse_marlin/src/test_2_4.py`` (``TEST``)
* ``kernel_experiments/sparse_marlin/src/marlin/common/mma.h`` (``MMA``)
* ``kernel_experiments/sparse_marlin/src/marlin/marlin_cuda_kernel_nm.cu`` (``NM``)
* ``kernel_experiments/sparse_marlin/metadata_decode/codec.cu`` (``CODEC``)
* ``kernel_experiments/sparse_marlin/decoder_dependency/pair.cu`` (``PAIR``)
* ``kernel_experiments/3bit_encoding/experiment.cu`` (``EXP3``)
* ``kernel_experiments/sparse_marlin/src/marlin/__init__.py`` dense part (``MRL:61-239``)

How each function is pinned (checks live in ``tests/test_oracle.py``):

==========================  ==========================================================
function                    pinned by
==========================  ==========================================================
get_perms_2_4               kernel-view closed form ``word_coords`` (derived from the
                            kernel's fragment use, NM:389-410, MMA:57-96,130-150 and
                            the write-out order NM:573-617); bijection
word_coords                 agrees with get_perms_2_4 (two derivations)
META_TABLE / encode         the 16-row truth table written in SEMI:99-124 comments;
                            golden vectors from the reference converter
meta_offsets                golden vectors from the reference converter (CPU import,
                            tests/golden/make_golden.py); bijection
compress / decompress       golden vectors; round trip; brute force on tiny inputs
mask_2_4                    brute force over all 4! orderings; golden vectors
                            (tie-free inputs only: ties are "parity unpinned", the
                            reference's argsort is not stable, SEMI:309)
quantize                    closed form |q-8| <= 8, s = max|w|*2/maxq, exact
                            reconstruction of on-grid weights
pack / unpack / dequant     round trip unpack(pack(W)) == W on tie-free inputs;
                            word_coords; scale permutation closed form
gemm                        fp32 matmul of the dequantized weight (the benchmark
                            oracle itself); brute-force triple loop on tiny shapes
meta3_pack / meta3_unpack   encode tables CODEC:12-13 vs decode tables PAIR:11 are
                            mutual inverses on the 6 valid nibbles; bit-exact
                            round trip over every valid 2:4 pattern
expand3                     truth table {0..7}->{4,4,9,8,E,E,D,C} (EXP3:83);
                            exhaustive over all 2^24 packed 8-code inputs
pack_values3                round trip; bit positions 3*i (EXP3 layout)
native_pack / native_unpack this build's own layout (no reference counterpart):
                            exact round trip with the reference layout; the
                            native fields read by native_dequant (stated without
                            the reference layout) give dequant()'s weight
get_perms_dense             the dense layout's closed form ``dense_word_coords``
                            (two derivations agree; a planted swap of nibble rows
                            is caught); bijections
dense_word_coords           agrees with get_perms_dense; known answer: codes planted
                            at the eight positions of one word are read back
dense_pack / dense_unpack_* round trip unpack(pack(W)) == W's codes and scales,
dense_dequant               bit-exact, grouped and per-column
==========================  ==========================================================
"""
from __future__ import annotations

import numpy as np

# --------------------------------------------------------------------------
# Weight permutation (MRL:242-271) and its kernel-view closed form
# --------------------------------------------------------------------------


def get_perms_2_4():
    """Restatement of ``_get_perms_2_4`` (MRL:242-268).

    Returns ``(perm[1024], scale_perm[64], scale_perm_single[64])`` as int64 arrays.
    ``perm`` maps a destination slot of a 1024-entry block (8 nibbles per int32,
    128 int32 per block) to the source index in the (n//16 % 4, kc % 16, n % 16)
    tiled order built by ``pack`` (MRL:375-377).
    """
    perm = []
    for i in range(32):
        t = i % 4
        col = i // 4
        rows = (2 * t, 2 * t + 1, 2 * (t + 4), 2 * (t + 4) + 1)
        perm1 = [16 * row + (col // 2) * 256 + 8 * (col % 2) + 4 * block
                 for block in (0, 1) for row in rows]
        for j in range(4):
            perm.extend(p + j for p in perm1)
    perm = np.asarray(perm, dtype=np.int64).reshape(-1, 8)[:, [0, 2, 4, 6, 1, 3, 5, 7]].ravel()
    scale_perm = np.asarray([8 * i + j for i in range(8) for j in (0, 4, 1, 5, 2, 6, 3, 7)], dtype=np.int64)
    scale_perm_single = np.arange(64, dtype=np.int64)
    return perm, scale_perm, scale_perm_single


#: Compressed-K row (within a 16-row k-block) of nibble p of a packed word, as a
#: function of t = lane % 4.  Derived from the kernel: dequant (MMA:130-150)
#: splits a word into half2 pairs (p0,p4),(p1,p5) and, after ``>> 8``,
#: (p2,p6),(p3,p7); mma_sp (MMA:57-96) feeds them as A-fragment registers
#: {a0[0], a1[0], a0[1], a1[1]}, whose PTX m16n8k32 sparse-A columns are
#: 2t, 2t+1 (regs 0,1) and 2t+8, 2t+9 (regs 2,3).
def _row_of_nibble(t: np.ndarray | int, p: np.ndarray | int):
    t = np.asarray(t)
    off = np.array([0, 8, 0, 8, 1, 9, 1, 9], dtype=np.int64)[np.asarray(p)]
    return 2 * t + off


#: Output sub-block (0: column n, 1: column n+4) of nibble p; the A-fragment rows
#: g and g+8 of the MMA land 4 output columns apart after write-out (NM:573-617).
_BLK = np.array([0, 0, 1, 1, 0, 0, 1, 1], dtype=np.int64)


def word_coords(K: int, N: int):
    """Kernel-view closed form of the packed weight layout.

    For packed ``B`` of shape ``[K/32, 2N]`` int32 returns integer arrays
    ``kc, n`` of shape ``[K/32, 2N, 8]``: nibble ``p`` of ``B[r, w]`` holds the
    code of compressed-K row ``kc`` (0..K/2) and output column ``n``.
    With ``w = 128*beta + 4*i + j``, ``g = i // 4``, ``t = i % 4``:
    ``kc = 16 r + ROW_t[p]``, ``n = 64 beta + 8 g + 4 BLK[p] + j``.
    """
    R = K // 32
    r = np.arange(R)[:, None, None]
    w = np.arange(2 * N)[None, :, None]
    p = np.arange(8)[None, None, :]
    beta, wl = w // 128, w % 128
    i, j = wl // 4, wl % 4
    g, t = i // 4, i % 4
    kc = 16 * r + _row_of_nibble(t, p)
    n = 64 * beta + 8 * g + 4 * _BLK[p] + j
    kc = np.broadcast_to(kc, (R, 2 * N, 8))
    n = np.broadcast_to(n, (R, 2 * N, 8))
    return kc, n


# --------------------------------------------------------------------------
# 2:4 metadata encoding (SEMI:54-179, 186-283)
# --------------------------------------------------------------------------

#: Nonzero-flag quadruple -> 4-bit metadata, from the table written out in the
#: comments SEMI:99-124 (flags listed as positions 0..3).
META_TABLE = {
    (1, 1, 0, 0): 0b0100, (1, 0, 1, 0): 0b1000, (0, 1, 1, 0): 0b1001,
    (1, 0, 0, 1): 0b1100, (0, 1, 0, 1): 0b1101, (0, 0, 1, 1): 0b1110,
    (0, 0, 0, 0): 0b1110, (0, 0, 0, 1): 0b1110, (0, 0, 1, 0): 0b1110,
    (0, 1, 0, 0): 0b1001, (0, 1, 1, 1): 0b1101, (1, 0, 0, 0): 0b1000,
    (1, 0, 1, 1): 0b1100, (1, 1, 0, 1): 0b0100, (1, 1, 1, 0): 0b0100,
    (1, 1, 1, 1): 0b0100,
}

_META_LUT = np.zeros(16, dtype=np.int64)
for _flags, _code in META_TABLE.items():
    _META_LUT[_flags[0] | _flags[1] << 1 | _flags[2] << 2 | _flags[3] << 3] = _code


def meta_offsets(rows: int, meta_ncols: int) -> np.ndarray:
    """Scatter offsets of ``_calculate_meta_reordering_scatter_offsets`` (SEMI:21-48)
    for int16 metadata, restated element-wise: returns ``off[rows, ncols]`` such that
    logical ``meta[n, c]`` is stored at flat position ``off[n, c]``."""
    n = np.arange(rows)[:, None]
    c = np.arange(meta_ncols)[None, :]
    # row swizzle inside groups of 64 rows (group_y = 32 for int16 metadata)
    a = (n % 64) // 8
    b = (n % 8) // 4
    cb = (n % 4) // 2
    d = n % 2
    r2 = (n // 64) * 64 + 2 * d + b + 32 * cb + 4 * a
    r2 = np.broadcast_to(r2, (rows, meta_ncols))
    c2 = np.broadcast_to(c, (rows, meta_ncols))
    # swap the off-diagonal elements of every 2x2 block
    topright = (r2 % 2 == 0) & (c2 % 2 == 1)
    bottomleft = (r2 % 2 == 1) & (c2 % 2 == 0)
    shift = topright.astype(np.int64) - bottomleft.astype(np.int64)
    r3 = r2 + shift
    c3 = c2 - shift
    # ColumnMajorInterleaved<2>
    return (c3 // 2) * rows * 2 + r3 * 2 + c3 % 2


def compress(dense: np.ndarray, mask: np.ndarray | None = None):
    """Restatement of ``sparse_semi_structured_from_dense_cutlass`` (SEMI:54-179)
    for 16-bit element types.  ``dense`` is ``[rows, k]``; returns
    ``(sparse[rows, k/2], meta[rows, k/16] int16)``.  When ``mask`` is given the
    kept positions come from it instead of the ``!= 0`` test (SEMI:92)."""
    rows, k = dense.shape
    if rows % 32 or k % 16:
        raise ValueError("rows must be a multiple of 32 and k of 16")
    flags = (dense != 0) if mask is None else mask.astype(bool)
    f4 = flags.reshape(rows, k // 4, 4).astype(np.int64)
    code = _META_LUT[f4[..., 0] | f4[..., 1] << 1 | f4[..., 2] << 2 | f4[..., 3] << 3]
    idx0 = code & 3
    idx1 = (code >> 2) & 3
    d4 = dense.reshape(rows, k // 4, 4)
    s0 = np.take_along_axis(d4, idx0[..., None], axis=-1)[..., 0]
    s1 = np.take_along_axis(d4, idx1[..., None], axis=-1)[..., 0]
    sparse = np.stack([s0, s1], axis=-1).reshape(rows, k // 2)
    q = code.reshape(rows, k // 16, 4)
    meta = (q[..., 0] | q[..., 1] << 4 | q[..., 2] << 8 | q[..., 3] << 12).astype(np.uint16)
    flat = np.zeros(rows * (k // 16), dtype=np.uint16)
    flat[meta_offsets(rows, k // 16).ravel()] = meta.ravel()
    return sparse, flat.view(np.int16).reshape(rows, k // 16)


def meta_logical(meta_phys: np.ndarray, rows: int, k: int) -> np.ndarray:
    """Undo the physical reorder: returns logical ``uint16 meta[rows, k/16]``."""
    flat = np.ascontiguousarray(meta_phys).view(np.uint16).ravel()
    return flat[meta_offsets(rows, k // 16)]


def decompress(sparse: np.ndarray, meta_phys: np.ndarray) -> np.ndarray:
    """Restatement of ``sparse_semi_structured_to_dense_cutlass`` (SEMI:186-283)."""
    rows, kh = sparse.shape
    k = 2 * kh
    meta = meta_logical(meta_phys, rows, k).astype(np.int64)
    nib = np.stack([(meta >> (4 * u)) & 15 for u in range(4)], axis=-1).reshape(rows, k // 4)
    idx = np.stack([nib & 3, (nib >> 2) & 3], axis=-1)  # [rows, k/4, 2]
    dense = np.zeros((rows, k // 4, 4), dtype=sparse.dtype)
    vals = sparse.reshape(rows, k // 4, 2)
    for slot in (0, 1):
        np.put_along_axis(dense, idx[..., slot:slot + 1], vals[..., slot:slot + 1], axis=-1)
    return dense.reshape(rows, k)


def mask_2_4(x: np.ndarray, axis: int = -1) -> np.ndarray:
    """Keep the two largest ``|x|`` of every 4 consecutive entries along ``axis``.

    Ties go to the LOWER index (the order used for the synthetic configs).  The
    reference ``mask_creator`` (SEMI:286-314) uses an unstable argsort, so its tie
    behaviour is not pinned; on tie-free input both agree.
    """
    x = np.moveaxis(np.asarray(x), axis, -1)
    shp = x.shape
    g = np.abs(x.astype(np.float64)).reshape(-1, 4)
    # rank: number of entries that beat entry i (larger, or equal with lower index)
    beat = np.zeros_like(g, dtype=np.int64)
    for i in range(4):
        for j in range(4):
            if i == j:
                continue
            beat[:, i] += (g[:, j] > g[:, i]) | ((g[:, j] == g[:, i]) & (j < i))
    keep = (beat < 2).reshape(shp)
    return np.moveaxis(keep, -1, axis)


# --------------------------------------------------------------------------
# Quantizer (TEST:22-37) and packing (MRL:331-388)
# --------------------------------------------------------------------------


def quantize(w: np.ndarray, groupsize: int, maxq: int = 15):
    """Symmetric grouped quantizer of ``gen_quant4_NT`` (TEST:22-37).

    ``w`` is the K x N fp16 weight.  Returns ``(q[K,N] int64 codes, s[K/g or 1, N] fp16,
    ref[K,N] fp16 = (q - zero) * s)`` with ``zero = (maxq + 1) // 2``.
    """
    w = np.asarray(w, dtype=np.float16)
    K, N = w.shape
    g = K if groupsize == -1 else groupsize
    wg = w.reshape(K // g, g, N)
    s = np.abs(wg).max(axis=1).astype(np.float16)  # [K/g, N]
    s = (s.astype(np.float32) * np.float32(2 / maxq)).astype(np.float16)
    ratio = (wg.astype(np.float32) / s[:, None, :].astype(np.float32)).astype(np.float16)
    zero = (maxq + 1) // 2
    with np.errstate(invalid="ignore"):
        q = np.round(ratio.astype(np.float64))
    q = np.nan_to_num(q, nan=-zero).astype(np.int64) + zero
    q = np.clip(q, 0, maxq)
    ref = ((q - zero).astype(np.float16).astype(np.float32) * s[:, None, :].astype(np.float32)).astype(np.float16)
    return q.reshape(K, N), s, ref.reshape(K, N)


def mask_creator_codes(q: np.ndarray) -> np.ndarray:
    """``mask_creator(w.T)`` as applied to the offset codes inside pack (MRL:367):
    keeps the two largest codes of each group of 4 along K.  ``q`` is K x N; the
    returned mask is K x N."""
    return mask_2_4(q, axis=0)


def pack(w: np.ndarray, s: np.ndarray, groupsize: int, mask: np.ndarray | None = None):
    """Restatement of ``Layer_2_4.pack(linear, scales, trans=True)`` (MRL:331-388).

    ``w`` is the K x N fp16 weight (the reference reads ``linear.weight`` as K x N,
    MRL:349), ``s`` the ``[K/g or 1, N]`` fp16 scales.  With ``mask=None`` the
    reference's own mask (two largest codes, MRL:367) and ``!= 0`` compression
    apply; an explicit K x N boolean ``mask`` selects the kept positions instead.
    Returns ``(B[K/32, 2N] int32, s_packed fp16, meta[N, K/16] int16)``.
    """
    w = np.asarray(w, dtype=np.float16)
    K, N = w.shape
    g = K if groupsize == -1 else groupsize
    sg = np.asarray(s, dtype=np.float16).reshape(K // g, N)
    ratio = (w.reshape(K // g, g, N).astype(np.float32) / sg[:, None, :].astype(np.float32)).astype(np.float16)
    q = np.clip(np.round(ratio.astype(np.float64)).astype(np.int64) + 8, 0, 15).reshape(K, N)
    perm, scale_perm, scale_perm_single = get_perms_2_4()
    sp = scale_perm if g != K else scale_perm_single
    s_packed = sg.reshape(-1, 64)[:, sp].reshape(K // g, N)
    if mask is None:
        keep = mask_creator_codes(q)
        sparse, meta = compress((q * keep).T)
    else:
        keep = np.asarray(mask, dtype=bool)
        sparse, meta = compress((q * keep).T, mask=keep.T)
    # sparse: [N, K/2] codes -> B words through the kernel-view coordinates
    kc, n = word_coords(K, N)
    codes = sparse.T[kc, n].astype(np.uint32)  # [K/32, 2N, 8]
    words = np.zeros(codes.shape[:2], dtype=np.uint32)
    for p in range(8):
        words |= codes[..., p] << np.uint32(4 * p)
    return words.view(np.int32), s_packed, meta


def unpack_codes(B: np.ndarray, meta: np.ndarray, K: int, N: int):
    """Exact inverse of the packed layout: returns ``(codes[K,N] int64, kept[K,N] bool)``;
    codes of pruned positions are 0 and ``kept`` is False there."""
    words = np.ascontiguousarray(B).view(np.uint32).reshape(K // 32, 2 * N)
    kc, n = word_coords(K, N)
    nib = (words[..., None] >> (4 * np.arange(8, dtype=np.uint32))) & 15
    sparse = np.zeros((N, K // 2), dtype=np.int64)
    sparse[n, kc] = nib
    ml = meta_logical(meta, N, K).astype(np.int64)
    nibm = np.stack([(ml >> (4 * u)) & 15 for u in range(4)], axis=-1).reshape(N, K // 4)
    idx = np.stack([nibm & 3, (nibm >> 2) & 3], axis=-1)
    codes = np.zeros((N, K // 4, 4), dtype=np.int64)
    kept = np.zeros((N, K // 4, 4), dtype=bool)
    vals = sparse.reshape(N, K // 4, 2)
    for slot in (0, 1):
        np.put_along_axis(codes, idx[..., slot:slot + 1], vals[..., slot:slot + 1], axis=-1)
        np.put_along_axis(kept, idx[..., slot:slot + 1], True, axis=-1)
    return codes.reshape(N, K).T.copy(), kept.reshape(N, K).T.copy()


def unpack_scales(s_packed: np.ndarray, K: int, N: int, groupsize: int) -> np.ndarray:
    """Invert the scale permutation: returns natural-order ``s[K/g or 1, N]``."""
    g = K if groupsize == -1 else groupsize
    _, scale_perm, scale_perm_single = get_perms_2_4()
    sp = scale_perm if g != K else scale_perm_single
    sp_inv = np.argsort(sp)
    return np.asarray(s_packed, dtype=np.float16).reshape(-1, 64)[:, sp_inv].reshape(K // g, N)


def dequant(B, meta, s_packed, K: int, N: int, groupsize: int, zero: int = 8, codes=None):
    """Dense fp16 weight ``W[K,N] = (code - zero) * s`` (fp16 product, MMA:130-158)
    with pruned positions zero.  ``codes`` may be supplied (3-bit value format)."""
    if codes is None:
        codes, kept = unpack_codes(B, meta, K, N)
    else:
        _, kept = unpack_codes(np.zeros((K // 32, 2 * N), np.int32), meta, K, N)
    g = K if groupsize == -1 else groupsize
    s = unpack_scales(s_packed, K, N, groupsize)
    srow = np.repeat(s, g, axis=0)  # [K, N]
    w = ((codes - zero).astype(np.float16).astype(np.float32) * srow.astype(np.float32)).astype(np.float16)
    return np.where(kept, w, np.float16(0))


def gemm(A: np.ndarray, W: np.ndarray) -> np.ndarray:
    """The benchmark oracle: ``A.float() @ W.float()`` in fp32."""
    return np.asarray(A, dtype=np.float32) @ np.asarray(W, dtype=np.float32)


# --------------------------------------------------------------------------
# 3-bit metadata codec (CODEC:7-29, PAIR:11)
# --------------------------------------------------------------------------

#: nibble -> 3-bit code, for words 0..31 ("high") and 32..63 ("low") of every
#: 64-word group (CODEC:12-13).
ENC_HIGH = {14: 0, 13: 1, 8: 2, 4: 5, 9: 6, 12: 7}
ENC_LOW = {12: 0, 13: 1, 14: 2, 8: 4, 9: 5, 4: 6}
#: 3-bit code -> nibble decode tables (PAIR:11).
DEC_HIGH = [14, 13, 8, 13, 3, 4, 9, 12]
DEC_LOW = [12, 13, 14, 10, 8, 9, 4, 0]


def _enc_word(x: np.ndarray, table: dict) -> tuple[np.ndarray, np.ndarray]:
    out = np.zeros(x.shape, dtype=np.uint64)
    bad = np.zeros(x.shape, dtype=bool)
    lut = np.full(16, 255, dtype=np.int64)
    for nib, code in table.items():
        lut[nib] = code
    for i in range(8):
        c = lut[(x >> np.uint32(4 * i)) & np.uint32(15)]
        bad |= c == 255
        out |= (np.where(c == 255, 0, c).astype(np.uint64)) << np.uint64(3 * i)
    return out, bad


def meta3_pack(meta: np.ndarray):
    """Pack 4-bit metadata (viewed as uint32 words, 64 per group) into 3-bit codes,
    48 words per group (CODEC:18-24).  Returns ``(packed uint32, n_invalid)``."""
    a = np.ascontiguousarray(meta).view(np.uint32).reshape(-1, 64)
    hi0, b0 = _enc_word(a[:, 0:16], ENC_HIGH)
    lo0, b1 = _enc_word(a[:, 32:48], ENC_LOW)
    hi1, b2 = _enc_word(a[:, 16:32], ENC_HIGH)
    lo1, b3 = _enc_word(a[:, 48:64], ENC_LOW)
    first = hi0 | (lo0 << np.uint64(24))
    second = hi1 | (lo1 << np.uint64(24))
    out = np.zeros((a.shape[0], 48), dtype=np.uint32)
    out[:, 0:16] = (first & np.uint64(0xFFFFFFFF)).astype(np.uint32)
    out[:, 16:32] = ((first >> np.uint64(32)) | ((second << np.uint64(16)) & np.uint64(0xFFFFFFFF))).astype(np.uint32)
    out[:, 32:48] = (second >> np.uint64(16)).astype(np.uint32)
    nbad = int(b0.sum() + b1.sum() + b2.sum() + b3.sum())
    return out.ravel(), nbad


def _dec_word(c24: np.ndarray, table: list) -> np.ndarray:
    lut = np.asarray(table, dtype=np.uint32)
    out = np.zeros(c24.shape, dtype=np.uint32)
    for i in range(8):
        out |= lut[(c24 >> np.uint64(3 * i)) & np.uint64(7)] << np.uint32(4 * i)
    return out


def meta3_unpack(packed: np.ndarray) -> np.ndarray:
    """Inverse of :func:`meta3_pack`: returns int16 metadata (flat)."""
    p = np.ascontiguousarray(packed).view(np.uint32).reshape(-1, 48).astype(np.uint64)
    first = p[:, 0:16] | ((p[:, 16:32] & np.uint64(0xFFFF)) << np.uint64(32))
    second = (p[:, 16:32] >> np.uint64(16)) | (p[:, 32:48] << np.uint64(16))
    m = np.uint64(0xFFFFFF)
    out = np.zeros((p.shape[0], 64), dtype=np.uint32)
    out[:, 0:16] = _dec_word(first & m, DEC_HIGH)
    out[:, 32:48] = _dec_word((first >> np.uint64(24)) & m, DEC_LOW)
    out[:, 16:32] = _dec_word(second & m, DEC_HIGH)
    out[:, 48:64] = _dec_word((second >> np.uint64(24)) & m, DEC_LOW)
    return out.ravel().view(np.int16)


# --------------------------------------------------------------------------
# 3-bit code stream (EXP3:12-17, 3bit_encoding/README.md:28-30)
# --------------------------------------------------------------------------

#: EXP3:83 truth table of ``dec(x) = 3 ^ (x | (7 + (x >> 1)))``.
EXPAND3_TABLE = [4, 4, 9, 8, 14, 14, 13, 12]


def expand3(stream: np.ndarray) -> np.ndarray:
    """Expand 3-bit codes (code i at bit 3*i, LSB first; 48 bytes per 128 codes)
    to 4-bit nibbles (nibble i at bit 4*i; 64 bytes per 128 codes)."""
    b = np.ascontiguousarray(stream).view(np.uint8).reshape(-1, 3).astype(np.uint32)
    x = b[:, 0] | (b[:, 1] << 8) | (b[:, 2] << 16)  # 8 codes per 24 bits
    return _dec_word(x.astype(np.uint64), EXPAND3_TABLE)


def pack_values3(codes: np.ndarray) -> np.ndarray:
    """Bit-pack 3-bit codes (0..7): code i at bit 3*i, LSB first (EXP3 layout).
    ``codes`` length must be a multiple of 8; returns uint8 bytes."""
    c = np.asarray(codes, dtype=np.uint32).reshape(-1, 8)
    x = np.zeros(c.shape[0], dtype=np.uint32)
    for i in range(8):
        x |= (c[:, i] & 7) << np.uint32(3 * i)
    out = np.stack([x & 255, (x >> 8) & 255, (x >> 16) & 255], axis=-1).astype(np.uint8)
    return out.ravel()


def unpack_values3(stream: np.ndarray, n: int) -> np.ndarray:
    """Inverse of :func:`pack_values3` for ``n`` codes."""
    b = np.ascontiguousarray(stream).view(np.uint8).reshape(-1, 3).astype(np.uint32)
    x = b[:, 0] | (b[:, 1] << 8) | (b[:, 2] << 16)
    return np.stack([(x >> np.uint32(3 * i)) & 7 for i in range(8)], axis=-1).ravel()[:n].astype(np.int64)


def pack_w3(w: np.ndarray, s: np.ndarray, groupsize: int, mask: np.ndarray):
    """3-bit-value variant of :func:`pack` (no reference implementation exists):
    codes ``q = clamp(round(w/s) + 4, 0, 7)`` in the same word order as the 4-bit
    layout, then re-packed as a 3-bit stream (code of nibble p of word w at bit
    3*(8*w + p)).  Returns ``(B3 uint8[K/32 * 2N * 3], s_packed, meta)``."""
    w = np.asarray(w, dtype=np.float16)
    K, N = w.shape
    g = K if groupsize == -1 else groupsize
    sg = np.asarray(s, dtype=np.float16).reshape(K // g, N)
    ratio = (w.reshape(K // g, g, N).astype(np.float32) / sg[:, None, :].astype(np.float32)).astype(np.float16)
    q = np.clip(np.round(ratio.astype(np.float64)).astype(np.int64) + 4, 0, 7).reshape(K, N)
    _, scale_perm, scale_perm_single = get_perms_2_4()
    sp = scale_perm if g != K else scale_perm_single
    s_packed = sg.reshape(-1, 64)[:, sp].reshape(K // g, N)
    keep = np.asarray(mask, dtype=bool)
    sparse, meta = compress((q * keep).T, mask=keep.T)
    kc, n = word_coords(K, N)
    codes = sparse.T[kc, n]  # [K/32, 2N, 8]
    return pack_values3(codes.ravel()), s_packed, meta


def unpack_codes_w3(B3: np.ndarray, K: int, N: int) -> np.ndarray:
    """Sparse codes of the 3-bit value stream scattered back to ``[N, K/2]``."""
    codes = unpack_values3(B3, (K // 32) * 2 * N * 8).reshape(K // 32, 2 * N, 8)
    kc, n = word_coords(K, N)
    sparse = np.zeros((N, K // 2), dtype=np.int64)
    sparse[n, kc] = codes
    return sparse


def dequant_w3(B3, meta, s_packed, K: int, N: int, groupsize: int):
    """Dense fp16 weight of the 3-bit value format: ``(code - 4) * s``."""
    sparse = unpack_codes_w3(B3, K, N)
    ml = meta_logical(meta, N, K).astype(np.int64)
    nibm = np.stack([(ml >> (4 * u)) & 15 for u in range(4)], axis=-1).reshape(N, K // 4)
    idx = np.stack([nibm & 3, (nibm >> 2) & 3], axis=-1)
    codes = np.full((N, K // 4, 4), 4, dtype=np.int64)
    vals = sparse.reshape(N, K // 4, 2)
    for slot in (0, 1):
        np.put_along_axis(codes, idx[..., slot:slot + 1], vals[..., slot:slot + 1], axis=-1)
    codes = codes.reshape(N, K).T
    return dequant(None, meta, s_packed, K, N, groupsize, zero=4, codes=codes)


# --------------------------------------------------------------------------
# Lane-native decode layout (this build's own repack; no reference counterpart)
# --------------------------------------------------------------------------

#: Nibble of a lane word holding sparse value e (0..7) of the lane: the order in
#: which the magic-number dequantization (masks 0x000f000f / 0x00f000f0 of the word
#: and of the word >> 8) produces the eight fp16 operand halves.
NATIVE_NIBBLE = np.array([0, 4, 1, 5, 2, 6, 3, 7], dtype=np.int64)


def _native_coords(K: int, N: int):
    """Index grids of the native layout, shape ``[N/16, K/256, 4 (h), 16 (rho), 4 (j)]``:
    lane ``16 h + rho`` of 16-column block ``c16`` and 256-deep quad ``q`` holds, in
    word ``j``, the 8 compressed values ``kc = 32 (4q + j) + 8h + e`` of column
    ``n = 16 c16 + rho`` (dense K ``64 (4q+j) + 16h`` .. +16) and, in index halfword
    ``j``, the logical metadata int16 ``meta[n, 4 (4q + j) + h]`` of those 4 groups."""
    c16 = np.arange(N // 16)[:, None, None, None, None]
    q = np.arange(K // 256)[None, :, None, None, None]
    h = np.arange(4)[None, None, :, None, None]
    rho = np.arange(16)[None, None, None, :, None]
    j = np.arange(4)[None, None, None, None, :]
    n = 16 * c16 + rho
    kp = 4 * q + j
    return n, kp, h


def native_pack(B, meta, s_packed, K: int, N: int, groupsize: int):
    """Reference layout -> lane-native layout.  Returns ``(Wn uint32 [N/16, K/256, 64, 4],
    Xn uint16 [N/16, K/256, 64, 4], Sn fp16)``; ``Sn`` is ``[N/16, K/256, 16, 2]`` (the
    scales of groups 2q, 2q+1 of column rho) for groupsize 128 and the natural-order
    ``[1, N]`` scales for groupsize -1."""
    if K % 256 or N % 64:
        raise ValueError("native layout needs K % 256 == 0 and N % 64 == 0")
    words = np.ascontiguousarray(B).view(np.uint32).reshape(K // 32, 2 * N)
    kc, n = word_coords(K, N)
    nib = (words[..., None] >> (4 * np.arange(8, dtype=np.uint32))) & 15
    sparse = np.zeros((N, K // 2), dtype=np.uint32)
    sparse[n, kc] = nib
    nn, kp, h = _native_coords(K, N)
    G, Q = N // 16, K // 256
    Wn = np.zeros((G, Q, 4, 16, 4), dtype=np.uint32)
    for e in range(8):
        Wn |= sparse[nn, 32 * kp + 8 * h + e] << np.uint32(4 * NATIVE_NIBBLE[e])
    ml = meta_logical(meta, N, K)
    Xn = np.broadcast_to(ml[nn, 4 * kp + h].astype(np.uint16), (G, Q, 4, 16, 4))
    Wn = Wn.reshape(G, Q, 64, 4)
    Xn = Xn.reshape(G, Q, 64, 4)
    s_nat = unpack_scales(s_packed, K, N, groupsize)
    if groupsize == -1:
        Sn = s_nat.copy()
    else:
        g2 = np.arange(Q)[:, None, None] * 2 + np.arange(2)[None, None, :]   # [Q, 1, 2]
        cols = (16 * np.arange(G)[:, None, None, None] + np.arange(16)[None, None, :, None])  # [G, 1, 16, 1]
        Sn = s_nat[g2[None, :, :, :], cols]                                   # [G, Q, 16, 2]
    return Wn, Xn, Sn


def native_unpack(Wn, Xn, Sn, K: int, N: int, groupsize: int):
    """Lane-native layout -> reference layout (inverse of :func:`native_pack`)."""
    G, Q = N // 16, K // 256
    Wn = np.asarray(Wn, dtype=np.uint32).reshape(G, Q, 4, 16, 4)
    Xn = np.asarray(Xn, dtype=np.uint16).reshape(G, Q, 4, 16, 4)
    nn, kp, h = _native_coords(K, N)
    shape = np.broadcast_shapes(nn.shape, kp.shape, h.shape)
    nn, kp, h = (np.broadcast_to(x, shape) for x in (nn, kp, h))
    sparse = np.zeros((N, K // 2), dtype=np.uint32)
    for e in range(8):
        sparse[nn, 32 * kp + 8 * h + e] = (Wn >> np.uint32(4 * NATIVE_NIBBLE[e])) & 15
    kc, n = word_coords(K, N)
    codes = sparse[n, kc]
    words = np.zeros(codes.shape[:2], dtype=np.uint32)
    for p in range(8):
        words |= codes[..., p] << np.uint32(4 * p)
    ml = np.zeros((N, K // 16), dtype=np.uint16)
    ml[nn, 4 * kp + h] = Xn
    flat = np.zeros(N * (K // 16), dtype=np.uint16)
    flat[meta_offsets(N, K // 16).ravel()] = ml.ravel()
    _, scale_perm, scale_perm_single = get_perms_2_4()
    if groupsize == -1:
        s_nat = np.asarray(Sn, dtype=np.float16).reshape(1, N)
        s_packed = s_nat.reshape(-1, 64)[:, scale_perm_single].reshape(1, N)
    else:
        s_nat = np.asarray(Sn, dtype=np.float16).reshape(G, Q, 16, 2).transpose(1, 3, 0, 2).reshape(K // 128, N)
        s_packed = s_nat.reshape(-1, 64)[:, scale_perm].reshape(K // 128, N)
    return words.view(np.int32), flat.view(np.int16).reshape(N, K // 16), s_packed


def native_dequant(Wn, Xn, Sn, K: int, N: int, groupsize: int) -> np.ndarray:
    """Dense fp16 ``W[K, N]`` read straight from the native layout (the meaning of
    its fields, stated without the reference layout): lane word ``j`` nibble
    ``NATIVE_NIBBLE[e]`` is the code of value ``e`` (group ``e // 2``, slot ``e % 2``)
    of the lane's 4 groups, whose positions are the 2-bit fields of the lane's index
    halfword ``j`` (nibble ``u`` = ``idx0 | idx1 << 2`` of group ``u``)."""
    G, Q = N // 16, K // 256
    Wn = np.asarray(Wn, dtype=np.uint32).reshape(G, Q, 4, 16, 4)
    Xn = np.asarray(Xn, dtype=np.uint16).reshape(G, Q, 4, 16, 4).astype(np.int64)
    W = np.zeros((N, K), dtype=np.float16)
    if groupsize == -1:
        s_nat = np.asarray(Sn, dtype=np.float16).reshape(1, N)
    else:
        s_nat = np.asarray(Sn, dtype=np.float16).reshape(G, Q, 16, 2).transpose(1, 3, 0, 2).reshape(K // 128, N)
    gs = K if groupsize == -1 else 128
    for c16 in range(G):
        for q in range(Q):
            for h in range(4):
                for rho in range(16):
                    n = 16 * c16 + rho
                    for j in range(4):
                        k0 = 64 * (4 * q + j) + 16 * h
                        word = int(Wn[c16, q, h, rho, j])
                        idx = int(Xn[c16, q, h, rho, j])
                        for e in range(8):
                            u, slot = e // 2, e % 2
                            pos = (idx >> (4 * u + 2 * slot)) & 3
                            code = (word >> (4 * int(NATIVE_NIBBLE[e]))) & 15
                            k = k0 + 4 * u + pos
                            sc = s_nat[k // gs, n]
                            W[n, k] = np.float16(np.float16(code - 8) * sc)
    return W.T.copy()


# --------------------------------------------------------------------------
# Dense Marlin layout (MRL:78-99 ``_get_perms``, MRL:177-226 ``Layer.pack``)
# --------------------------------------------------------------------------


def get_perms_dense():
    """Restatement of ``_get_perms`` (MRL:78-99), step by step: for each of the 32
    groups i of 32 entries, the 8 sources (output block b, row pair of i % 4) of
    column i // 4 in tile 0, repeated for the 4 tiles of a 1024-entry chunk; then the
    entries of every 8 reordered by [0, 2, 4, 6, 1, 3, 5, 7].  Returns
    ``(perm[1024], scale_perm[64], scale_perm_single[32])``; ``perm[d]`` is the source
    index ``256 * tile + 16 * k + n`` (k, n within the 16 x 16 tile) of destination
    nibble ``d`` (word ``d // 8``, nibble ``d % 8``) of the chunk."""
    perm = []
    for i in range(32):
        rows = (2 * (i % 4), 2 * (i % 4) + 1, 2 * (i % 4) + 8, 2 * (i % 4) + 9)
        first = [16 * row + i // 4 + 8 * blk for blk in (0, 1) for row in rows]
        for tile in range(4):
            perm.extend(x + 256 * tile for x in first)
    perm = np.asarray(perm, dtype=np.int64).reshape(-1, 8)[:, [0, 2, 4, 6, 1, 3, 5, 7]].ravel()
    scale_perm = np.asarray([i + 8 * j for i in range(8) for j in range(8)], dtype=np.int64)
    scale_perm_single = np.asarray([2 * i + j for i in range(4) for j in (0, 1, 8, 9, 16, 17, 24, 25)],
                                   dtype=np.int64)
    return perm, scale_perm, scale_perm_single


#: Row (within the 16-deep k-tile) and output block of nibble t of a dense word:
#: low nibbles of bytes 0/2 hold k = 2rq / 2rq+1 and the high nibbles 2rq+8 / 2rq+9
#: of column ci; bytes 1/3 the same of column ci + 8.
_DENSE_KOFF = np.array([0, 8, 0, 8, 1, 9, 1, 9], dtype=np.int64)
_DENSE_BLK = np.array([0, 0, 1, 1, 0, 0, 1, 1], dtype=np.int64)


def dense_word_coords(K: int, N: int):
    """Closed form of the dense layout: for ``B`` of shape ``[K/16, 2N]`` int32 returns
    ``k, n`` of shape ``[K/16, 2N, 8]``: nibble t of ``B[r, 128 c + w]`` holds the code
    of ``k = 16 r + 2 rq + KOFF[t]`` and ``n = 64 c + 16 jt + ci + 8 BLK[t]`` with
    ``jt = w % 4``, ``rq = (w // 4) % 4``, ``ci = w // 16``."""
    R = K // 16
    r = np.arange(R)[:, None, None]
    w = np.arange(2 * N)[None, :, None]
    t = np.arange(8)[None, None, :]
    c, wl = w // 128, w % 128
    jt, rq, ci = wl % 4, (wl // 4) % 4, wl // 16
    k = 16 * r + 2 * rq + _DENSE_KOFF[t]
    n = 64 * c + 16 * jt + ci + 8 * _DENSE_BLK[t]
    return np.broadcast_to(k, (R, 2 * N, 8)), np.broadcast_to(n, (R, 2 * N, 8))


def dense_pack(w: np.ndarray, s: np.ndarray, groupsize: int):
    """Restatement of the dense ``Layer.pack(linear, scales)`` (MRL:177-226, the default
    ``trans=False`` permutation): codes ``clamp(round(w / s) + 8, 0, 15)`` of the K x N
    weight (``linear.weight`` read as K x N, MRL:193), placed by ``get_perms_dense``
    over 16 x 16 tiles (MRL:213-219), 8 nibbles per int32 (MRL:220-223); scales
    permuted by ``scale_perm`` (grouped) or ``scale_perm_single``.  Returns
    ``(B[K/16, 2N] int32, s_packed)``."""
    w = np.asarray(w, dtype=np.float16)
    K, N = w.shape
    g = K if groupsize == -1 else groupsize
    sg = np.asarray(s, dtype=np.float16).reshape(K // g, N)
    ratio = (w.reshape(K // g, g, N).astype(np.float32) / sg[:, None, :].astype(np.float32)).astype(np.float16)
    q = np.clip(np.round(ratio.astype(np.float64)).astype(np.int64) + 8, 0, 15).reshape(K, N)
    perm, scale_perm, scale_perm_single = get_perms_dense()
    sp = scale_perm if g != K else scale_perm_single
    s_packed = sg.reshape(-1, sp.size)[:, sp].reshape(K // g, N)
    tiles = q.reshape(K // 16, 16, N // 16, 16).transpose(0, 2, 1, 3).reshape(K // 16, N * 16)
    res = tiles.reshape(-1, perm.size)[:, perm].reshape(K // 16, N * 16).astype(np.uint32)
    words = np.zeros((K // 16, 2 * N), dtype=np.uint32)
    for t in range(8):
        words |= res[:, t::8] << np.uint32(4 * t)
    return words.view(np.int32), s_packed


def dense_unpack_codes(B: np.ndarray, K: int, N: int) -> np.ndarray:
    """Inverse of the dense layout through the closed form: codes ``q[K, N]``."""
    words = np.ascontiguousarray(B).view(np.uint32).reshape(K // 16, 2 * N)
    k, n = dense_word_coords(K, N)
    nib = (words[..., None] >> (4 * np.arange(8, dtype=np.uint32))) & 15
    q = np.zeros((K, N), dtype=np.int64)
    q[k, n] = nib
    return q


def dense_unpack_scales(s_packed: np.ndarray, K: int, N: int, groupsize: int) -> np.ndarray:
    g = K if groupsize == -1 else groupsize
    _, scale_perm, scale_perm_single = get_perms_dense()
    sp = scale_perm if g != K else scale_perm_single
    return np.asarray(s_packed, dtype=np.float16).reshape(-1, sp.size)[:, np.argsort(sp)].reshape(K // g, N)


def dense_dequant(B, s_packed, K: int, N: int, groupsize: int) -> np.ndarray:
    """Dense fp16 weight ``W[K, N] = (q - 8) * s`` (fp16 product, as the kernel's
    dequant and scale, marlin_cuda_kernel.cu:334-349)."""
    q = dense_unpack_codes(B, K, N)
    g = K if groupsize == -1 else groupsize
    srow = np.repeat(dense_unpack_scales(s_packed, K, N, groupsize), g, axis=0)
    return ((q - 8).astype(np.float16).astype(np.float32) * srow.astype(np.float32)).astype(np.float16)
