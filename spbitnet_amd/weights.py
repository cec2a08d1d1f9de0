"""Host-side weight format: synthetic generation and packing of 2:4 sparse
ternary matrices in spbitnet's compressed layout.

Layout (include/spbitnet/sparse_ternary_tensor.h:12-39 and
docs/compression_format.md:120-225 of the reference):

* ``meta``   uint32 [rows][meta_stride], meta_stride = ceil(cols/32).  Group g
  (columns 4g..4g+3) stores a 4-bit position bitmap at bits 4*(g%8) of word
  g/8; bit i set <=> column 4g+i is non-zero.  Because of this, bit j of meta
  word w is simply "column 32w+j is kept".
* ``values`` uint32 [rows][values_stride], values_stride = ceil(cols/64).
  Group g stores 2 sign bits at bits 2*(g%16) of word g/16: bit 0 for the
  lower kept column, bit 1 for the higher one; 1 means -1.

Generation follows python/convert_model.py:257-316 (export_sparse_layer):
top-2 |W| per group of 4 with the higher index winning ties
(generate_24_mask, :88-119), gamma = mean|W| (quantize_ternary_absmean,
:122-138), kept value = sign(W) with W >= 0 -> +1 (the zero-at-mask fix,
:281-283).  Everything here is host-side numpy (the reference does the same
in Python); it runs once per weight matrix, never per token.
"""
from __future__ import annotations

from dataclasses import dataclass

import numpy as np

GROUP = 4
META_GROUPS_PER_WORD = 8
VALUES_GROUPS_PER_WORD = 16


def meta_words_per_row(cols: int) -> int:
    """sparse_ternary_tensor.h:254-257"""
    return (cols // GROUP + META_GROUPS_PER_WORD - 1) // META_GROUPS_PER_WORD


def values_words_per_row(cols: int) -> int:
    """sparse_ternary_tensor.h:261-264"""
    return (cols // GROUP + VALUES_GROUPS_PER_WORD - 1) // VALUES_GROUPS_PER_WORD


# --------------------------------------------------------------------------
# Deterministic synthetic data
# --------------------------------------------------------------------------

_GOLDEN = np.uint64(0x9E3779B97F4A7C15)
_M1 = np.uint64(0xBF58476D1CE4E5B9)
_M2 = np.uint64(0x94D049BB133111EB)


def _splitmix64(seed: int, start: int, n: int) -> np.ndarray:
    k = np.arange(start + 1, start + n + 1, dtype=np.uint64)
    with np.errstate(over="ignore"):
        z = np.uint64(seed & 0xFFFFFFFFFFFFFFFF) + k * _GOLDEN
        z = (z ^ (z >> np.uint64(30))) * _M1
        z = (z ^ (z >> np.uint64(27))) * _M2
    return z ^ (z >> np.uint64(31))


def normal_f32(seed: int, n: int, chunk: int = 1 << 22) -> np.ndarray:
    """N(0,1) float32 samples: SplitMix64 (Steele, Lea & Flood, 2014) feeding
    the Box-Muller transform, evaluated in float64 and rounded once."""
    out = np.empty(n, np.float32)
    npairs = (n + 1) // 2
    for p0 in range(0, npairs, chunk):
        p1 = min(npairs, p0 + chunk)
        raw = _splitmix64(seed, 2 * p0, 2 * (p1 - p0)).reshape(-1, 2)
        u1 = ((raw[:, 0] >> np.uint64(40)).astype(np.float64) + 1.0) / 16777216.0
        u2 = (raw[:, 1] >> np.uint64(40)).astype(np.float64) / 16777216.0
        r = np.sqrt(-2.0 * np.log(u1))
        t = 2.0 * np.pi * u2
        pair = np.empty((p1 - p0, 2), np.float64)
        pair[:, 0] = r * np.cos(t)
        pair[:, 1] = r * np.sin(t)
        flat = pair.reshape(-1).astype(np.float32)
        lo = 2 * p0
        hi = min(n, 2 * p1)
        out[lo:hi] = flat[: hi - lo]
    return out


def seed_for(*parts) -> int:
    """Stable 64-bit seed from a tuple of names / ints (FNV-1a over repr)."""
    h = 0xCBF29CE484222325
    for b in repr(parts).encode():
        h = ((h ^ b) * 0x100000001B3) & 0xFFFFFFFFFFFFFFFF
    return h


# --------------------------------------------------------------------------
# 2:4 mask, ternary sign, packing
# --------------------------------------------------------------------------

def top2_mask(w: np.ndarray) -> np.ndarray:
    """Keep the 2 largest |w| in every group of 4 along a row; on equal
    magnitudes the higher column index wins (convert_model.py:108-111 sorts
    ascending with a stable sort and keeps the last two)."""
    rows, cols = w.shape
    if cols % GROUP:
        raise ValueError(f"cols={cols} is not a multiple of 4")
    a = np.abs(w.astype(np.float32, copy=False)).reshape(rows, cols // GROUP, GROUP)
    idx = np.arange(GROUP)
    # beats[..., i, j]: position j outranks position i.
    aj = a[..., None, :]
    ai = a[..., :, None]
    beats = (aj > ai) | ((aj == ai) & (idx[None, :] > idx[:, None]))
    beaten_by = beats.sum(axis=-1)
    return (beaten_by < 2).reshape(rows, cols)


def absmean_gamma(w: np.ndarray) -> float:
    """gamma = mean(|W|) in float32 arithmetic (convert_model.py:132)."""
    return float(np.mean(np.abs(w.astype(np.float32, copy=False))))


def ternary_sparse(w: np.ndarray, mask: np.ndarray) -> np.ndarray:
    """Dense int8 {-1,0,+1} matrix the packed format represents: kept
    positions carry sign(w) (w >= 0 -> +1), the rest are 0."""
    return np.where(mask, np.where(w < 0, -1, 1), 0).astype(np.int8)


def pack(dense: np.ndarray, mask: np.ndarray):
    """Pack a ternary matrix with a 2:4 mask into (meta, values) uint32
    arrays.  Kept positions whose value is 0 are encoded as +1, as
    SparseTernaryTensor::pack_from_dense does (sparse_ternary_tensor.h:87-91)."""
    rows, cols = dense.shape
    if cols % GROUP:
        raise ValueError(f"cols={cols} is not a multiple of 4")
    ng = cols // GROUP
    m = mask.astype(bool).reshape(rows, ng, GROUP)
    if not np.all(m.sum(axis=-1) == 2):
        raise ValueError("every group of 4 must keep exactly 2 positions")
    neg = (dense.reshape(rows, ng, GROUP) < 0) & m
    bit = (1 << np.arange(GROUP)).astype(np.uint32)
    bitmap = (m.astype(np.uint32) * bit).sum(axis=-1, dtype=np.uint32)
    # first kept column = lowest set bit; second = the other one
    first = np.argmax(m, axis=-1)
    second = GROUP - 1 - np.argmax(m[..., ::-1], axis=-1)
    s_lo = np.take_along_axis(neg, first[..., None], axis=-1)[..., 0]
    s_hi = np.take_along_axis(neg, second[..., None], axis=-1)[..., 0]
    signs = s_lo.astype(np.uint32) | (s_hi.astype(np.uint32) << 1)

    ms = meta_words_per_row(cols)
    vs = values_words_per_row(cols)
    bm = np.zeros((rows, ms * META_GROUPS_PER_WORD), np.uint32)
    bm[:, :ng] = bitmap
    meta = np.bitwise_or.reduce(
        bm.reshape(rows, ms, META_GROUPS_PER_WORD)
        << (4 * np.arange(META_GROUPS_PER_WORD, dtype=np.uint32)), axis=-1)
    sg = np.zeros((rows, vs * VALUES_GROUPS_PER_WORD), np.uint32)
    sg[:, :ng] = signs
    values = np.bitwise_or.reduce(
        sg.reshape(rows, vs, VALUES_GROUPS_PER_WORD)
        << (2 * np.arange(VALUES_GROUPS_PER_WORD, dtype=np.uint32)), axis=-1)
    return np.ascontiguousarray(meta, np.uint32), np.ascontiguousarray(values, np.uint32)


def unpack(meta: np.ndarray, values: np.ndarray, rows: int, cols: int) -> np.ndarray:
    """Dense int8 view of a packed matrix (host-side, for inspection)."""
    ng = cols // GROUP
    g = np.arange(ng)
    bitmap = (meta[:, g // META_GROUPS_PER_WORD] >> (4 * (g % META_GROUPS_PER_WORD)).astype(np.uint32)) & 0xF
    signs = (values[:, g // VALUES_GROUPS_PER_WORD] >> (2 * (g % VALUES_GROUPS_PER_WORD)).astype(np.uint32)) & 0x3
    kept = ((bitmap[..., None] >> np.arange(GROUP, dtype=np.uint32)) & 1).astype(bool)
    rank = np.cumsum(kept, axis=-1) - 1  # 0 for the lower kept column, 1 for the higher
    sbit = (signs[..., None] >> np.clip(rank, 0, 1).astype(np.uint32)) & 1
    out = np.where(kept, np.where(sbit == 1, -1, 1), 0).astype(np.int8)
    return out.reshape(rows, cols)


@dataclass
class PackedLayer:
    """Host copy of one packed projection: the data behind a SparseLinear
    handle (include/spbitnet/model.h:46-60 of the reference)."""
    meta: np.ndarray
    values: np.ndarray
    gamma: float
    rows: int
    cols: int

    @property
    def meta_stride(self) -> int:
        return self.meta.shape[1]

    @property
    def values_stride(self) -> int:
        return self.values.shape[1]

    def nbytes(self) -> int:
        return self.meta.nbytes + self.values.nbytes


def make_layer_from_latent(w: np.ndarray) -> PackedLayer:
    """export_sparse_layer (convert_model.py:257-316) without the file I/O."""
    rows, cols = w.shape
    mask = top2_mask(w)
    dense = ternary_sparse(w, mask)
    meta, values = pack(dense, mask)
    return PackedLayer(meta, values, absmean_gamma(w), rows, cols)


def random_layer(rows: int, cols: int, seed: int) -> PackedLayer:
    """Config-0 recipe: latent W ~ N(0,1) float32, 2:4 top-2 mask, ternary
    signs, packed."""
    w = normal_f32(seed, rows * cols).reshape(rows, cols)
    return make_layer_from_latent(w)


def quantize_absmax_host(x: np.ndarray):
    """Per-token absmax int8 quantisation on the host, with the float32 order
    of operations of absmax_quantize_kernel (inference_kernels.cu:69-114):
    scale = 127/absmax in float32, q = clamp(rint(x*scale), -128, 127).
    Used to build synthetic int8 inputs; the GPU path has its own kernel."""
    x = np.asarray(x, np.float32)
    amax = np.float32(np.max(np.abs(x))) if x.size else np.float32(0)
    scale = np.float32(127.0) / amax if amax > 0 else np.float32(0)
    q = np.clip(np.rint(x * scale), -128, 127).astype(np.int8)
    return q, float(amax)
