"""Writes the golden vectors in tests/golden/ from the reference's own tests.

Run in the build container, where the reference tree is present:

    python tests/golden/make_golden.py

Inputs come from oracle/_ref/libspb_ref.so (oracle/ref_bridge.cpp), which
re-runs the reference tests' input generation (std::mt19937 seeds 123 / 42 /
77 with the same distribution calls, tests/test_sparse_ternary.cu:184-402)
and packs/unpacks with the reference's own SparseTernaryTensor class.  The
expected GEMV outputs are the int32 product of the reference's unpacked
dense matrix with x, i.e. what cpu_sparse_gemv (:17-33) returns.

Outputs
  ref_vectors.npz  data arrays (small cases in full; the 2048x2048 case as
                   x, y and a SHA-256 of its packed words)
"""
from __future__ import annotations

import hashlib
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)

from oracle import oracle as O  # noqa: E402


def dense_gemv(dense: np.ndarray, x: np.ndarray) -> np.ndarray:
    return (dense.astype(np.int64) @ x.astype(np.int64)).astype(np.int32)


def sha(*arrays) -> str:
    h = hashlib.sha256()
    for a in arrays:
        h.update(np.ascontiguousarray(a).tobytes())
    return h.hexdigest()


def main() -> None:
    O.build()
    if not O.ref_available():
        raise SystemExit("oracle/_ref/libspb_ref.so is not built (reference tree absent?)")
    out = {}

    # UnpackMatchesCPU: 8x64, seed 123 (tests/test_sparse_ternary.cu:184-247)
    w, m, _ = O.ref_make_test_case(123, 8, 64, False)
    meta, values = O.ref_pack_from_dense(w, m)
    out.update(unpack8x64_w=w, unpack8x64_mask=m, unpack8x64_meta=meta, unpack8x64_values=values,
               unpack8x64_dense=O.ref_unpack(meta, values, 8, 64))

    # GemvCorrectness: 64x256, seed 42 (:252-324)
    w, m, x = O.ref_make_test_case(42, 64, 256, True)
    meta, values = O.ref_pack_from_dense(w, m)
    dense = O.ref_unpack(meta, values, 64, 256)
    out.update(gemv64x256_meta=meta, gemv64x256_values=values, gemv64x256_x=x,
               gemv64x256_y=dense_gemv(dense, x))

    # GemvLargeDimension: 2048x2048, seed 77 (:330-402)
    w, m, x = O.ref_make_test_case(77, 2048, 2048, True)
    meta, values = O.ref_pack_from_dense(w, m)
    dense = O.ref_unpack(meta, values, 2048, 2048)
    out.update(gemv2048_x=x, gemv2048_y=dense_gemv(dense, x),
               gemv2048_meta_values_sha256=np.frombuffer(
                   bytes.fromhex(sha(meta, values)), np.uint8),
               gemv2048_meta_row0=meta[0], gemv2048_values_row0=values[0])

    # PackFromDenseRoundtrip: 4x32, pattern {+1,-1,+1,-1}, keep positions 0 and 2 (:38-84)
    w = np.tile(np.array([1, -1, 1, -1], np.int8), (4, 8))
    m = np.tile(np.array([1, 0, 1, 0], np.uint8), (4, 8))
    meta, values = O.ref_pack_from_dense(w, m)
    out.update(roundtrip4x32_meta=meta, roundtrip4x32_values=values,
               roundtrip4x32_dense=O.ref_unpack(meta, values, 4, 32))

    # PackWithPruning: 2x8 latent floats (:90-142), via the reference's pack_with_pruning
    latent = np.array([[0.1, -0.9, 0.8, -0.2, -0.7, 0.3, -0.6, 0.05],
                       [0.95, -0.1, 0.02, -0.85, -0.4, 0.9, -0.8, 0.3]], np.float32)
    meta, values = O.ref_pack_with_pruning(latent)
    out.update(pruning2x8_latent=latent, pruning2x8_meta=meta, pruning2x8_values=values,
               pruning2x8_dense=O.ref_unpack(meta, values, 2, 8))

    path = os.path.join(HERE, "ref_vectors.npz")
    np.savez_compressed(path, **out)
    print(f"wrote {path} ({os.path.getsize(path)} bytes, {len(out)} arrays)")


if __name__ == "__main__":
    main()
