"""The allocation-free BitLinear (spb_bitlinear_{f16,bf16}_noalloc: the
workspace of spb_bitlinear_* held in the library's static device scratch),
called through the C ABI: its output bits equal the workspace entry point's
and the oracle's on two calls in a row, the second on a smaller input, at
the largest vector the scratch holds, and sizes beyond it are refused on the
host."""
import ctypes

import numpy as np
import pytest
import torch

from oracle import oracle as O
from spbitnet_amd import weights as W

pytestmark = pytest.mark.gpu

HALF = {"f16": torch.float16, "bf16": torch.bfloat16}


def _u32(a):
    return torch.from_numpy(np.ascontiguousarray(a, np.uint32).view(np.int32)).cuda()


def _bits(t):
    return t.view(torch.int16).cpu().numpy().view(np.uint16)


def _case(lib, kind, rows, cols, seed):
    L = W.random_layer(rows, cols, W.seed_for("noalloc", rows, cols, seed))
    a = W.normal_f32(W.seed_for("noalloc-x", rows, cols, seed), cols)
    xt = torch.from_numpy(a).to(HALF[kind])
    x = xt.cuda()
    xf = xt.float().numpy()
    meta, values = _u32(L.meta), _u32(L.values)
    out_na = torch.zeros(rows, dtype=HALF[kind], device="cuda")
    out_ws = torch.zeros(rows, dtype=HALF[kind], device="cuda")
    ws = torch.zeros(lib.spb_bitlinear_workspace_size(cols), dtype=torch.uint8, device="cuda")
    stream = torch.cuda.current_stream().cuda_stream or None
    print(f"noalloc {kind} {rows}x{cols}", flush=True)
    rc = getattr(lib, f"spb_bitlinear_{kind}_noalloc")(
        meta.data_ptr(), values.data_ptr(), x.data_ptr(), out_na.data_ptr(),
        ctypes.c_float(L.gamma), rows, cols, L.meta_stride, L.values_stride, stream)
    assert rc == 0, lib.spb_last_error_string()
    rc = getattr(lib, f"spb_bitlinear_{kind}")(
        meta.data_ptr(), values.data_ptr(), x.data_ptr(), out_ws.data_ptr(),
        ctypes.c_float(L.gamma), rows, cols, L.meta_stride, L.values_stride, ws.data_ptr(),
        ws.numel(), stream)
    assert rc == 0, lib.spb_last_error_string()
    torch.cuda.synchronize()
    want, _ = O.fused_bitlinear(L.meta, L.values, xf, O.absmax(xf), L.gamma, rows, cols)
    want_bits = O.to_f16_bits(want) if kind == "f16" else O.to_bf16_bits(want)
    got = _bits(out_na)
    assert (got == _bits(out_ws)).all()
    assert (got == want_bits).all()


@pytest.mark.parametrize("kind", ["bf16", "f16"])
def test_noalloc_matches_workspace_entry_point(gpu, kind):
    from spbitnet_amd import _lib
    lib = _lib.load()
    _case(lib, kind, 2560, 6912, 1)   # the down projection
    _case(lib, kind, 640, 2560, 2)    # then a smaller input: the scratch keeps the last
    _case(lib, kind, 8, 32768, 3)     # the largest vector the scratch holds


def test_noalloc_rejects_oversize(gpu):
    from spbitnet_amd import _lib
    lib = _lib.load()
    fake = ctypes.c_void_p(0x10000)
    rc = lib.spb_bitlinear_bf16_noalloc(fake, fake, fake, fake, ctypes.c_float(1.0), 4, 32896,
                                        1028, 514, None)
    assert rc == 1
    assert b"32768" in lib.spb_last_error_string()
    # zero rows / columns are successful no-ops, as in the reference
    assert lib.spb_bitlinear_f16_noalloc(fake, fake, fake, fake, ctypes.c_float(1.0), 0, 256,
                                         8, 4, None) == 0
