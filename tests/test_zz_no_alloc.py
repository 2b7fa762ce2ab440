"""aeisu_upscale_noalloc (static scratch, no allocation) against aeisu_upscale_async, through the C ABI.

Two calls in a row per policy, the second on a smaller frame, each compared bit for bit with the
configured entry point on the same input (the same kernels run on the same arithmetic; only the
scratch memory differs).  A frame whose scratch exceeds the static array is rejected.
"""
from __future__ import annotations

import ctypes
import sys

import pytest
import torch

from tests._util import WEIGHTS

pytestmark = pytest.mark.gpu


def say(msg: str) -> None:
    print(msg, flush=True)
    sys.stdout.flush()


def _runtime(path, precision):
    from aeisu_amd import _lib as L
    from aeisu_amd.artifacts import load_blob
    blob, _ = load_blob(path)
    h = ctypes.c_void_p()
    buf = ctypes.create_string_buffer(blob, len(blob))
    L.check(L.lib().aeisu_create_from_memory(buf, len(blob), L.PRECISION[precision], ctypes.byref(h)))
    return h


@pytest.mark.parametrize("artifact,precision", [("aeisu_area_mixed_fp8.bin", "mixed"),
                                                ("aeisu_int8_fp16.pt", "int8"),
                                                ("aeisu_area.pt", "fp16")])
def test_noalloc_equals_configured_entry_point(gpu, artifact, precision):
    from aeisu_amd import _lib as L
    from aeisu_amd import frames
    lib = L.lib()
    ref = _runtime(WEIGHTS / artifact, precision)     # configured path
    noa = _runtime(WEIGHTS / artifact, precision)     # never configured: only the weights were uploaded
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    try:
        for b, h, w in ((1, 1080, 1920), (2, 270, 480)):
            say(f"case: aeisu_upscale_noalloc {precision} {b}x3x{h}x{w}")
            x = torch.stack([frames.scene(h, w, 50 + i, shapes=6, texture=True) for i in range(b)]).half()
            x = x.cuda().contiguous()
            want = torch.empty(b, 3, 2 * h, 2 * w, dtype=torch.float16, device="cuda")
            got = torch.full_like(want, float("nan"))
            L.check(lib.aeisu_configure(ref, b, h, w, L.LAYOUT_F16, L.LAYOUT_F16, 0, 0))
            L.check(lib.aeisu_upscale(ref, ctypes.c_void_p(x.data_ptr()), ctypes.c_void_p(want.data_ptr()), stream))
            L.check(lib.aeisu_upscale_noalloc(noa, b, h, w, L.LAYOUT_F16, L.LAYOUT_F16, ctypes.c_void_p(x.data_ptr()),
                                              ctypes.c_void_p(got.data_ptr()), stream))
            torch.cuda.synchronize()
            diff = (got.float() - want.float()).abs().max().item()
            say(f"  max |noalloc - configured| = {diff}")
            assert torch.equal(got, want)
        # a frame that needs more scratch than the static array holds is refused before any launch
        big = 2 if precision != "fp16" else 1
        rc = lib.aeisu_upscale_noalloc(noa, big, 1440, 2560, L.LAYOUT_F16, L.LAYOUT_F16,
                                       ctypes.c_void_p(x.data_ptr()), ctypes.c_void_p(got.data_ptr()), stream)
        assert rc == L.AEISU_ERR_INVALID_ARGUMENT and b"scratch" in lib.aeisu_last_error()
    finally:
        lib.aeisu_destroy(ref)
        lib.aeisu_destroy(noa)
