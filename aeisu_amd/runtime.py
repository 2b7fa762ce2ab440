"""Python shim over the native MI355X runtime, mirroring aeisu/runtime.py.

``load_model(path, device, precision)`` loads any released weight file and
``upscale(model, source, tile)`` reproduces the reference's
``upscale(model, source, tile=128)`` (aeisu/runtime.py:70-103): CHW RGB in
[0, 1] -> 2x CHW float32 on the CPU, clipped, with the same align32/halo16
replicate padding, the same phase-aligned tiling with a 32-LR-pixel halo, and
the same errors (``ValueError`` for bad shapes or tiles,
``FloatingPointError`` for a non-finite reconstruction).  All arithmetic runs
in the HIP kernels of ``libaeisu_amd.so``; there is no CPU fallback.
"""
from __future__ import annotations

import ctypes
from pathlib import Path
from collections import OrderedDict
from typing import Dict, Optional, Tuple

import torch
from torch.nn import functional as F

from . import _lib as L
from .artifacts import load_blob

_DTYPES = {torch.float16: L.LAYOUT_F16, torch.float32: L.LAYOUT_F32}


def _stream_ptr(stream: Optional[torch.cuda.Stream]) -> int:
    s = stream if stream is not None else torch.cuda.current_stream()
    return s.cuda_stream


class _Handle:
    """One native runtime configured for one (batch, H, W, layouts, flags).

    The first handle of an Upscaler loads the artifact; every further one is a sibling
    (aeisu_create_sibling) that shares its uploaded weights and owns only its scratch.
    """

    def __init__(self, precision: str, blob: Optional[bytes] = None, sibling_of: Optional["_Handle"] = None):
        self.ptr = ctypes.c_void_p()
        self.precision = precision
        if sibling_of is not None:
            L.check(L.lib().aeisu_create_sibling(sibling_of.ptr, ctypes.byref(self.ptr)))
        else:
            buf = ctypes.create_string_buffer(blob, len(blob))
            L.check(L.lib().aeisu_create_from_memory(buf, len(blob), L.PRECISION[precision], ctypes.byref(self.ptr)))
        self.key = None

    def configure(self, key) -> None:
        if key != self.key:
            batch, h, w, lin, lout, flags = key
            L.check(L.lib().aeisu_configure(self.ptr, batch, h, w, lin, lout, L.PRECISION[self.precision], flags))
            self.key = key

    def report(self) -> str:
        n = L.lib().aeisu_startup_report(self.ptr, None, 0)
        buf = ctypes.create_string_buffer(max(int(n), 1))
        L.lib().aeisu_startup_report(self.ptr, buf, len(buf))
        return buf.value.decode()

    def close(self) -> None:
        if self.ptr:
            L.lib().aeisu_destroy(self.ptr)
            self.ptr = ctypes.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class Upscaler:
    """AEISU weights resident on one GPU, driven through the C ABI.

    The reference counterparts are ``FoldedAEISU`` (aeisu/model.py:554-596)
    for the Python path and ``aess::srcpyr::CudaRuntime``
    (SrcPyrCudaRuntime.h:29-96) for the native one.  The artifact is parsed and
    its weights uploaded once; each frame geometry gets a sibling runtime with
    its own scratch, and at most ``max_handles`` geometries are kept (least
    recently used first out), so tiled or mixed-size workloads do not grow
    device memory without bound.
    """

    def __init__(self, blob: bytes, precision: str, device: str = "cuda", max_handles: int = 8):
        if precision not in L.PRECISION:
            raise ValueError(f"precision must be one of {sorted(L.PRECISION)}")
        dev = torch.device(device)
        if dev.type != "cuda" or not torch.cuda.is_available():
            raise ValueError("the AEISU MI355X runtime needs a HIP device (device='cuda')")
        self.device = torch.device("cuda", dev.index if dev.index is not None else torch.cuda.current_device())
        self.precision = precision
        self.max_handles = max(1, max_handles)
        self._handles: "OrderedDict[Tuple, _Handle]" = OrderedDict()
        with torch.cuda.device(self.device):
            self._main = _Handle(precision, blob=blob)     # validates the artifact and uploads once

    # -- handles ---------------------------------------------------------------------------
    def handle(self, batch: int, h: int, w: int, in_dtype=torch.float16, out_dtype=torch.float16,
               flags: int = 0) -> _Handle:
        key = (batch, h, w, _DTYPES[in_dtype], _DTYPES[out_dtype], flags)
        hd = self._handles.get(key)
        if hd is not None:
            self._handles.move_to_end(key)
            return hd
        with torch.cuda.device(self.device):
            if len(self._handles) >= self.max_handles:
                _, old = self._handles.popitem(last=False)
                if old is not self._main:
                    old.close()
                else:
                    old.key = None
            hd = self._main if self._main.key is None else _Handle(self.precision, sibling_of=self._main)
            hd.configure(key)
        self._handles[key] = hd
        return hd

    def report(self, hd: Optional[_Handle] = None) -> str:
        """Startup report of a configured handle (default: the most recently configured one)."""
        if hd is None:
            hd = next(reversed(self._handles.values()))
        return hd.report()

    def _check_frames(self, frames: torch.Tensor) -> None:
        if frames.ndim != 4 or frames.shape[1] != 3:
            raise ValueError(f"Expected frames [B,3,H,W], got {tuple(frames.shape)}")
        if frames.device != self.device or frames.dtype not in _DTYPES or not frames.is_contiguous():
            raise ValueError("frames must be contiguous float16/float32 tensors on the runtime's device")

    # -- whole-frame entry points -----------------------------------------------------------
    def run(self, frames: torch.Tensor, out: Optional[torch.Tensor] = None, out_dtype=None, pad: bool = True,
            graph: bool = False, check_finite: bool = True, flags: int = 0,
            stream: Optional[torch.cuda.Stream] = None) -> torch.Tensor:
        """[B,3,H,W] -> [B,3,2H,2W] clipped to [0,1] (pad=False: input already on the padded grid)."""
        self._check_frames(frames)
        b, _, h, w = frames.shape
        out_dtype = out_dtype or (out.dtype if out is not None else frames.dtype)
        if not pad:
            flags |= L.FLAG_NO_PAD
        hd = self.handle(b, h, w, frames.dtype, out_dtype, flags)
        if out is None:
            out = torch.empty(b, 3, 2 * h, 2 * w, dtype=out_dtype, device=self.device)
        elif out.shape != (b, 3, 2 * h, 2 * w) or out.dtype != out_dtype or not out.is_contiguous():
            raise ValueError("output buffer has the wrong shape, dtype or layout")
        sp = _stream_ptr(stream)
        fn = L.lib().aeisu_upscale_graph if graph else L.lib().aeisu_upscale_async
        L.check(fn(hd.ptr, ctypes.c_void_p(frames.data_ptr()), ctypes.c_void_p(out.data_ptr()), ctypes.c_void_p(sp)))
        if check_finite:
            L.check(L.lib().aeisu_check_finite(hd.ptr, ctypes.c_void_p(sp)))
        return out

    def geometry(self, hd: _Handle) -> Tuple[int, ...]:
        g = (ctypes.c_int * 6)()
        L.check(L.lib().aeisu_geometry(hd.ptr, g))
        return tuple(g)

    def controller(self, frames: torch.Tensor, pad: bool = True, stream=None) -> torch.Tensor:
        """Packed FP16 coefficients [B, Hp/2, Wp/2, 64] (NHWC) of the controller alone."""
        self._check_frames(frames)
        b, _, h, w = frames.shape
        hd = self.handle(b, h, w, frames.dtype, torch.float16, 0 if pad else L.FLAG_NO_PAD)
        _, _, _, _, hq, wq = self.geometry(hd)
        meta = torch.empty(b, hq, wq, 64, dtype=torch.float16, device=self.device)
        L.check(L.lib().aeisu_controller_async(hd.ptr, ctypes.c_void_p(frames.data_ptr()),
                                               ctypes.c_void_p(meta.data_ptr()), ctypes.c_void_p(_stream_ptr(stream))))
        return meta

    def head(self, frames: torch.Tensor, meta: torch.Tensor, out_dtype=torch.float32, pad: bool = True,
             stream=None) -> torch.Tensor:
        """Reconstruction head alone on caller coefficients [B, Hp/2, Wp/2, 64] FP16."""
        self._check_frames(frames)
        b, _, h, w = frames.shape
        hd = self.handle(b, h, w, frames.dtype, out_dtype, 0 if pad else L.FLAG_NO_PAD)
        _, _, _, _, hq, wq = self.geometry(hd)
        if meta.shape != (b, hq, wq, 64) or meta.dtype != torch.float16 or not meta.is_contiguous() \
                or meta.device != self.device:
            raise ValueError("coefficients must be contiguous FP16 [B, Hp/2, Wp/2, 64] on the device")
        out = torch.empty(b, 3, 2 * h, 2 * w, dtype=out_dtype, device=self.device)
        L.check(L.lib().aeisu_head_async(hd.ptr, ctypes.c_void_p(frames.data_ptr()), ctypes.c_void_p(meta.data_ptr()),
                                         ctypes.c_void_p(out.data_ptr()), ctypes.c_void_p(_stream_ptr(stream))))
        return out

    def intermediate(self, hd: _Handle, which: int, stream=None) -> torch.Tensor:
        """Raw bytes of an intermediate activation of the last frame run on ``hd``."""
        n = L.lib().aeisu_intermediate_bytes(hd.ptr, which)
        buf = torch.empty(n, dtype=torch.uint8, device=self.device)
        L.check(L.lib().aeisu_copy_intermediate(hd.ptr, which, ctypes.c_void_p(buf.data_ptr()), n,
                                                ctypes.c_void_p(_stream_ptr(stream))))
        return buf

    def stage_timings(self, hd: _Handle, reset: bool = True) -> Tuple[Dict[str, float], int]:
        ms = (ctypes.c_float * 7)()
        frames = ctypes.c_int()
        L.check(L.lib().aeisu_stage_timings(hd.ptr, ms, ctypes.byref(frames)))
        if reset:
            L.check(L.lib().aeisu_reset_timings(hd.ptr))
        return dict(zip(L.STAGES, list(ms))), frames.value

    def persistent_bytes(self) -> int:
        """Uploaded weights (shared by every handle) plus every live handle's scratch: a handle reports
        weights + its scratch, an unconfigured sibling the weights alone."""
        probe = _Handle(self.precision, sibling_of=self._main)
        try:
            weights = int(L.lib().aeisu_persistent_bytes(probe.ptr))
        finally:
            probe.close()
        handles = {id(h): h for h in [self._main, *self._handles.values()] if h.ptr}.values()
        return weights + sum(int(L.lib().aeisu_persistent_bytes(h.ptr)) - weights for h in handles)

    def checksum(self) -> str:
        out = ctypes.create_string_buffer(65)
        L.check(L.lib().aeisu_artifact_checksum(self._main.ptr, out))
        return out.value.decode()

    def close(self) -> None:
        for h in list(self._handles.values()) + [self._main]:
            h.close()
        self._handles.clear()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def load_model(path, device: str = "cuda", precision: Optional[str] = None) -> Upscaler:
    """Load a released weight file (folded .pt, SPYR8F8 .bin or INT8 .pt) onto the GPU.

    Mirrors aeisu/runtime.py:45-56.  ``precision`` defaults to the file's
    natural policy; an FP8 artifact can also run at "fp16" (its FP16 weights), a folded FP32
    checkpoint also at "fp32" (FP32 activations and arithmetic: the reference's PyTorch path).
    """
    blob, natural = load_blob(Path(path))
    precision = precision or natural
    allowed = {"fp16": {"fp16", "fp32"}, "mixed": {"mixed", "mixed-fp8mma", "fp16"}, "int8": {"int8"}}[natural]
    if precision not in allowed:
        raise ValueError(f"{Path(path).name} provides {sorted(allowed)}, not {precision!r}")
    return Upscaler(blob, precision, device)


@torch.inference_mode()
def upscale(model: Upscaler, source: torch.Tensor, tile: int = 128) -> torch.Tensor:
    """aeisu/runtime.py:70-103 on the GPU runtime: CHW [0,1] -> clipped 2x CHW float32 (CPU)."""
    if source.ndim != 3 or source.shape[0] != 3:
        raise ValueError("Expected CHW RGB image")
    if tile < 0 or tile % 32:
        raise ValueError("tile must be zero or a positive multiple of 32")
    h, w = source.shape[-2:]
    image = source[None].to(model.device, torch.float32).contiguous()
    if tile == 0:
        return model.run(image, out_dtype=torch.float32)[0].cpu()
    ey, ex = -h % 32, -w % 32
    py, px = 16 + ey // 2, 16 + ex // 2
    padded = F.pad(image, (px, 32 + ex - px, py, 32 + ey - py), mode="replicate")
    ph, pw = padded.shape[-2:]
    result = torch.empty(1, 3, 2 * ph, 2 * pw, dtype=torch.float32, device=model.device)
    for y in range(0, ph, tile):
        for x in range(0, pw, tile):
            y1, x1 = min(y + tile, ph), min(x + tile, pw)
            sy, sx = max(0, y - 32), max(0, x - 32)
            ey_, ex_ = min(ph, y1 + 32), min(pw, x1 + 32)
            pred = model.run(padded[:, :, sy:ey_, sx:ex_].contiguous(), out_dtype=torch.float32, pad=False)
            result[:, :, 2 * y:2 * y1, 2 * x:2 * x1] = pred[:, :, 2 * (y - sy):2 * (y1 - sy), 2 * (x - sx):2 * (x1 - sx)]
    return result[0, :, 2 * py:2 * (py + h), 2 * px:2 * (px + w)].cpu()
