"""CPU FP32 restatement of the AEISU inference path -- TEST INFRASTRUCTURE ONLY.

This module is the checker for the HIP runtime in ``aeisu_amd``.  Only
``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import it; the product never does.

Every function restates one piece of the reference algorithm and cites the
reference file:line it follows (paths relative to the reference checkout):

* analysis features           aeisu/model.py:273-341
* controller conv stack       aeisu/model.py:473-492 (layer table 20-27)
* LeakyReLU slope 0.1         aeisu/reparameterization.py:8
* basis projection            aeisu/reconstruction.py:8-12
* coefficient clamp           aeisu/reconstruction.py:15-17
* parity unpacking            aeisu/reconstruction.py:20-26
* polyphase reconstruction    aeisu/reconstruction.py:29-83 (trim=0 path)
* align32/halo16 pad + tiling aeisu/runtime.py:70-103
* checkpoint state lookup     aeisu/runtime.py:35-56

Pinning (what checks each function):
* ``coefficient_clamp``  -- known-answer table of tests/test_reference.py:31-34.
* ``unpack_coefficients`` -- closed-form parity index (tests/test_reference.py:36-45).
* ``project_basis``       -- zero-DC / L1<=0.5 invariants and the artifact's
  stored ``adaptive_basis`` (equal to project_basis(basis_raw) to ~2e-8).
* ``reconstruct``         -- zero coefficients + exact-bilinear base equals
  ``F.interpolate(bilinear, align_corners=False)``; flat-field invariant;
  brute-force per-pixel loop on tiny inputs.
* ``forward`` / ``upscale`` -- golden vectors written by
  tests/golden/make_golden.py from the reference's own FoldedAEISU.
"""
from __future__ import annotations

from typing import Dict, Mapping

import torch
from torch.nn import functional as F

LEAKY_SLOPE = 0.1

# (name, in, out, kernel) in execution order; aeisu/model.py:20-27.
CONV_LAYERS = (
    ("project_540", 32, 32, 1),
    ("compress_270", 128, 64, 1),
    *((f"bottleneck_270_{side}{i}", 32, 32, 3) for side in ("a", "b") for i in range(1, 5)),
    ("expand_270", 64, 128, 1),
    ("refine_540", 32, 64, 3),
    ("metadata_head", 64, 64, 1),
)
ANALYSIS_KEYS = ("analysis_rgb_basis", "analysis_rgb_mix", "analysis_dx_rows",
                 "analysis_dy_cols", "analysis_diag45", "analysis_diag135")


def exact_bilinear_base() -> torch.Tensor:
    """[25 taps, 4 phases] base of the untrained model (aeisu/model.py:171-199).

    Tap index is y*5+x with the centre at (2,2); phases TL, TR, BL, BR.  A 2x
    align_corners=False upsample samples +-1/4 pixel away from each source
    pixel, so the separable weights are (1/4, 3/4) and the products are 1/16,
    3/16 and 9/16.
    """
    base = torch.zeros(25, 4)
    for phase in range(4):
        oy, ox = phase >> 1, phase & 1
        # rows/cols touched: (1,2) for the top/left phase, (2,3) for bottom/right
        ys = (1, 2) if oy == 0 else (2, 3)
        xs = (1, 2) if ox == 0 else (2, 3)
        wy = (0.25, 0.75) if oy == 0 else (0.75, 0.25)
        wx = (0.25, 0.75) if ox == 0 else (0.75, 0.25)
        for y, a in zip(ys, wy):
            for x, b in zip(xs, wx):
                base[y * 5 + x, phase] = a * b
    return base


def leaky(x: torch.Tensor) -> torch.Tensor:
    return torch.where(x >= 0, x, x * LEAKY_SLOPE)


def _shift(img: torch.Tensor, dy: int, dx: int) -> torch.Tensor:
    """img[y+dy, x+dx] with replicate (clamp-to-edge) addressing."""
    h, w = img.shape[-2:]
    ys = torch.clamp(torch.arange(h) + dy, 0, h - 1)
    xs = torch.clamp(torch.arange(w) + dx, 0, w - 1)
    return img[..., ys, :][..., :, xs]


def rgb_to_feature8(src: torch.Tensor, p: Mapping[str, torch.Tensor]) -> torch.Tensor:
    """Eight analysis maps at LR resolution (aeisu/model.py:273-341).

    Channels: learned RGB (3x3 matrix), luma (3-term mix), then four
    directional responses of the replicate-padded luma.  Products and sums
    are written in the reference's evaluation order (no fused multiply-add).
    """
    r, g, b = src[:, 0:1], src[:, 1:2], src[:, 2:3]
    m = p["analysis_rgb_basis"]
    learned = [r * m[i, 0] + g * m[i, 1] + b * m[i, 2] for i in range(3)]
    mix = p["analysis_rgb_mix"]
    y = r * mix[0] + g * mix[1] + b * mix[2]
    n = {(dy, dx): _shift(y, dy, dx) for dy in (-1, 0, 1) for dx in (-1, 0, 1)}
    ul, uc, ur = n[(-1, -1)], n[(-1, 0)], n[(-1, 1)]
    cl, cr = n[(0, -1)], n[(0, 1)]
    dl, dc, dr = n[(1, -1)], n[(1, 0)], n[(1, 1)]
    horiz = cr - cl
    vert = dc - uc
    a = p["analysis_dx_rows"]
    dx = (ur - ul) * a[0] + horiz * a[1] + (dr - dl) * a[2]
    a = p["analysis_dy_cols"]
    dy = (dl - ul) * a[0] + vert * a[1] + (dr - ur) * a[2]
    a = p["analysis_diag45"]
    d45 = (dr - ul) * a[0] + vert * a[1] + horiz * a[2]
    a = p["analysis_diag135"]
    d135 = (ur - dl) * a[0] - vert * a[1] + horiz * a[2]
    return torch.cat((*learned, y, dx, dy, d45, d135), dim=1)


def conv(x: torch.Tensor, state: Mapping[str, torch.Tensor], name: str) -> torch.Tensor:
    weight = state[f"{name}.weight"]
    return F.conv2d(x, weight, state[f"{name}.bias"], padding=weight.shape[-1] // 2)


def controller(src: torch.Tensor, state: Mapping[str, torch.Tensor]) -> torch.Tensor:
    """Packed coefficient tensor [B,64,H/2,W/2] (aeisu/model.py:473-492)."""
    if src.ndim != 4 or src.shape[1] != 3:
        raise ValueError("Expected source RGB [B,3,H,W]")
    if src.shape[-2] % 4 or src.shape[-1] % 4:
        raise ValueError("Source H/W must be divisible by 4")
    feat = rgb_to_feature8(src, state)
    enc540 = leaky(conv(F.pixel_unshuffle(feat, 2), state, "project_540"))
    enc270 = leaky(conv(F.pixel_unshuffle(enc540, 2), state, "compress_270"))
    a, b = enc270[:, :32], enc270[:, 32:]
    for i in range(1, 5):
        a = leaky(conv(a, state, f"bottleneck_270_a{i}"))
        b = leaky(conv(b, state, f"bottleneck_270_b{i}"))
    up = F.pixel_shuffle(leaky(conv(torch.cat((a, b), 1), state, "expand_270")), 2)
    dec = leaky(conv(enc540 + up, state, "refine_540"))
    return conv(dec, state, "metadata_head")


def project_basis(raw: torch.Tensor, scale: float = 0.5) -> torch.Tensor:
    """[16,4,25] raw -> zero-mean, L1=scale, [25,16,4] (reconstruction.py:8-12)."""
    centred = raw - raw.mean(dim=-1, keepdim=True)
    l1 = centred.abs().sum(dim=-1, keepdim=True).clamp_min(1e-6)
    return (centred * (scale / l1)).permute(2, 0, 1).contiguous()


def coefficient_clamp(t: torch.Tensor) -> torch.Tensor:
    """Identity on |t|<=2, then slope 0.05 up to a 2.5 ceiling (reconstruction.py:15-17)."""
    mag = t.abs()
    soft = torch.clamp(2 + 0.05 * (mag - 2), max=2.5)
    return torch.where(mag <= 2, t, torch.sign(t) * soft)


def unpack_coefficients(meta: torch.Tensor, clamp=None) -> torch.Tensor:
    """[B,64,h,w] parity-major -> clamped [B,16,2h,2w] (reconstruction.py:20-26).

    Channel 16*rho + k of packed cell (i, j) is coefficient k of the LR pixel
    (2i + rho//2, 2j + rho%2).  ``clamp`` replaces ``coefficient_clamp`` (the
    quantized deployments' head rounds the clamped value to FP16, see
    ``oracle.deploy.coefficient_clamp_fp16``).
    """
    bsz, ch, h, w = meta.shape
    if ch != 64:
        raise ValueError("Expected 64 packed coefficient channels")
    out = meta.new_empty(bsz, 16, 2 * h, 2 * w)
    for rho in range(4):
        out[:, :, rho >> 1::2, rho & 1::2] = meta[:, 16 * rho:16 * rho + 16]
    return (clamp or coefficient_clamp)(out)


def reconstruct(src: torch.Tensor, meta: torch.Tensor, base: torch.Tensor,
                basis: torch.Tensor, clamp=None) -> torch.Tensor:
    """Unclipped 2x RGB (reconstruction.py:29-83 with trim=0).

    out[2y+oy, 2x+ox, c] = sum_t (base[t,ph] + sum_k a_k(y,x) basis[t,k,ph])
                            * src[c, clamp(y+ty-2), clamp(x+tx-2)],  ph = 2*oy+ox.
    """
    bsz, _, h, w = src.shape
    if meta.shape != (bsz, 64, h // 2, w // 2):
        raise ValueError("Source/metadata geometry mismatch")
    coeff = unpack_coefficients(meta, clamp)                # [B,16,H,W]
    out = src.new_zeros(bsz, 3, 2 * h, 2 * w)
    for ph in range(4):
        acc = src.new_zeros(bsz, 3, h, w)
        # filter weights per tap: [B,25,H,W]
        weights = base[:, ph].view(1, 25, 1, 1) + torch.einsum("bkhw,tk->bthw", coeff, basis[:, :, ph])
        for t in range(25):
            acc = acc + weights[:, t:t + 1] * _shift(src, t // 5 - 2, t % 5 - 2)
        out[:, :, ph >> 1::2, ph & 1::2] = acc
    return out


def state_tensors(payload) -> Dict[str, torch.Tensor]:
    """Tensor state dict inside a checkpoint payload (aeisu/runtime.py:35-42)."""
    if isinstance(payload, dict):
        for key in ("model", "model_state_dict", "state_dict"):
            if isinstance(payload.get(key), dict):
                return payload[key]
        if payload and all(torch.is_tensor(v) for v in payload.values()):
            return payload
    raise ValueError("Checkpoint does not contain a tensor state dictionary")


def load_folded(path) -> Dict[str, torch.Tensor]:
    """Folded FP32 state plus derived ``base`` and ``basis`` tensors."""
    payload = torch.load(path, map_location="cpu", weights_only=True)
    state = {k: v.float() for k, v in state_tensors(payload).items()}
    scale = float(payload.get("basis_l1_scale", 0.5)) if isinstance(payload, dict) else 0.5
    state["base"] = state["base_kernel"]
    state["basis"] = project_basis(state["basis_raw"], scale)
    return state


def forward(src: torch.Tensor, state: Mapping[str, torch.Tensor]) -> torch.Tensor:
    """FoldedAEISU.forward (aeisu/model.py:546-551): unclipped 2x RGB."""
    return reconstruct(src, controller(src, state), state["base"], state["basis"])


def pad_geometry(h: int, w: int):
    """(top, bottom, left, right) replicate pad of aeisu/runtime.py:82-84."""
    ey, ex = -h % 32, -w % 32
    py, px = 16 + ey // 2, 16 + ex // 2
    return py, 32 + ey - py, px, 32 + ex - px


@torch.inference_mode()
def upscale(state: Mapping[str, torch.Tensor], source: torch.Tensor, tile: int = 0,
            model=None) -> torch.Tensor:
    """aeisu/runtime.py:70-103: pad, (optionally tiled) forward, crop, finite check, clip.

    ``model`` overrides the whole-image forward (used to drive the mixed and
    INT8 emulations through the same geometry).
    """
    if source.ndim != 3 or source.shape[0] != 3:
        raise ValueError("Expected CHW RGB image")
    if tile < 0 or tile % 32:
        raise ValueError("tile must be zero or a positive multiple of 32")
    run = model if model is not None else (lambda x: forward(x, state))
    h, w = source.shape[-2:]
    top, bottom, left, right = pad_geometry(h, w)
    image = F.pad(source[None].float(), (left, right, top, bottom), mode="replicate")
    ph, pw = image.shape[-2:]
    if tile == 0:
        result = run(image)
    else:
        result = torch.empty(1, 3, 2 * ph, 2 * pw)
        for y in range(0, ph, tile):
            for x in range(0, pw, tile):
                y1, x1 = min(y + tile, ph), min(x + tile, pw)
                sy, sx = max(0, y - 32), max(0, x - 32)
                ey, ex = min(ph, y1 + 32), min(pw, x1 + 32)
                pred = run(image[:, :, sy:ey, sx:ex])
                result[:, :, 2 * y:2 * y1, 2 * x:2 * x1] = \
                    pred[:, :, 2 * (y - sy):2 * (y1 - sy), 2 * (x - sx):2 * (x1 - sx)]
    out = result[0, :, 2 * top:2 * (top + h), 2 * left:2 * (left + w)].float()
    if not torch.isfinite(out).all():
        raise FloatingPointError("Non-finite model reconstruction")
    return out.clamp(0, 1)
