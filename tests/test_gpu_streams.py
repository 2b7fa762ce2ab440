"""Stream semantics of the boundary: work is ordered on the caller's stream only.

aeisu_upscale_async / aeisu_upscale_graph enqueue on the stream they are given (the reference's
ProcessAsync on its engine stream, SrcPyrCudaRuntime.cu:5135-5206), so a caller that produces its
frames and consumes the outputs on a side stream needs no device-wide synchronisation, and two
runtimes on two streams may run at the same time.  The 1080p Mixed frame takes the compress
exchange between neighbouring body tiles; with a second runtime's kernels holding CUs, a tile whose
neighbours are not resident computes its halo itself after a bounded wait, with the same result, so
every output must equal the one computed alone, bit for bit.
"""
from __future__ import annotations

import sys

import pytest
import torch

from tests._util import WEIGHTS

pytestmark = pytest.mark.gpu


def say(msg: str) -> None:
    print(msg, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def R(gpu):
    from aeisu_amd import runtime
    return runtime


def _frames(n: int, h: int, w: int, seed: int) -> torch.Tensor:
    gen = torch.Generator().manual_seed(seed)
    base = torch.rand(n, 3, h // 8, w // 8, generator=gen)
    smooth = torch.nn.functional.interpolate(base, size=(h, w), mode="bilinear", align_corners=False)
    return (smooth + 0.03 * torch.rand(n, 3, h, w, generator=gen)).clamp(0, 1).half()


@pytest.mark.parametrize("precision,artifact", [("mixed", "aeisu_area_mixed_fp8.bin"), ("fp16", "aeisu_area.pt")])
def test_side_stream_eager_and_graph(R, precision, artifact):
    say(f"case: {precision}, 540x960 frames produced, upscaled and consumed on a side stream")
    host = _frames(3, 540, 960, seed=3)
    model = R.load_model(WEIGHTS / artifact, precision=precision)
    try:
        want = [model.run(host[i:i + 1].cuda().contiguous()) for i in range(3)]
        torch.cuda.synchronize()
        side = torch.cuda.Stream()
        got, got_graph = [], []
        with torch.cuda.stream(side):
            for i in range(3):
                src = host[i:i + 1].to("cuda", non_blocking=False).contiguous()
                src = src * 1                                  # produced by a kernel on the side stream
                out = model.run(src, stream=side)
                got.append(out.float() * 1)                    # consumed on the side stream
                outg = model.run(src, stream=side, graph=True)
                got_graph.append(outg.float() * 1)
        side.synchronize()
        for i in range(3):
            assert torch.equal(got[i], want[i].float()), f"eager frame {i}"
            assert torch.equal(got_graph[i], want[i].float()), f"graph frame {i}"
    finally:
        model.close()


def test_two_runtimes_on_two_streams(R):
    say("case: Mixed 1080p, two runtimes on two streams at once, 4 frames each (compress exchange)")
    host = _frames(4, 1080, 1920, seed=4)
    a = R.load_model(WEIGHTS / "aeisu_area_mixed_fp8.bin", precision="mixed")
    b = R.load_model(WEIGHTS / "aeisu_area_mixed_fp8.bin", precision="mixed")
    try:
        dev = [host[i:i + 1].cuda().contiguous() for i in range(4)]
        want = [a.run(d) for d in dev]
        torch.cuda.synchronize()
        s1, s2 = torch.cuda.Stream(), torch.cuda.Stream()
        s1.wait_stream(torch.cuda.current_stream())
        s2.wait_stream(torch.cuda.current_stream())
        outs1, outs2 = [], []
        for rep in range(3):
            for i in range(4):
                with torch.cuda.stream(s1):
                    outs1.append((i, a.run(dev[i], stream=s1, check_finite=False)))
                with torch.cuda.stream(s2):
                    outs2.append((i, b.run(dev[3 - i], stream=s2, check_finite=False)))
        s1.synchronize()
        s2.synchronize()
        for i, o in outs1:
            assert torch.equal(o, want[i]), f"stream 1 frame {i}"
        for i, o in outs2:
            assert torch.equal(o, want[3 - i]), f"stream 2 frame {3 - i}"
        say(f"  {len(outs1) + len(outs2)} concurrent frames equal to the frames run alone")
    finally:
        a.close()
        b.close()


def test_graph_cache_eviction_while_graphs_run(R):
    """A runtime keeps 16 captured graphs; the 17th (input, output) pair drops them after draining the
    device, so graphs launched just before, still running, finish on intact resources: 24 pairs
    launched back to back without a synchronisation all give the eager result."""
    say("case: Mixed 540x960, 24 graph pairs launched back to back (cache of 16)")
    model = R.load_model(WEIGHTS / "aeisu_area_mixed_fp8.bin", precision="mixed")
    try:
        src = _frames(1, 540, 960, seed=5).cuda().contiguous()
        want = model.run(src)
        outs = [torch.empty_like(want) for _ in range(24)]
        srcs = [src.clone() for _ in range(2)]
        torch.cuda.synchronize()
        for i, o in enumerate(outs):
            model.run(srcs[i % 2], out=o, graph=True, check_finite=False)
        torch.cuda.synchronize()
        for i, o in enumerate(outs):
            assert torch.equal(o, want), f"pair {i}"
    finally:
        model.close()
