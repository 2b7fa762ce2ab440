"""The public C header driven from compiled code and the Python shim's handle cache, on the GPU.

* tests/abi_smoke (built from tests/abi_smoke.cpp by aeisu_amd/build.py) includes
  include/aeisu_amd.h and runs create -> configure -> upscale -> destroy, a weight-sharing
  sibling, a precision change at configure, the startup report, a non-finite input and the
  error codes, as a native caller of the reference's CudaRuntime would.
* Upscaler uploads the weights once and serves further geometries from sibling runtimes,
  bounded by an LRU of handles.
"""
from __future__ import annotations

import subprocess
import sys

import pytest
import torch

from tests._util import ROOT, WEIGHTS

pytestmark = pytest.mark.gpu


def say(msg: str) -> None:
    print(msg, flush=True)
    sys.stdout.flush()


def test_compiled_cpp_caller(gpu):
    exe = ROOT / "tests" / "abi_smoke"
    if not exe.exists():
        pytest.fail("tests/abi_smoke is not built; run `python -m aeisu_amd.build`")
    say("case: tests/abi_smoke (C++ caller of include/aeisu_amd.h)")
    artifact = WEIGHTS / "aeisu_area_mixed_fp8.bin"
    stored = artifact.read_bytes()[184:216].hex()        # SHA-256 field of the SPYR8F8 header
    res = subprocess.run([str(exe), str(artifact), stored], capture_output=True, text=True, timeout=120)
    say(res.stdout)
    assert res.returncode == 0 and "abi_smoke: OK" in res.stdout, res.stdout + res.stderr


def test_upscaler_shares_weights_and_bounds_handles(gpu):
    from aeisu_amd import _lib as L
    from aeisu_amd import frames
    from aeisu_amd import runtime as R
    say("case: Upscaler sibling handles and LRU bound")
    model = R.load_model(WEIGHTS / "aeisu_area_mixed_fp8.bin", precision="mixed")
    model.max_handles = 2
    shapes = [(40, 56), (64, 96), (72, 104), (40, 56)]
    outs = []
    for h, w in shapes:
        x = frames.scene(h, w, h + w, shapes=5, texture=True).half()[None].cuda().contiguous()
        outs.append(model.run(x))
    torch.cuda.synchronize()
    assert len(model._handles) == 2
    live = [hd for hd in model._handles.values()]
    assert all(L.lib().aeisu_shares_weights(model._main.ptr, hd.ptr) == 1 for hd in live)
    report = model.report()
    say(f"  {report}")
    assert "precision=FP8/FP16-Mixed" in report and "shared_model_users=" in report
    # a fresh model gives the same results: sharing changes nothing numerically
    fresh = R.load_model(WEIGHTS / "aeisu_area_mixed_fp8.bin", precision="mixed")
    for (h, w), got in zip(shapes, outs):
        x = frames.scene(h, w, h + w, shapes=5, texture=True).half()[None].cuda().contiguous()
        assert torch.equal(fresh.run(x), got)
    # weights are counted once: the two live handles hold the weights plus each its own scratch
    import ctypes
    bare = ctypes.c_void_p()
    L.check(L.lib().aeisu_create_sibling(model._main.ptr, ctypes.byref(bare)))
    weights = int(L.lib().aeisu_persistent_bytes(bare))
    L.lib().aeisu_destroy(bare)
    per_handle = [int(L.lib().aeisu_persistent_bytes(hd.ptr)) for hd in live]
    total = model.persistent_bytes()
    say(f"  persistent bytes: weights {weights}, handles {per_handle}, model total {total}")
    assert all(b > weights for b in per_handle)
    assert total == weights + sum(b - weights for b in per_handle)
    model.close()
    fresh.close()


def test_fp32_policy_refuses_the_coefficient_stages(gpu):
    """The FP32 policy has no FP16 coefficient stage: aeisu_controller_async / aeisu_head_async return
    AEISU_ERR_STATE with a message instead of launching the FP16 kernels on absent weights."""
    from aeisu_amd import _lib as L
    from aeisu_amd import runtime as R
    say("case: FP32 policy, controller() and head() refused with AEISU_ERR_STATE")
    model = R.load_model(WEIGHTS / "aeisu_area.pt", precision="fp32")
    frames = torch.rand(1, 3, 40, 56, device=gpu)
    for call in (lambda: model.controller(frames),
                 lambda: model.head(frames, torch.zeros(1, 48, 48, 64, dtype=torch.float16, device=gpu))):
        with pytest.raises(L.AeisuError) as info:
            call()
        assert info.value.code == L.AEISU_ERR_STATE and "FP32 policy" in str(info.value)
    out = model.run(frames)                                 # the whole frame still runs
    torch.cuda.synchronize()
    assert out.shape == (1, 3, 80, 112) and bool(torch.isfinite(out).all())
    # the allocation-free entry point's static array (per GPU, held by the process) is reported
    assert f"static_scratch_bytes={72 << 20}" in model.report()


def test_sibling_runtimes_on_threads(gpu):
    """Runtimes are not thread-safe one by one, but siblings sharing one model may run on their own
    threads (the reference gives each runtime its own engine slot, SrcPyrCudaRuntime.cu:5392-5439):
    four threads each configure a sibling of one Mixed runtime for its own geometry, switch it to the
    FP16 policy and back (the FP16 weights are packed and uploaded once, on first use, under the
    model's lock) and run frames on their own stream, while the other threads do the same; every
    output equals the single-threaded result and every thread's error message stays its own."""
    import ctypes
    import threading
    from aeisu_amd import _lib as L
    from aeisu_amd import frames
    say("case: 4 threads, one sibling runtime each, shared Mixed model, policy switch on first use")
    lib = L.lib()
    main = ctypes.c_void_p()
    blob = (WEIGHTS / "aeisu_area_mixed_fp8.bin").read_bytes()
    buf = ctypes.create_string_buffer(blob, len(blob))
    L.check(lib.aeisu_create_from_memory(buf, len(blob), L.PRECISION["mixed"], ctypes.byref(main)))
    shapes = [(96, 160), (72, 104), (135, 240), (33, 65)]
    inputs = [frames.scene(h, w, 7 + i, shapes=5, texture=True).half()[None].cuda().contiguous()
              for i, (h, w) in enumerate(shapes)]

    def run(rt, x, precision, stream):
        h, w = x.shape[-2:]
        L.check(lib.aeisu_configure(rt, 1, h, w, L.LAYOUT_F16, L.LAYOUT_F16, L.PRECISION[precision], 0))
        out = torch.empty(1, 3, 2 * h, 2 * w, dtype=torch.float16, device=x.device)
        L.check(lib.aeisu_upscale(rt, ctypes.c_void_p(x.data_ptr()), ctypes.c_void_p(out.data_ptr()),
                                  ctypes.c_void_p(stream.cuda_stream)))
        return out

    # single-threaded references on one sibling
    ref_rt = ctypes.c_void_p()
    L.check(lib.aeisu_create_sibling(main, ctypes.byref(ref_rt)))
    s0 = torch.cuda.Stream()
    want = {(i, p): run(ref_rt, x, p, s0).cpu() for i, x in enumerate(inputs) for p in ("mixed", "fp16")}
    lib.aeisu_destroy(ref_rt)
    # a fresh model, so that the FP16 weights are uploaded on first use inside the threads
    lib.aeisu_destroy(main)
    L.check(lib.aeisu_create_from_memory(buf, len(blob), L.PRECISION["mixed"], ctypes.byref(main)))
    errors, results = [], {}
    barrier = threading.Barrier(len(inputs))

    def worker(i):
        try:
            rt = ctypes.c_void_p()
            L.check(lib.aeisu_create_sibling(main, ctypes.byref(rt)))
            stream = torch.cuda.Stream()
            barrier.wait()
            for rep in range(3):
                for p in ("mixed", "fp16"):
                    results[(i, p, rep)] = run(rt, inputs[i], p, stream).cpu()
            # this thread's own error message, unaffected by the others
            bad = lib.aeisu_configure(rt, 1, 9000, 16, 0, 0, 0, 0)
            msg = lib.aeisu_last_error().decode()
            if bad != L.AEISU_ERR_INVALID_ARGUMENT or "8192" not in msg:
                errors.append(f"thread {i}: rc {bad} message {msg!r}")
            lib.aeisu_destroy(rt)
        except Exception as e:                              # reported below
            errors.append(f"thread {i}: {e!r}")

    threads = [threading.Thread(target=worker, args=(i,)) for i in range(len(inputs))]
    for t in threads:
        t.start()
    for t in threads:
        t.join(timeout=120)
    lib.aeisu_destroy(main)
    assert not errors, errors
    assert len(results) == len(inputs) * 2 * 3
    for (i, p, rep), got in results.items():
        assert torch.equal(got, want[(i, p)]), f"thread {i} {p} rep {rep}"


_EAGER_CHILD = """
import sys, torch
from aeisu_amd import runtime as R
from aeisu_amd import _lib as L
out = {}
x = (torch.rand(2, 3, 135, 240, generator=torch.Generator().manual_seed(3)) * 0.9 + 0.05).half().cuda()
for name, path in [("mixed", "aeisu_area_mixed_fp8.bin"), ("int8", "aeisu_int8_fp16.pt"), ("fp16", "aeisu_area.pt"),
                   ("fp32", "aeisu_area.pt")]:
    m = R.load_model("weights/" + path, precision=name)
    out[name] = m.run(x).cpu()
    out[name + "_graph"] = m.run(x, graph=True).cpu()
    out[name + "_unfused"] = m.run(x, flags=L.FLAG_UNFUSED).cpu()
    m.close()
torch.save(out, sys.argv[1])
"""


def test_eager_validation_mode(gpu, tmp_path):
    """AEISU_EAGER_VALIDATE=1 (the reference's AESS_NEURAL_EAGER_VALIDATE diagnostic,
    SrcPyrCudaRuntime.cu:5349-5354) synchronises the stream after every launch outside graph capture;
    a process run with it gives the same frames, eager, graph and per-layer, in every policy."""
    import os
    from aeisu_amd import runtime as R
    say("case: a child process with AEISU_EAGER_VALIDATE=1, every policy, eager / graph / per-layer")
    script = tmp_path / "eager_child.py"
    script.write_text(_EAGER_CHILD)
    result = tmp_path / "frames.pt"
    env = dict(os.environ, AEISU_EAGER_VALIDATE="1", PYTHONPATH=str(ROOT))
    subprocess.run([sys.executable, str(script), str(result)], cwd=str(ROOT), env=env, check=True, timeout=240)
    got = torch.load(result, weights_only=True)
    x = (torch.rand(2, 3, 135, 240, generator=torch.Generator().manual_seed(3)) * 0.9 + 0.05).half().cuda()
    for name, path in [("mixed", "aeisu_area_mixed_fp8.bin"), ("int8", "aeisu_int8_fp16.pt"),
                       ("fp16", "aeisu_area.pt"), ("fp32", "aeisu_area.pt")]:
        m = R.load_model(WEIGHTS / path, precision=name)
        want = m.run(x).cpu()
        m.close()
        for kind in ("", "_graph", "_unfused"):
            assert torch.equal(got[name + kind], want), name + kind
