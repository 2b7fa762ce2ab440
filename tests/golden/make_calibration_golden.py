"""Extract the DIV2K-L1 calibration record of the reference into a small fixture.

Source (reference checkout, data file): research/studies/div2k_l1_3000_mixed/calibration/
calibration_report.json -- the record the reference's external FP8 exporter wrote when it
produced research/studies/div2k_l1_3000_mixed/artifact/adaptive_fp8.bin (shipped here as
weights/aeisu_div2k_l1_mixed_fp8.bin).  Kept: per-channel selected weight percentile and
scale, the FP8 bias corrections, the activation scales and the scale-search selections.

Run in the build container only (the reference does not exist on the GPU box):
    python tests/golden/make_calibration_golden.py /root/reference
"""
import json
import sys
from pathlib import Path

ref = Path(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
rep = json.loads((ref / "research/studies/div2k_l1_3000_mixed/calibration/calibration_report.json").read_text())
out = {
    "source": "research/studies/div2k_l1_3000_mixed/calibration/calibration_report.json",
    "method": rep["method"],
    "checkpoint_sha256": rep["checkpoint_sha256"],
    "weights": {w["layer"]: [[c["selected_percentile"], c["scale"]] for c in w["channels"]]
                for w in rep["weight_quantization"]},
    "fp8_bias_correction": rep["fp8_bias_correction"],
    "activation_scales": rep["activation_scales"],
    "scale_search_selected": [[s["pass"], s["boundary"], s["selected"]] for s in rep["scale_search"]],
}
dst = Path(__file__).with_name("div2k_calibration_record.json")
dst.write_text(json.dumps(out, separators=(",", ":")))
print(f"wrote {dst} ({dst.stat().st_size} bytes)")
