"""Copies the reference's frozen quantization answers into a small fixture (data only).

Reads the JSON data file tests/golden.json of playidea-lab/borch (answers frozen from
real torch, cases.py:8110-8121, 8140-8141) and keeps the path-relevant entries with their
inputs restated from cases.py:8083-8121. Run once where /root/reference exists:
``python tests/golden/extract_ref_golden.py`` -> tests/golden/ref_fake_quantize.json.
"""
import json
import pathlib
import sys

SRC = pathlib.Path(sys.argv[1] if len(sys.argv) > 1 else "/root/reference/tests/golden.json")
OUT = pathlib.Path(__file__).with_name("ref_fake_quantize.json")

KEYS = ["top::fake_quantize(per_tensor)", "top::fake_quantize(zp=2)",
        "top::fake_quantize(per_channel)", "top::grad::fake_quantize", "top::dequantize"]

cases = json.loads(SRC.read_text())["cases"]
grid = [-1.7, 0.3, 2.9, 5.5]
inputs = {
    "top::fake_quantize(per_tensor)": {"x": grid, "scale": 0.5, "zero_point": 0, "qmin": 0, "qmax": 7},
    "top::fake_quantize(zp=2)": {"x": grid, "scale": 0.5, "zero_point": 2, "qmin": 0, "qmax": 7},
    "top::fake_quantize(per_channel)": {"x": [[-1.7, 0.3], [2.9, 5.5]], "scale": [0.5, 0.25],
                                        "zero_point": [0.0, 1.0], "axis": 0, "qmin": 0, "qmax": 7},
    "top::grad::fake_quantize": {"x": grid, "scale": 0.5, "zero_point": 0, "qmin": 0, "qmax": 7},
    "top::dequantize": {"x": grid},
}
out = {"source": "playidea-lab/borch tests/golden.json (frozen from real torch)",
       "cases": {k: {"input": inputs[k], "expected": cases[k]} for k in KEYS}}
OUT.write_text(json.dumps(out, indent=1) + "\n")
print(f"wrote {OUT}")
