"""Harvests the reference's stored GEMM vectors into tests/golden/*.json.

Run in a container where /root/reference exists (it never exists on the GPU
box; the JSON it writes is what travels). The only stored numbers the
reference holds for this path are the printed outputs of demo.ipynb cells
1-3 (demo.ipynb:37-46 prints `a`, :72-73 prints `b`, :101-110 prints `a@b`
computed by `cuten.matmul` -> seera_cuda.cuda_matmul -> GEMM.cu:13-91), plus
the 2x2 known answer of Testing/test_14.py:994-1010 and
Testing/diagnose_gpu_ops.py:64-75. The notebook is read as JSON text; no
reference code is imported or executed.
"""
from __future__ import annotations

import json
import os
import re

REF = "/root/reference"
OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "demo_matmul.json")


def _numbers(text: str) -> list[float]:
    return [float(t) for t in re.findall(r"-?\d+\.\d*(?:e[-+]?\d+)?|-?\d+", text)]


def _stdout(cell) -> str:
    return "".join("".join(o.get("text", [])) for o in cell.get("outputs", [])
                   if o.get("output_type") == "stream")


def main() -> None:
    nb = json.load(open(os.path.join(REF, "demo.ipynb")))
    cells = nb["cells"]
    assert "".join(cells[1]["source"]).strip() == "a"
    assert "".join(cells[2]["source"]).strip() == "b"
    assert "".join(cells[3]["source"]).strip() == "a@b"
    a = _numbers(_stdout(cells[1]))
    b = _numbers(_stdout(cells[2]))
    c = _numbers(_stdout(cells[3]))
    assert (len(a), len(b), len(c)) == (12, 4, 12)
    golden = {
        "source": "demo.ipynb cells 1-3 (lines 37-46, 72-73, 101-110)",
        "entry": "cuda_matmul(A, B, C, M=2, N=2, K=2, Nbatch=3)",
        "a_shape": [3, 2, 2], "a": a,
        "b_shape": [2, 2], "b": b,
        "c_shape": [3, 2, 2], "c": c,
        "note": "a is printed with float32 repr; the printed c equals fp32 "
                "matmul of fp16-rounded operands exactly",
        "kat_2x2": {"source": "Testing/test_14.py:994-1010",
                    "a": [[1, 2], [3, 4]], "b": [[5, 6], [7, 8]],
                    "c": [[19, 22], [43, 50]]},
    }
    with open(OUT, "w") as f:
        json.dump(golden, f, indent=1)
    print("wrote", OUT)


if __name__ == "__main__":
    main()
