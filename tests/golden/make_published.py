"""Write published.json: the reference's own published end-to-end results for this path, read from its results
files (data, not code). Run in a container that has the reference checked out:

    python tests/golden/make_published.py /root/reference

Source rows: results/sinkhorn_trn1.2xlarge_2026-10-30.csv, the converge runs of the mixture clouds 10k x 10k,
d 64, eps 0.05, tol 1e-4, mean normalisation (examples/sinkhorn_benchmark.py:79, 105-118): `ref_cost` is the
float64 CPU run (preset "cpu", torch half-step), `cost` the float32 device runs (torch half-step; NKI kernel).
"""

import csv
import json
import sys
from pathlib import Path


def main(root):
    rows = list(csv.DictReader((Path(root) / "results/sinkhorn_trn1.2xlarge_2026-10-30.csv").open()))
    conv = [r for r in rows if r["conv_iters"] and r["n"] == "10000" and r["d"] == "64" and r["eps"] == "0.05"]
    ref_costs = {r["ref_cost"] for r in conv}
    assert len(ref_costs) == 1, ref_costs
    torch32 = [r for r in conv if r["kernel"] == "torch"]
    nki32 = [r for r in conv if r["kernel"] == "nki" and r["cores"] == "1"]
    out = {
        "mixture_10k_eps0.05": {
            "source": "results/sinkhorn_trn1.2xlarge_2026-10-30.csv (converge runs, n = m = 10000, d = 64, eps 0.05)",
            "inputs": "x = mixture(10000, 64, k=20, seed=0), y = mixture(10000, 64, k=20, seed=1, shift=0.3)",
            "options": {"eps": 0.05, "tol": 1e-4, "max_iters": 2000, "normalize": "mean", "block": 2048},
            "iterations": int(conv[0]["conv_iters"]),
            "cost_float64": float(ref_costs.pop()),
            "cost_float32_torch": float(torch32[0]["cost"]),
            "error_float32_torch": float(torch32[0]["conv_error"]),
            "cost_float32_nki": float(nki32[0]["cost"]),
            "error_float32_nki": float(nki32[0]["conv_error"]),
        }
    }
    dst = Path(__file__).resolve().parent / "published.json"
    dst.write_text(json.dumps(out, indent=2) + "\n")
    print(dst.read_text())


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
