"""Collect the reference's recorded structure of every qualified TensorProduct
family (benchmarks/eqx/results/raw/C*/qualification-*.json: paths, parameters,
width, error maxima) into tests/golden/qualification_structure.json.

Run in the build container: python tests/golden/make_structure.py /root/reference
"""
import json
import sys
from pathlib import Path

root = Path(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
records = []
for path in sorted((root / "benchmarks/eqx/results/raw").glob("C*/qualification-*.json")):
    data = json.loads(path.read_text())
    records.append({"C": data["C"], "m_max": data["m_max"], "parity": data["parity"],
                    "N": data["N"], "paths": data["paths"], "parameters": data["parameters"],
                    "width": data["width"], "errors": data.get("candidate_errors"),
                    "source": str(path.relative_to(root))})
out = Path(__file__).resolve().parent / "qualification_structure.json"
out.write_text(json.dumps(records, indent=1) + "\n")
print(len(records), "records ->", out)
