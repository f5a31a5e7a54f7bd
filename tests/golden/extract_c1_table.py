"""Writes tests/golden/c1_tcq_K2_h2.json: the K=2, h=2 trellis table of the reference's Gaussian rig (BASELINE
config C1), read as data from the reference's results/universal_gaussian.json["tcq_K2_h2"] (JSON, no code)."""
import json
from pathlib import Path

SRC = Path("/root/reference/results/universal_gaussian.json")
OUT = Path(__file__).resolve().parent / "c1_tcq_K2_h2.json"

if __name__ == "__main__":
    d = json.loads(SRC.read_text())["tcq_K2_h2"]
    OUT.write_text(json.dumps({"tab": d["tab"], "step": d["step"], "K": 2, "h": 2, "m": 359,
                               "source": "results/universal_gaussian.json[tcq_K2_h2]"}, indent=1))
    print("wrote", OUT)
