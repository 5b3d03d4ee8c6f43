"""Writes tiered_397b_hot.json: the hot (4-bit) expert sets of the 397B model
from the reference's hot_experts_397B.json (data file, read as JSON), the input
repack_experts_tiered.py:256-276 turns into a tiered manifest.  Run in a
container that has /root/reference; the fixture is committed."""
import json
import os
import sys

src = sys.argv[1] if len(sys.argv) > 1 else "/root/reference/hot_experts_397B.json"
d = json.load(open(src))
out = {"source": "hot_experts_397B.json", "num_layers": d["num_layers"], "num_experts": d["num_experts"],
       "threshold": d["threshold"], "total_hot": d["total_hot"], "total_cold": d["total_cold"],
       "hot_experts": {k: sorted(int(e) for e in v) for k, v in d["hot_experts"].items()}}
with open(os.path.join(os.path.dirname(os.path.abspath(__file__)), "tiered_397b_hot.json"), "w") as f:
    json.dump(out, f, separators=(",", ":"))
