"""Copies the k-quant golden blocks on the decode path out of the reference's
own test data (tests/data/kquant_cases.json there: random blocks and gguf-py's
decoded values for them, written by its tools/gen_kquant_cases.py, seed 7).

Run here, where /root/reference exists; the output is a data fixture (inputs
and expected outputs only) that the tests read on any machine.
"""
import json
import os

SRC = "/root/reference/tests/data/kquant_cases.json"
DST = os.path.join(os.path.dirname(os.path.abspath(__file__)), "kquant_cases.json")
KEEP = ("q4_1", "q4_K", "q6_K")  # the block types the decode path loads

with open(SRC) as f:
    cases = json.load(f)
kept = [c for c in cases if c["type"] in KEEP]
with open(DST, "w") as f:
    json.dump(kept, f, indent=0)
print("wrote", DST, [c["type"] for c in kept])
