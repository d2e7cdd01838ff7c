"""Extract the torch golden vectors of the reference's tiny MoE decoder into
tests/golden/clef_mini_expected.json.

    python tests/golden/make_clef_mini.py [/root/reference]

The reference's src/clef/model/mini_expected.in (generated there by
tools/clef_mini_gen.py from a torch manual layer) holds, for a 2-layer decoder
of hidden 64, 4 query / 2 kv heads of 16, 4 experts, top-2, inter 32 on 5
tokens: each layer's output hidden state [5, 64] and its router ids / weights
[5, 2]. Only those numbers are copied; the weights are the closed formula of
the reference test (src/clef/model/tests.rs: val / one_plus / mini_layer),
restated in tests/test_golden_clef.py.
"""
import json
import os
import re
import sys

ref = sys.argv[1] if len(sys.argv) > 1 else "/root/reference"
src = open(os.path.join(ref, "src/clef/model/mini_expected.in")).read()
out = {}
for name, body in re.findall(r"pub const (\w+): \[\w+; \d+\] = \[([^\]]*)\];", src):
    vals = [v.strip() for v in body.split(",") if v.strip()]
    out[name] = [int(v) for v in vals] if name.startswith("IDS") else [float(v) for v in vals]
dst = os.path.join(os.path.dirname(os.path.abspath(__file__)), "clef_mini_expected.json")
with open(dst, "w") as f:
    json.dump({"source": "src/clef/model/mini_expected.in", **out}, f)
print(dst, {k: len(v) for k, v in out.items()})
