"""Write nf4_code.json: the NF4 code table as the reference's source holds it.

Reads app/engine/nf4gemv.py of the reference tree as text and evaluates only
the `NF4_CODE = (...)` tuple literal with `ast.literal_eval` (nothing is
imported or executed). Usage: python tests/golden/make_nf4_code.py [REF_ROOT]
"""

import ast
import json
import sys
from pathlib import Path

root = Path(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
src = (root / "app/engine/nf4gemv.py").read_text()
tree = ast.parse(src)
for node in tree.body:
    if isinstance(node, ast.Assign) and any(getattr(t, "id", "") == "NF4_CODE" for t in node.targets):
        code = ast.literal_eval(node.value)
        break
else:
    raise SystemExit("NF4_CODE not found")
out = Path(__file__).resolve().parent / "nf4_code.json"
out.write_text(json.dumps({"source": "app/engine/nf4gemv.py:75-92", "NF4_CODE": list(code)}, indent=1) + "\n")
print(f"wrote {out} ({len(code)} values)")
