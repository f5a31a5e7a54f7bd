"""Extracts the TCQ format tables (trained LUTs, gain steps, masks, scales) from a reference checkout into
ltq-research_amd/ltq_amd/data/tcq_tables.json. Data only: the numbers must be identical for .ltq compatibility.

    python tests/golden/make_tables.py /root/reference

Sources: src/liqk_v2.py:786-833 (TCQ_CONFIG literals, R / RH variants, TCQ_X_SCALE, read as text with ast)
and results/tcq_x_tables.json (night-2 tail-biting tables)."""
import ast
import json
import sys
from pathlib import Path


def main(ref: str):
    src = (Path(ref) / "src" / "liqk_v2.py").read_text()
    tree = ast.parse(src)
    base, x_scale, variants = None, None, {}
    for node in tree.body:
        if isinstance(node, ast.AnnAssign) and isinstance(node.target, ast.Name):
            if node.target.id == "TCQ_CONFIG":
                base = ast.literal_eval(node.value)
            elif node.target.id == "TCQ_X_SCALE":
                x_scale = ast.literal_eval(node.value)
        if isinstance(node, ast.Assign) and len(node.targets) == 1 and isinstance(node.targets[0], ast.Subscript):
            t = node.targets[0]
            if isinstance(t.value, ast.Name) and t.value.id == "TCQ_CONFIG" and isinstance(node.value, ast.Call):
                name = ast.literal_eval(t.slice)
                call = node.value
                parent = ast.literal_eval(call.args[0].slice)
                kw = {k.arg: ast.literal_eval(k.value) for k in call.keywords}
                variants[name] = {"parent": parent, **kw}
    x_tables = json.loads((Path(ref) / "results" / "tcq_x_tables.json").read_text())
    out = {"base": base, "variants": variants, "x_scale": x_scale,
           "x_tables": {k: {kk: v[kk] for kk in ("K", "h", "step", "m_extra", "lut", "sub", "pp") if kk in v}
                        for k, v in x_tables.items()}}
    dst = Path(__file__).resolve().parents[2] / "ltq-research_amd" / "ltq_amd" / "data" / "tcq_tables.json"
    dst.write_text(json.dumps(out, indent=1))
    print("wrote", dst, len(out["x_tables"]), "x tables,", len(variants), "variants")


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
