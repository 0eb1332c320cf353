"""Writes atom_reference.json: the per-head atomic reference energies that the
reference's calculator adds to the model energy (src/molfm/data/utils.py:9-289,
``get_data_defult_config``; used as ``atom_reference * unit`` at
src/molfm/interface/model_interface.py:208-223).

The tables are constants of that source file.  This script reads the file as
text (``ast``; nothing of the reference is imported or executed), walks the
function's if / elif chain and records, per branch, how the head name is
matched (``startswith`` or ``==`` on ``head_name.lower()``), the ``unit``
factor and the ``atom_reference`` literal; the ``else`` branch is the default
(zeros, unit 1).  Run it where the reference tree is present:

    python ubio-molfm_amd/make_atom_reference.py /root/reference/src/molfm/data/utils.py
"""
from __future__ import annotations

import ast
import json
import sys
from pathlib import Path

OUT = Path(__file__).resolve().parent / "atom_reference.json"


def _match(test: ast.expr):
    """('startswith' | 'eq', name) of ``data_name.lower().startswith("x")`` or
    ``data_name.lower() == "x"``."""
    if isinstance(test, ast.Call) and isinstance(test.func, ast.Attribute) and test.func.attr == "startswith":
        return "startswith", ast.literal_eval(test.args[0])
    if isinstance(test, ast.Compare) and isinstance(test.ops[0], ast.Eq):
        return "eq", ast.literal_eval(test.comparators[0])
    raise ValueError(f"unrecognised head-name test: {ast.dump(test)}")


def _branch(body):
    unit, ref = None, None
    for st in body:
        if not isinstance(st, ast.Assign) or len(st.targets) != 1 or not isinstance(st.targets[0], ast.Name):
            continue
        name, v = st.targets[0].id, st.value
        if name == "unit":
            unit = float(ast.literal_eval(v))
        elif name == "atom_reference":
            if not (isinstance(v, ast.Call) and isinstance(v.func, ast.Attribute)):
                raise ValueError("atom_reference is not an np.array / np.zeros call")
            if v.func.attr == "array":
                ref = [float(x) for x in ast.literal_eval(v.args[0])]
            elif v.func.attr == "zeros":
                ref = [0.0] * int(ast.literal_eval(v.args[0])[0])
            else:
                raise ValueError(f"atom_reference built by np.{v.func.attr}")
    return unit, ref


def extract(path: str):
    tree = ast.parse(Path(path).read_text())
    fn = next(n for n in ast.walk(tree) if isinstance(n, ast.FunctionDef) and n.name == "get_data_defult_config")
    chain = next(st for st in fn.body if isinstance(st, ast.If))
    heads = []
    node = chain
    while True:
        kind, key = _match(node.test)
        unit, ref = _branch(node.body)
        heads.append({"match": kind, "key": key, "unit": unit, "atom_reference": ref})
        if len(node.orelse) == 1 and isinstance(node.orelse[0], ast.If):
            node = node.orelse[0]
            continue
        unit, ref = _branch(node.orelse)
        default = {"unit": unit, "atom_reference": ref}
        break
    return {"source": "src/molfm/data/utils.py get_data_defult_config", "heads": heads, "default": default}


if __name__ == "__main__":
    src = sys.argv[1] if len(sys.argv) > 1 else "/root/reference/src/molfm/data/utils.py"
    data = extract(src)
    OUT.write_text(json.dumps(data, indent=1) + "\n")
    print(f"wrote {OUT}: " + ", ".join(f"{h['match']} {h['key']!r} ({len(h['atom_reference'])} Z, unit "
                                        f"{h['unit']})" for h in data["heads"]))
