"""Transcribe the reference's literal golden index maps into ``index_maps.json``.

Run once, in a container where the reference checkout is mounted; the tests only
read the JSON it writes.  Sources (literal arrays, read as text with ``ast``):
  - tests/test_debugging.py:13-239  addmm arrangement, m=3 n=4 k=5, blocks 2x2x2:
    source tensors and target tensors of ``simulate_arrangement`` / ``eval``;
  - tests/test_eval.py:11-198       eval of plain, permuted, tiled, tiled-tiled and
    flattened 5x6 tensors with block sizes (2, 3).
Nothing from the reference is imported or executed.
"""

import ast
import json
import sys
from pathlib import Path

REFERENCE = Path(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
OUT = Path(__file__).with_name("index_maps.json")


def literal_calls(tree, func_attr):
    """Literal first arguments of every call `<x>.<func_attr>(...)` / `<func_attr>(...)`."""
    found = []
    for node in ast.walk(tree):
        if isinstance(node, ast.Call):
            f = node.func
            name = f.attr if isinstance(f, ast.Attribute) else getattr(f, "id", None)
            if name == func_attr and node.args:
                try:
                    found.append((node.lineno, ast.literal_eval(node.args[0])))
                except ValueError:
                    pass
    return sorted(found)


def main():
    debugging = ast.parse((REFERENCE / "tests/test_debugging.py").read_text())
    tensors = [v for _, v in literal_calls(debugging, "tensor")]
    # 6 source tensors then 6 target tensors (addmm: input, mat1, mat2, beta, alpha, output)
    evals = ast.parse((REFERENCE / "tests/test_eval.py").read_text())
    arrays = [v for _, v in literal_calls(evals, "array")]
    data = {
        "source": "reference tests/test_debugging.py:13-239 and tests/test_eval.py:11-198",
        "addmm_debugging": {
            "m": 3, "n": 4, "k": 5, "block_size": 2,
            "source_tensors": tensors[:6],
            "target_tensors": tensors[6:12],
        },
        "eval_5x6": {
            "shape": [5, 6], "block_size_m": 2, "block_size_n": 3,
            "plain_2x3": arrays[0],
            "plain": arrays[1],
            "permuted": arrays[2],
            "tiled": arrays[3],
            "tiled_tiled": arrays[4],
            "tiled_tiled_mid_flattened": arrays[5],
            "tiled_tiled_both_flattened": arrays[6],
        },
    }
    OUT.write_text(json.dumps(data))
    print(f"wrote {OUT}: {len(tensors)} debugging tensors, {len(arrays)} eval arrays")


if __name__ == "__main__":
    main()
