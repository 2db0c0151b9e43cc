"""Writes reference_roots.json: every (modulus, n, root) record that the
reference's own result snapshots hold for its cyclic NTT runs.

Run in a container where the reference tree is present (it is read as data,
not imported):  python tests/golden/extract_reference_roots.py [/root/reference]

The reference passes cuntt::find_primitive_power_of_two_root(log2 n, q)
(src/reference.cpp:564-582) to every NTT backend it times, and its runner
records the root beside the modulus and shape in
experiments/snapshots/*/identities.json and snapshot.json. Those records pin
the root convention the oracle restates.
"""
import glob
import json
import os
import sys

HERE = os.path.dirname(os.path.abspath(__file__))


def records(root):
    found = {}
    for path in sorted(glob.glob(os.path.join(root, "experiments", "snapshots", "**", "*.json"), recursive=True)):
        try:
            with open(path) as f:
                data = json.load(f)
        except (OSError, ValueError):
            continue
        stack = [data]
        while stack:
            node = stack.pop()
            if isinstance(node, dict):
                if isinstance(node.get("modulus"), int) and isinstance(node.get("root"), int) \
                        and isinstance(node.get("logical_shape"), list) and len(node["logical_shape"]) == 1:
                    key = (node["modulus"], node["logical_shape"][0], node["root"])
                    found.setdefault(key, os.path.relpath(path, root))
                stack.extend(node.values())
            elif isinstance(node, list):
                stack.extend(node)
    return [{"modulus": q, "n": n, "root": r, "source": src} for (q, n, r), src in sorted(found.items())]


if __name__ == "__main__":
    root = sys.argv[1] if len(sys.argv) > 1 else "/root/reference"
    out = records(root)
    with open(os.path.join(HERE, "reference_roots.json"), "w") as f:
        json.dump({"description": "cyclic NTT roots recorded by the reference's benchmark runner "
                                  "(modulus, transform length n, forward root)", "records": out}, f, indent=1)
    print(f"{len(out)} records")
