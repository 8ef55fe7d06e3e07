"""Regenerate neuralscript_amd/nets/<net>.mlir from oracle/nets/<net>.ns with
the reference compiler built by oracle/Makefile (oracle/_ref/nsc --mlir).

The printer drops MoE(initial_experts: K0); it is restored as `initial=K0`
in the ns.layer.moe comment, the key libnship's plan parser reads.
Runs in the build container only (it needs the reference build).
"""
import os
import re
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
OUT = os.path.join(os.path.dirname(HERE), "neuralscript_amd", "nets")


def ir_of(ns_path):
    text = subprocess.check_output([os.path.join(HERE, "_ref", "nsc"), ns_path, "--mlir"]).decode()
    src = open(ns_path).read()
    m = re.search(r"initial_experts:\s*(\d+)", src)
    if m:
        text = re.sub(r"(// moe\([^)]*?)(ffn=)", r"\g<1>initial=%s, \g<2>" % m.group(1), text)
    return text


def main(names):
    os.makedirs(OUT, exist_ok=True)
    for ns in sorted(os.listdir(os.path.join(HERE, "nets"))):
        if not ns.endswith(".ns"):
            continue
        name = ns[:-3]
        if names and name not in names:
            continue
        with open(os.path.join(OUT, name + ".mlir"), "w") as f:
            f.write(ir_of(os.path.join(HERE, "nets", ns)))


if __name__ == "__main__":
    main(sys.argv[1:])
