"""Regenerate neuralscript_amd/nets/<net>.mlir from oracle/nets/<net>.ns with
oracle/_ref/irdump, built by oracle/Makefile against the reference compiler's
own objects: the text of `nsc --mlir`, plus the instruction attributes that
printer drops (MoE initial experts, binop operator, slice/index/scatter/concat
arguments, constants) as key=value tokens at the end of each comment -- the
keys libnship's plan parser reads.
Runs in the build container only (it needs the reference build).
"""
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
OUT = os.path.join(os.path.dirname(HERE), "neuralscript_amd", "nets")


def ir_of(ns_path):
    return subprocess.check_output([os.path.join(HERE, "_ref", "irdump"), ns_path]).decode()


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
