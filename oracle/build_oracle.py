"""Compile oracle/c/*.c into oracle/_build/liboracle.so with gcc (test oracle
only; built by __graft_entry__.build() and on first use by oracle.router)."""
import os
import subprocess

HERE = os.path.dirname(os.path.abspath(__file__))
OUT = os.path.join(HERE, "_build", "liboracle.so")


def build() -> str:
    os.makedirs(os.path.dirname(OUT), exist_ok=True)
    srcs = sorted(os.path.join(HERE, "c", f) for f in os.listdir(os.path.join(HERE, "c"))
                  if f.endswith(".c"))
    tmp = OUT + ".tmp"
    # strict IEEE float: no contraction, no fast-math; fmaf is libm's correctly rounded fma
    cmd = ["gcc", "-O2", "-fPIC", "-shared", "-ffp-contract=off", "-fno-fast-math", *srcs,
           "-o", tmp, "-lm"]
    subprocess.run(cmd, check=True)
    os.replace(tmp, OUT)
    return OUT


if __name__ == "__main__":
    print(build())
