"""Builds the C++ test programs under tests/cpp (test infrastructure: they link the oracle, the
checker, next to the product libraries)."""
import os
import subprocess

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
PKG = os.path.join(ROOT, "talos-xii_amd")
ORACLE = os.path.join(ROOT, "oracle")
TAPE_TEST = os.path.join(HERE, "test_tape")


def build():
    tmp = TAPE_TEST + ".tmp"
    cmd = ["g++", "-O2", "-std=c++17", "-Wall", os.path.join(HERE, "test_tape.cpp"), "-o", tmp,
           f"-L{PKG}", "-ltalos_tape", "-ltalos_hip", f"-L{ORACLE}", "-loracle",
           "-Wl,-rpath,$ORIGIN/../../talos-xii_amd", "-Wl,-rpath,$ORIGIN/../../oracle"]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"g++ failed for test_tape.cpp:\n{r.stdout}\n{r.stderr}")
    os.replace(tmp, TAPE_TEST)
    return TAPE_TEST


if __name__ == "__main__":
    print(build())
