# SPDX-License-Identifier: Apache-2.0
"""Writes tests/golden/ref_container.npz: a container written by the
reference's own test-container tool (tools/make_test_container.py, stdlib
only: a Kimi-Linear-shaped model at 1/18 scale, 4 layers, 8 experts, VQ3R
banks, Q4G trunk), so that the reader is checked against the engine's
format as the engine's tooling writes it, not only against this repo's
writer.  The fixture is the tool's output files, byte for byte, each as a
uint8 array named after the file.

  python tests/golden/make_ref_container.py [/root/reference]
"""
import os
import subprocess
import sys
import tempfile

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))


def main():
    ref = sys.argv[1] if len(sys.argv) > 1 else "/root/reference"
    tool = os.path.join(ref, "tools", "make_test_container.py")
    with tempfile.TemporaryDirectory() as d:
        out = os.path.join(d, "tiny")
        subprocess.check_call([sys.executable, tool, out, "--seed", "0"])
        files = {f: np.frombuffer(open(os.path.join(out, f), "rb").read(), np.uint8)
                 for f in sorted(os.listdir(out))}
    np.savez_compressed(os.path.join(HERE, "ref_container.npz"), **files)
    print("ref_container.npz:", ", ".join(f"{k} {v.size}" for k, v in files.items()))


if __name__ == "__main__":
    main()
