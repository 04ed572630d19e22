"""Writes tests/golden/weights-manifest.txt: the reference's expected checkpoint
tensor list (docs/weights-manifest.txt, name<TAB>shape per line, [unet] and
[vae] sections), copied as data for the CPU tests that pin the UNet and VAE
tensor sets. Run from the repository root with the reference mounted:

    python tests/golden/make_manifest_fixture.py /root/reference
"""
from __future__ import annotations

import os
import sys


def main():
    ref = sys.argv[1] if len(sys.argv) > 1 else "/root/reference"
    src = os.path.join(ref, "docs", "weights-manifest.txt")
    dst = os.path.join(os.path.dirname(os.path.abspath(__file__)), "weights-manifest.txt")
    with open(src, encoding="utf-8") as f:
        text = f.read()
    with open(dst, "w", encoding="utf-8", newline="\n") as f:
        f.write(text)
    print(f"wrote {dst} ({text.count(chr(10))} lines)")


if __name__ == "__main__":
    main()
