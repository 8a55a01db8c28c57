"""Writes readme_spy_128x96_ws15.txt: the braille sparsity picture the
reference's README prints for `display(S)` of the 128x96, ws = 15 Circulant
(README.md:72-91, batch [:, :, 1, 1]; batch [:, :, 1, 2] at :93-112 is the
same picture).  Run in the build container, where the reference is mounted;
the fixture it writes is committed, so nothing reads the reference later.
"""
import os
import sys

README = "/root/reference/README.md"
OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "readme_spy_128x96_ws15.txt")


def block(lines, tag):
    start = next(i for i, line in enumerate(lines) if line.startswith(tag))
    out = []
    for line in lines[start + 1:]:
        if not line:
            break
        out.append(line)
    return out


def main():
    lines = open(README, encoding="utf-8").read().split("\n")
    b1 = block(lines, "[:, :, 1, 1]")
    b2 = block(lines, "[:, :, 1, 2]")
    if b1 != b2 or len(b1) != 19:
        sys.exit("unexpected README layout")
    with open(OUT, "w", encoding="utf-8") as f:
        f.write("\n".join(b1) + "\n")


if __name__ == "__main__":
    main()
