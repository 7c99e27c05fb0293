"""Writes tk_real_decode.log: three launches of the reference's real GLM-5.2
decode routing corpus (test/76.real_decode/dataset.tk_info, per-rank expert
counts in its TK_INFO line format), excerpted verbatim as data:

* 45400  -- the corpus's most skewed launch (T=512, one expert with 398 rows,
            116 of 256 experts active);
* 84900  -- a median launch (T=512, busiest expert 210 rows, 242 active);
* 151000 -- the smallest (T=96).

Run from the repository root with the reference checked out at
/root/reference; the tests read only the committed excerpt."""
import re
import sys

SRC = "/root/reference/test/76.real_decode/dataset.tk_info"
KEEP = (45400, 84900, 151000)


def main(out="tests/golden/tk_real_decode.log"):
    lines = []
    for line in open(SRC, encoding="utf-8"):
        m = re.search(r"\[TK_INFO\] rank=(\d+) launch=(\d+) n=8 : ", line)
        if m and int(m.group(2)) in KEEP:
            lines.append(line.rstrip("\n"))
    assert len(lines) == 32 * len(KEEP), len(lines)
    with open(out, "w") as f:
        f.write("# excerpt of test/76.real_decode/dataset.tk_info (launches "
                + ", ".join(map(str, KEEP)) + ")\n")
        f.write("\n".join(lines) + "\n")


if __name__ == "__main__":
    main(*sys.argv[1:])
