"""Extract a new file's text from a unified diff (the reference ships its CPU core only as a patch).

Used by oracle/Makefile to build the reference CPU core into oracle/_ref/ (git-ignored).
Usage: python3 extract_ref.py PATCH PATH_IN_PATCH OUT_FILE
Reads the '+++ b/<PATH_IN_PATCH>' hunk '@@ -0,0 +1,N @@' and writes its N added lines.
"""
import re
import sys


def extract(patch_path, rel, out_path):
    lines = open(patch_path, encoding="utf-8", errors="surrogateescape").read().split("\n")
    for i, ln in enumerate(lines):
        if ln == "+++ b/" + rel:
            m = re.match(r"@@ -0,0 \+1,(\d+) @@", lines[i + 1])
            if not m:
                raise SystemExit(f"{rel}: not a new-file hunk")
            n = int(m.group(1))
            body = lines[i + 2:i + 2 + n]
            if any(not b.startswith("+") for b in body):
                raise SystemExit(f"{rel}: unexpected line in hunk")
            with open(out_path, "w", encoding="utf-8", errors="surrogateescape") as f:
                f.write("\n".join(b[1:] for b in body) + "\n")
            return
    raise SystemExit(f"{rel}: not found in {patch_path}")


if __name__ == "__main__":
    extract(sys.argv[1], sys.argv[2], sys.argv[3])
