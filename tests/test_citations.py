"""Every reference citation `path:line[-line]` in the committed sources and notes names a file of
the reference checkout and lines that exist in it (skipped where the checkout is absent)."""
import os
import re
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
REF = "/root/reference"
CITE = re.compile(r"((?:spike|tools|docs|outputs)/[\w./-]+?\.(?:py|md|json|sh|txt))"
                  r"((?::\d+(?:-\d+)?)(?:,\d+(?:-\d+)?)*)?")
# a bare ":N-M" later on a line that cites a path refers to that path ("a.py:1-5, :9-12")
BARE = re.compile(r"(?<![\w.\[/:])(:\d+(?:-\d+)?(?:,\d+(?:-\d+)?)*)(?![\w.])")
# driver-written records and the survey quote the reference too, but are not this build's text
SKIP_PREFIX = ("SURVEY", "VERDICT", "ADVICE", "BASELINE", "BENCH_", "GPUTEST_", "SCALE_",
               "MULTICHIP_", "PROGRESS")


@pytest.mark.skipif(not os.path.isdir(REF), reason="reference checkout not present")
def test_reference_citations_point_at_existing_lines():
    files = subprocess.run(["git", "ls-files"], cwd=ROOT, capture_output=True, text=True,
                           check=True).stdout.split()
    lengths, bad = {}, []
    for f in files:
        if f.startswith(SKIP_PREFIX) or f.endswith((".npz", ".so")):
            continue
        try:
            text = open(os.path.join(ROOT, f), encoding="utf-8").read()
        except (UnicodeDecodeError, FileNotFoundError):
            continue
        for ln, line in enumerate(text.splitlines(), 1):
            cites = [(m.start(), m.end(), m.group(1), m.group(2)) for m in CITE.finditer(line)]
            for b in BARE.finditer(line):
                prev = [c for c in cites if c[1] <= b.start()]
                if prev and not any(s <= b.start() < e for s, e, _, _ in cites):
                    cites.append((b.start(), b.end(), prev[-1][2], b.group(1)))
            for _, _, path, rng in cites:
                full = os.path.join(REF, path)
                if not os.path.isfile(full):
                    bad.append(f"{f}:{ln} {path}: no such reference file")
                    continue
                if rng:
                    if path not in lengths:
                        with open(full, errors="replace") as fh:
                            lengths[path] = sum(1 for _ in fh)
                    for part in rng[1:].split(","):
                        lo, _, hi = part.partition("-")
                        hi = int(hi or lo)
                        if int(lo) < 1 or hi > lengths[path] or hi < int(lo):
                            bad.append(f"{f}:{ln} {path}{rng}: file has {lengths[path]} lines")
    assert not bad, "\n".join(bad)
