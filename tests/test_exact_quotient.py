"""Runs tests/exact_quotient_check.c: the int8 quantize kernel's reciprocal-and-correction
quotient gives the same codes as IEEE division for every fp16 and bf16 (element, scale)
pair, and for random fp32 pairs; and for fp16 with a normal scale the plain product with
the reciprocal already does (about a minute of CPU)."""

from __future__ import annotations

import os
import re
import subprocess

from conftest import REPO_ROOT


def test_markstein_quotient_is_exact_where_codes_depend_on_it(tmp_path):
    src = os.path.join(REPO_ROOT, "tests", "exact_quotient_check.c")
    exe = str(tmp_path / "eqc")
    subprocess.run(["gcc", "-O2", "-mfma", "-ffp-contract=off", "-o", exe, src, "-lm"], check=True)
    out = subprocess.run([exe, "2000000"], check=True, capture_output=True, text=True, timeout=900).stdout
    rows = dict(re.findall(r"(\w+) pairs=\d+ code_mismatch=(\d+ quotient_mismatch=\d+)", out))
    assert set(rows) == {"bf16", "f16", "f32"}, out
    for name, counts in rows.items():
        assert counts == "0 quotient_mismatch=0", (name, out)
    # fp16 with a normal scale: the plain product RN(t * RN(1/s)) already gives every code
    assert re.search(r"f16 product_mismatch=0\b", out), out
