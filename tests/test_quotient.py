"""The division-free e4m3 quantisation of the GPU kernels (quant.hip
`quot_abs`: q0 = |v|*r, one fma for the residual, one for the correction,
sign or-ed into the code) against the IEEE quotient the contract prescribes.

The claim is finite: v and amax are bf16, so every (v, amax) pair can be
enumerated; tests/native/fma_quotient_check.c does that in IEEE fp32 on the
host (the GPU's v_mul_f32 / v_fma_f32 are IEEE with fp32 denormals kept).
The full enumeration (1.07e9 pairs, ~40 s) passes; here every 16th amax
pattern plus the extremes are checked, and a planted error must be caught.
"""
import os
import subprocess
import tempfile

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
SRC = os.path.join(HERE, "native", "fma_quotient_check.c")
ORACLE_C = os.path.join(ROOT, "oracle", "fvsr_oracle.c")


def _build(tmp, extra=()):
    exe = os.path.join(tmp, "fma_quotient_check")
    subprocess.run(["gcc", "-O2", "-ffp-contract=off", *extra, "-o", exe, SRC, ORACLE_C, "-lm"],
                   check=True)
    return exe


@pytest.fixture(scope="module")
def checker():
    with tempfile.TemporaryDirectory() as tmp:
        yield _build(tmp)


def test_fma_quotient_codes_sampled(checker):
    # every 16th amax pattern, two different phases, so all exponents appear
    for off in (0, 7):
        r = subprocess.run([checker, "16", str(off)], capture_output=True, text=True)
        assert r.returncode == 0, r.stdout
        assert " mismatches 0" in r.stdout


def test_fma_quotient_codes_extremes(checker):
    # the last amax patterns: largest finite values and +inf (s = inf, r = 0)
    r = subprocess.run([checker, "1", str(0x7f80 - 3)], capture_output=True, text=True)
    assert r.returncode == 0 and " mismatches 0" in r.stdout, r.stdout


def test_fma_quotient_check_catches_a_dropped_correction():
    """Without the correction step (q1 = q0), codes differ from the quotient's:
    the checker must report it."""
    src = open(SRC).read().replace("const float q1 = fmaf(e, r, q0);",
                                   "const float q1 = q0; (void)e;")
    with tempfile.TemporaryDirectory() as tmp:
        planted = os.path.join(tmp, "planted.c")
        open(planted, "w").write(src)
        exe = os.path.join(tmp, "planted")
        subprocess.run(["gcc", "-O2", "-ffp-contract=off", "-o", exe, planted, ORACLE_C, "-lm"],
                       check=True)
        r = subprocess.run([exe, "64", "3"], capture_output=True, text=True)
        assert r.returncode == 1 and " mismatches 0" not in r.stdout, r.stdout


@pytest.mark.parametrize("plant", [
    # no correction step in the signed form
    ("const uint8_t got_signed = code_of(fmaf(t, -r, p0));",
     "const uint8_t got_signed = code_of(p0); (void)t;"),
    # the residual of quot_abs carried over to signed values: -0 then loses
    # its sign (q0 = -0, e = +0, -0 + 0 = +0)
    ("const float t = fmaf(p0, sc, -v);\n        const uint8_t got_signed = code_of(fmaf(t, -r, p0));",
     "const float t = fmaf(-p0, sc, v);\n        const uint8_t got_signed = code_of(fmaf(t, r, p0));"),
])
def test_fma_quotient_check_catches_signed_form_mistakes(plant):
    """The signed form (quot_signed) is checked on the same pairs; a dropped
    correction or the abs-form residual applied to signed values must be
    reported."""
    old, new = plant
    src = open(SRC).read()
    assert old in src
    src = src.replace(old, new)
    with tempfile.TemporaryDirectory() as tmp:
        planted = os.path.join(tmp, "planted.c")
        open(planted, "w").write(src)
        exe = os.path.join(tmp, "planted")
        subprocess.run(["gcc", "-O2", "-ffp-contract=off", "-o", exe, planted, ORACLE_C, "-lm"],
                       check=True)
        r = subprocess.run([exe, "64", "3"], capture_output=True, text=True)
        assert r.returncode == 1 and " mismatches 0" not in r.stdout, r.stdout
