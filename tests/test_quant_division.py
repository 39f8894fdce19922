"""The fused W8A8 quantizer divides by the row scale s through one reciprocal per row:
q = x * y, r = fma(-q, s, x), q' = copysign(fma(r, y, q), x) with y = 1 / s. It must give
the e4m3 codes of the per-token quantizer's IEEE divide x / s for every input. This is an
exhaustive CPU check (tests/c/quant_div_check.c): every positive finite bf16 and fp16 amax
against every x of the same format with |x| <= amax, both signs. The same program without
the correction step must fail, and its e4m3 encoder must agree with the oracle's."""

import os
import shutil
import subprocess
import tempfile

import numpy as np
import pytest

from oracle import oracle as O

SRC = os.path.join(os.path.dirname(os.path.abspath(__file__)), "c", "quant_div_check.c")


@pytest.fixture(scope="module")
def checker():
    if shutil.which("gcc") is None:
        pytest.skip("gcc not available")
    d = tempfile.mkdtemp()
    exe = os.path.join(d, "quant_div_check")
    subprocess.run(["gcc", "-O2", "-fopenmp", "-ffp-contract=off", SRC, "-o", exe, "-lm"], check=True)
    yield exe
    shutil.rmtree(d, ignore_errors=True)


def _run(exe, *args, stdin=None):
    return subprocess.run([exe, *args], input=stdin, capture_output=True, text=True, check=True,
                          env={**os.environ, "OMP_NUM_THREADS": str(min(8, os.cpu_count() or 1))}).stdout


@pytest.mark.parametrize("fmt", ["bf16", "fp16"])
def test_reciprocal_division_gives_the_quantizer_codes(checker, fmt):
    bad_code, _, pairs = map(int, _run(checker, fmt).split())
    assert pairs > 10**9 and bad_code == 0


def test_check_fails_without_the_correction_step(checker):
    bad_code, _, _ = map(int, _run(checker, "bf16", "nocorrect").split())
    assert bad_code > 1000


def test_checker_encoder_matches_oracle(checker):
    rng = np.random.default_rng(3)
    v = np.concatenate([
        (rng.standard_normal(4000) * np.exp2(rng.integers(-12, 9, 4000))).astype(np.float32),
        np.array([0.0, -0.0, 2.0**-10, 1.5 * 2.0**-9, 448.0, 464.0, -464.0, 2.0**-6, 15.0 / 8 * 2.0**-7], np.float32),
    ])
    v = v[np.abs(v) <= 464]
    got = np.array(_run(checker, "encode", stdin="\n".join(repr(float(x)) for x in v)).split(), dtype=np.int64)
    assert np.array_equal(got, O.e4m3_encode(v).astype(np.int64))
