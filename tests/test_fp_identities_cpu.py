"""Floating-point identities behind two cheaper forms in the GPU kernels, checked exhaustively on
the CPU (tests/fp_identities.c, built here with gcc):

* the per-token quantizer divides by Markstein's correction (y = 1/s once per row, then
  q0 = x*y, r = fma(s, q0, -x), q = fma(-r, y, q0)) instead of a full IEEE division: over every
  finite row scale and every bf16 x the row can hold, the e4m3 code is the same (x = -0 included:
  the residual formed the other way round, fma(x - s q0, y, q0), gives +0 there);
* exp_f32 in the fused producers is branch-free (a clamp): equal to the branching form, which the
  oracle restates, for every non-NaN fp32 input; for a NaN, silu's dividing path (every group
  holding a NaN takes it) gives the same bits with either form.
A planted mistake (the residual the other way round, a clamp that is too narrow) is caught by the
same checks."""
import os
import shutil
import subprocess

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))


@pytest.fixture(scope="module")
def checker(tmp_path_factory):
    gcc = shutil.which("gcc")
    if gcc is None:
        pytest.skip("gcc not available")
    out = str(tmp_path_factory.mktemp("fpid") / "fp_identities")

    def build(*defs):
        exe = out + "".join(d.replace("=", "_") for d in defs)
        subprocess.run([gcc, "-O2", "-ffp-contract=off", "-fopenmp", *[f"-D{d}" for d in defs],
                        os.path.join(HERE, "fp_identities.c"), "-o", exe, "-lm"], check=True)
        return exe
    return build


def run(exe, *args):
    env = dict(os.environ, OMP_NUM_THREADS=str(min(8, os.cpu_count() or 1)))
    return subprocess.run([exe, *args], capture_output=True, text=True, env=env, timeout=600)


def test_markstein_quotient_gives_the_ieee_code(checker):
    r = run(checker(), "markstein")
    assert r.returncode == 0, r.stdout
    assert r.stdout.startswith("ok ") and int(r.stdout.split()[1]) > 1_000_000_000


def test_branch_free_exp_equals_the_branching_form(checker):
    r = run(checker(), "exp", "31")         # every 31st fp32 input plus every float in 64..128
    assert r.returncode == 0, r.stdout


def test_planted_mistakes_are_caught(checker, tmp_path):
    """The same checks on copies of the identities with a known mistake must fail."""
    src = open(os.path.join(HERE, "fp_identities.c")).read()
    bad = (src.replace("fmaf(-fmaf(s, q0, -x), y, q0)", "fmaf(fmaf(-s, q0, x), y, q0)")
              .replace("fminf(fmaxf(y_in, -104.0f), 89.0f)", "fminf(fmaxf(y_in, -90.0f), 89.0f)"))
    assert bad != src
    p = tmp_path / "planted.c"
    p.write_text(bad)
    exe = str(tmp_path / "planted")
    subprocess.run([shutil.which("gcc"), "-O2", "-ffp-contract=off", "-fopenmp", str(p), "-o", exe,
                    "-lm"], check=True)
    assert run(exe, "markstein").returncode == 1     # -0 quotients lose their sign
    assert run(exe, "exp", "4099").returncode == 1    # e^-95 is subnormal, not 0
