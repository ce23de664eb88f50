"""The softmax kernels scale their exp2 polynomial by ldexp (v_ldexp_f32)
where the host form multiplies by 2^k built in the exponent field
(mx_common.hpp: exp2_poly_neg, exp2_poly_aie_neg). Over [-120, 0], the
softmaxes' clamped argument range, the product is exact and normal, so the two
must agree bit for bit; this runs the check on the CPU over a stride of the
floats there (every float with MX_EXP2_EXHAUSTIVE=1, about a minute and a
half), in the fused and the unfused Horner forms."""
import os
import shutil
import subprocess

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))


@pytest.mark.skipif(shutil.which("gcc") is None, reason="needs gcc")
def test_ldexp_scaling_equals_the_exponent_field_multiply(tmp_path):
    exe = tmp_path / "exp2_scaling"
    subprocess.run(["gcc", "-O2", "-ffp-contract=off", "-o", str(exe),
                    os.path.join(HERE, "cpu_checks", "exp2_scaling.c"), "-lm"], check=True)
    stride = "1" if os.environ.get("MX_EXP2_EXHAUSTIVE") == "1" else "97"
    r = subprocess.run([str(exe), stride], capture_output=True, text=True)
    assert r.returncode == 0, r.stdout + r.stderr
    n = int(r.stdout.split()[-1])
    # both forms, every `stride`-th float of [-120, 0]
    assert n >= 2 * (0x42F00000 // int(stride))
