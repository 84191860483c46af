"""The rasterizer's 2^t (blend_exp2f in fastgs_core_amd/csrc/fgs_device.hpp)
takes f and floor(t) from v_fract_f32 and v_cvt_flr_i32_f32, and the CPU
oracle (orc_blend_exp2f) computes them as fminf(t - floorf(t), 0x1.fffffep-1)
and floorf(t).  The checker built beside the library
(fastgs_core_amd/check_fract_floor, from csrc/check_fract_floor.hip) compares
the two on the GPU for every float t in [-126, 8]; any mismatch would make
n_contrib depend on which side computed alpha."""
import os
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CHECK = os.path.join(ROOT, "fastgs_core_amd", "check_fract_floor")


@pytest.mark.gpu
def test_fract_and_floor_match_the_oracle_for_every_float():
    assert os.path.exists(CHECK), "build the library first (make -C fastgs_core_amd/csrc)"
    print("running", CHECK, flush=True)
    r = subprocess.run([CHECK], capture_output=True, text=True, timeout=120)
    print(r.stdout, r.stderr, flush=True)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "mismatches 0," in r.stdout
    assert "checked 2214330370 floats" in r.stdout
