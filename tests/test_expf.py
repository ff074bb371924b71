"""The kernels' expf (litemind_amd/csrc/lm_math.h, a restatement of glibc's
expf) against the C library LiteMind calls through std::exp(float)."""
import ctypes as C

import numpy as np

import oracle_lib as ol


def test_expf_matches_libc_on_a_sweep_of_all_floats():
    from litemind_amd import workload as wl

    checked = C.c_uint64()
    # every 4099th bit pattern in [-105, 89]: ~550k values across all exponents
    bad = wl.synth().lms_expf_sweep(4099, -105.0, 89.0, C.byref(checked))
    assert checked.value > 500_000
    assert bad == 0


def test_expf_special_values():
    from litemind_amd import workload as wl

    xs = np.array([0.0, -0.0, 1.0, -1.0, 88.72, 88.73, -87.3, -103.9, -104.0, -200.0, np.inf, -np.inf, np.nan,
                   1e-30, -1e-30], np.float32)
    out = np.zeros_like(xs)
    wl.synth().lms_expf_ref(xs.ctypes.data, out.ctypes.data, xs.size)
    libc = np.array([ol.oracle().orc_expf(float(v)) for v in xs], np.float32)
    same = (out.view(np.uint32) == libc.view(np.uint32)) | (np.isnan(out) & np.isnan(libc))
    assert np.all(same), (xs[~same], out[~same], libc[~same])
