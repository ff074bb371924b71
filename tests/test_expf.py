"""The kernels' expf (litemind_amd/csrc/lm_math.h, a restatement of glibc's
expf) against the C library LiteMind calls through std::exp(float)."""
import ctypes as C

import numpy as np

import oracle_lib as ol


def test_expf_matches_libc_on_every_float_in_range():
    from litemind_amd import workload as wl

    checked = C.c_uint64()
    # every float bit pattern in [-105, 89] (2,240,020,482 values): below -104
    # the result is 0 or a subnormal, above 88.72 it is +inf
    bad = wl.synth().lms_expf_sweep(1, -105.0, 89.0, C.byref(checked))
    assert checked.value == 2_240_020_482
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
