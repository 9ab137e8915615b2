"""The RMSNorm+FP8 kernel's exact-division forms (tokenforge_amd/csrc/norm_row.h).

GPU: the dynamic-scale quotient, y / s by Markstein's correction in fp32 followed by the
v_med3 clamp and the packed e4m3 conversion, gives the codes of the IEEE fp32 division
clamped and encoded by the torch-pinned encoder, for every positive finite fp16 absmax (every
scale a row can hold) and every finite fp16 y of both signs (tfp_norm_quotient_check in this folder's norm_probes.hip). The same run counts the y for which the uncorrected product y * (1 / s)
differs from y / s: a nonzero count shows the correction is needed and the check is not
vacuous. The per-row divisions are checked on the CPU in tests/unit/test_norm_division.py.
"""

from __future__ import annotations

import ctypes
from pathlib import Path

import pytest
import torch

ROOT = Path(__file__).resolve().parents[2]
PROBES = ROOT / "tests" / "gpu" / "lib" / "libtokenforge_norm_probes.so"


@pytest.mark.gpu
def test_dynamic_quotient_codes_exhaustive(device: torch.device) -> None:
    if not PROBES.exists():
        pytest.fail(f"{PROBES} is missing: build it with `python __graft_entry__.py build`")
    lib = ctypes.CDLL(str(PROBES))
    lib.tfp_norm_quotient_check.restype = ctypes.c_int
    lib.tfp_norm_quotient_check.argtypes = [ctypes.c_void_p] * 4
    lib.tfp_norm_quotient_scales.restype = ctypes.c_int
    n = lib.tfp_norm_quotient_scales()
    assert n == 0x7BFF
    out = torch.full((3, n), 0x7FFFFFFF, dtype=torch.int32, device=device)
    rc = lib.tfp_norm_quotient_check(
        out[0].data_ptr(), out[1].data_ptr(), out[2].data_ptr(), torch.cuda.current_stream(device).cuda_stream
    )
    torch.cuda.synchronize(device)
    assert rc == 0
    bad_codes, bad_scale, uncorrected = (int(v) for v in out.sum(dim=1).tolist())
    assert bad_scale == 0, "dynamic_scale differs from max(amax / 448, 1 / (448 * 512))"
    assert bad_codes == 0, f"{bad_codes} (scale, y) pairs encode differently from the IEEE division"
    assert uncorrected > 1000, "the uncorrected product never differs: the check would not see an error"
