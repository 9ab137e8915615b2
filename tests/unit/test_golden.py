"""The committed golden vectors (tests/golden/golden.json) against the oracle (CPU) and the
HIP kernels (GPU). Regenerate with ``python -m tests.golden.make_golden``."""

from __future__ import annotations

import hashlib
import json
from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import pack as P
from oracle import reference as R
from tests.golden import make_golden as MG

GOLDEN = json.loads((Path(__file__).resolve().parents[1] / "golden" / "golden.json").read_text())


def _sha(a: np.ndarray) -> str:
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def _probe() -> np.ndarray:
    return np.array([int(h, 16) for h in GOLDEN["e4m3"]["probe_f32_hex"]], dtype=np.uint32).view(np.float32)


def test_e4m3_fixture_matches_oracle_and_torch() -> None:
    probe = _probe()
    codes = np.array(GOLDEN["e4m3"]["codes"], dtype=np.uint8)
    assert np.array_equal(R.e4m3_encode(probe), codes)
    assert np.array_equal(torch.from_numpy(probe).to(torch.float8_e4m3fn).view(torch.uint8).numpy(), codes)


def test_repack_fixture_matches_oracle() -> None:
    g = GOLDEN["repack"]
    awq = np.array(g["awq_qweight"], dtype=np.uint32).view(np.int32)
    tf = np.array(g["tf_qweight_t"], dtype=np.uint32).view(np.int32)
    assert np.array_equal(P.repack_awq_to_tf(awq), tf)
    assert np.array_equal(P.repack_tf_to_awq(tf), awq)


def test_config1_fixture_matches_oracle() -> None:
    g = GOLDEN["gemv_config1"]
    qweight, qzeros, scales, x = MG.config1_inputs()
    assert _sha(qweight) == g["sha256_qweight"] and _sha(x) == g["sha256_x"]
    w = P.pack_awq(qweight, qzeros, scales, 128)
    assert _sha(w.qweight_t) == g["sha256_qweight_t"]
    y = R.w4a16_reference(x, w)
    assert np.allclose(y[0, :32], g["ref_first32"], rtol=0, atol=1e-9)
    assert abs(float(y.sum()) - g["ref_sum"]) <= 1e-6 * max(1.0, abs(g["ref_sum"]))


def test_config2_fixture_matches_oracle() -> None:
    g = GOLDEN["rmsnorm_fp8_config2"]
    x, gamma = MG.config2_inputs()
    assert _sha(x) == g["sha256_x"]
    q, s = R.rmsnorm_fp8_reference(x, gamma, g["eps"])
    assert _sha(q) == g["sha256_codes"] and _sha(s) == g["sha256_scales"]


@pytest.mark.gpu
def test_gpu_kernels_match_fixtures(device: torch.device) -> None:
    import tokenforge.kernels.ops  # noqa: F401
    from tokenforge.kernels import pack as tp
    from tokenforge.kernels.hip.rmsnorm_fp8 import e4m3_encode, rmsnorm_fp8_quant
    from tests.numerics.tolerance import contract

    codes = np.array(GOLDEN["e4m3"]["codes"], dtype=np.uint8)
    got = e4m3_encode(torch.from_numpy(_probe()).to(device)).cpu().view(torch.uint8).numpy()
    assert np.array_equal(got, codes)

    g = GOLDEN["repack"]
    awq = torch.from_numpy(np.array(g["awq_qweight"], dtype=np.uint32).view(np.int32)).to(device)
    tf = np.array(g["tf_qweight_t"], dtype=np.uint32).view(np.int32)
    assert np.array_equal(tp.repack_awq_to_tf(awq).cpu().numpy(), tf)

    g1 = GOLDEN["gemv_config1"]
    qweight, qzeros, scales, x = MG.config1_inputs()
    w = tp.pack_awq(*(torch.from_numpy(a).to(device) for a in (qweight, qzeros, scales)), 128)
    tiled = P.pack_awq_tiles(qweight, qzeros, scales, 128)
    assert np.array_equal(w.qweight_t.cpu().numpy(), tiled.qweight_t)
    # Undoing the tile layout gives the reference's TokenForge layout of the fixture.
    back = P.tile_unpack(w.qweight_t.cpu().numpy(), w.scales.cpu().numpy(), w.qzeros.cpu().numpy(), 128)
    assert _sha(back[0]) == g1["sha256_qweight_t"]
    y = torch.ops.tokenforge.w4a16_linear(torch.from_numpy(x).to(device), w.qweight_t, w.scales, w.qzeros,
                                          None, 128, "hip").cpu().numpy().astype(np.float64)
    tol = contract("cuda").atol(x, P.dequantize_tf(P.pack_awq(qweight, qzeros, scales, 128)))
    assert float(np.abs(y[0, :32] - np.array(g1["ref_first32"])).max()) <= tol
    assert abs(float(y.sum()) - g1["ref_sum"]) <= 3584 * tol

    g2 = GOLDEN["rmsnorm_fp8_config2"]
    xr, gamma = MG.config2_inputs()
    q, s = rmsnorm_fp8_quant(torch.from_numpy(xr).to(device), torch.from_numpy(gamma).to(device), g2["eps"])
    assert _sha(q.cpu().view(torch.uint8).numpy()) == g2["sha256_codes"]
    assert _sha(s.cpu().numpy()) == g2["sha256_scales"]
