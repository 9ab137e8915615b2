"""T0: dispatcher decisions, counters and launch-config validity (test_dispatch.py in the
reference, with the gfx950 buckets, arch key, kernel families and HIP-only policy)."""

from __future__ import annotations

import pytest
from hypothesis import given
from hypothesis import strategies as st

from tokenforge.kernels import dispatch
from tokenforge.kernels.config import (
    GEMM_MIN_M,
    GEMV_MAX_M,
    M_BUCKETS,
    VARIANTS,
    GemmConfig,
    candidate_configs,
    default_config,
    family_for_bucket,
    m_bucket,
)
from tokenforge.kernels.metrics import FALLBACKS, KERNEL_CALLS


@pytest.fixture(autouse=True)
def _reset_counters() -> None:
    KERNEL_CALLS.reset()
    FALLBACKS.reset()


@given(st.integers(1, 4096))
def test_m_bucket_is_tight(m: int) -> None:
    b = m_bucket(m)
    assert b in M_BUCKETS
    assert b >= m
    assert b == 1 or b // 2 < m


def test_m_bucket_rejects_out_of_range() -> None:
    with pytest.raises(ValueError, match=">= 1"):
        m_bucket(0)
    with pytest.raises(ValueError, match="exceeds"):
        m_bucket(4097)


@pytest.mark.parametrize(
    ("n", "k", "group", "dtype", "arch", "backend", "expected"),
    [
        (1152, 896, 128, "float16", "gfx950", "hip", None),
        (1152, 896, 128, "torch.float16", None, "triton", None),
        (1152, 896, 128, "float16", "gfx950", "cuda", None),
        (1152, 896 + 64, 128, "float16", "gfx950", "hip", "unsupported_shape"),  # F2
        (1150, 896, 128, "float16", "gfx950", "hip", "unsupported_shape"),
        (1152, 896, 256, "float16", "gfx950", "hip", "unsupported_group_size"),
        (1152, 896, 128, "bfloat16", "gfx950", "hip", "unsupported_dtype"),
        (1152, 896, 128, "float16", "gfx942", "hip", "unsupported_arch"),
        (1152, 896, 128, "float16", "gfx950", "marlin", "kill_switch"),
    ],
)
def test_layer_support(n, k, group, dtype, arch, backend, expected) -> None:  # type: ignore[no-untyped-def]
    assert dispatch.layer_support(n, k, group, dtype, arch, backend) == expected


@pytest.mark.parametrize(
    ("m", "backend", "kernel", "bucket"),
    [
        (1, "hip", "hip_gemv", "1"),
        (3, "triton", "hip_gemv", "4"),
        (4, "cuda", "hip_gemv", "4"),
        (5, "hip", "hip_gemv", "8"),
        (8, "hip", "hip_gemv", "8"),
        (9, "hip", "hip_gemm", "16"),  # bucket 16 starts the GEMM family
        (32, "hip", "hip_gemm", "32"),
        (33, "hip", "hip_gemm", "64"),
        (128, "hip", "hip_gemm", "128"),
        (129, "hip", "hip_gemm", "256"),
        (4096, "cuda", "hip_gemm", "4096"),
        (5000, "hip", "hip_gemm", ">4096"),
    ],
)
def test_select(m, backend, kernel, bucket) -> None:  # type: ignore[no-untyped-def]
    d = dispatch.select(m, backend=backend, on_gpu=True, triton_ok=True, cuda_ext_available=True)
    assert (d.kernel, d.bucket, d.fallback) == (kernel, bucket, None)
    # hip_ok is this build's name for the same flag; either keyword may be given.
    assert dispatch.select(m, backend=backend, on_gpu=True, hip_ok=True) == d


def test_lookup_bucket_clamps_above_largest() -> None:
    assert dispatch.lookup_bucket(5000) == 4096
    assert dispatch.lookup_bucket(17) == 32


def test_select_without_gpu_is_the_reference_decision() -> None:
    """The reference's table (test_dispatch.py:75-80): a call that cannot run the compiled
    kernels is a ``torch_reference`` decision, with the reference's keyword call."""
    d = dispatch.select(8, backend="triton", on_gpu=False, triton_ok=False, cuda_ext_available=False)
    assert d.kernel == "torch_reference"
    assert dispatch.select(8, backend="hip", on_gpu=True, triton_ok=False).kernel == "torch_reference"
    assert dispatch.select(8, backend="hip", on_gpu=True, hip_ok=False).kernel == "torch_reference"
    # cuda_ext_available names the reference's separate CUDA GEMV extension; the HIP library is
    # this build's one compiled extension, so the flag never splits the decision.
    d = dispatch.select(2, backend="cuda", on_gpu=True, triton_ok=True, cuda_ext_available=False)
    assert (d.kernel, d.fallback) == ("hip_gemv", None)


def test_torch_reference_decision_raises_for_gpu_calls() -> None:
    """A GPU call never falls back: a torch_reference decision on GPU tensors (library missing,
    other GPU) is an error naming the library; host tensors take the ops' torch route before
    this check is reached, and asking it for them is an error that says so."""
    d = dispatch.select(8, backend="hip", on_gpu=False, triton_ok=False)
    with pytest.raises(dispatch.HipUnavailableError, match="host tensors"):
        dispatch.require_gpu_decision(d, on_gpu=False)
    d = dispatch.select(8, backend="hip", on_gpu=True, triton_ok=False)
    with pytest.raises(dispatch.HipUnavailableError, match="library"):
        dispatch.require_gpu_decision(d, on_gpu=True)
    dispatch.require_gpu_decision(dispatch.select(8, backend="hip", on_gpu=True, triton_ok=True), on_gpu=True)


def test_select_rejects_marlin_per_call() -> None:
    with pytest.raises(ValueError, match="per layer"):
        dispatch.select(1, backend="marlin", on_gpu=True, triton_ok=True, cuda_ext_available=True)


def test_record_counts_calls_and_layer_fallbacks() -> None:
    d = dispatch.select(2, backend="hip", on_gpu=True, triton_ok=True, cuda_ext_available=True)
    dispatch.record(d)
    dispatch.record(d)
    assert KERNEL_CALLS.value(kernel="hip_gemv", bucket="2") == 2
    dispatch.record_layer_fallback("unsupported_shape")
    assert FALLBACKS.value(reason="unsupported_shape") == 1
    dispatch.record(dispatch.Decision("hip_gemv", "4", fallback="cuda_ext_unavailable"))
    assert FALLBACKS.value(reason="cuda_ext_unavailable") == 1


def test_backend_from_env(monkeypatch: pytest.MonkeyPatch) -> None:
    monkeypatch.delenv(dispatch.BACKEND_ENV, raising=False)
    assert dispatch.backend_from_env() == "hip"
    monkeypatch.setenv(dispatch.BACKEND_ENV, " Marlin ")
    assert dispatch.backend_from_env() == "marlin"
    monkeypatch.setenv(dispatch.BACKEND_ENV, "Triton")
    assert dispatch.backend_from_env() == "triton"
    monkeypatch.setenv(dispatch.BACKEND_ENV, "cublas")
    with pytest.raises(ValueError, match="TOKENFORGE_BACKEND"):
        dispatch.backend_from_env()


SHAPES = [(1152, 896), (896, 4864), (37888, 3584), (3584, 18944), (4608, 3584), (200, 256)]


@pytest.mark.parametrize("group", [32, 64, 128])
@pytest.mark.parametrize("bucket", M_BUCKETS)
@pytest.mark.parametrize(("n", "k"), SHAPES)
def test_default_config_is_valid(bucket: int, n: int, k: int, group: int) -> None:
    cfg = default_config(bucket, n, k, group)
    cfg.validate(group)
    assert cfg.fits_bucket(bucket)
    assert cfg.family == family_for_bucket(bucket)
    if cfg.kernel == "gemm_mfma":
        assert cfg.split_k <= k // cfg.block_k


@pytest.mark.parametrize("group", [32, 64, 128])
@pytest.mark.parametrize("bucket", M_BUCKETS)
def test_candidates_are_valid(bucket: int, group: int) -> None:
    cands = candidate_configs(bucket, group)
    assert cands
    for cfg in cands:
        cfg.validate(group)
        assert cfg.fits_bucket(bucket)
    families = {c.family for c in cands}
    if bucket < GEMM_MIN_M:
        assert families == {"gemv"}
    elif bucket > GEMV_MAX_M:
        assert families == {"gemm"}
    else:  # the tuner weighs both families where both serve
        assert families == {"gemv", "gemm"}


def test_decode_buckets_offer_both_gemv_forms_and_work_splits() -> None:
    cands = candidate_configs(1, 128)
    assert {c.kernel for c in cands} == {"gemv_dot", "gemv_mfma"}
    # K split over the waves, columns split over the waves, or the stream form
    assert {c.block_k for c in cands} == {128, 256, 512}
    assert {c.kernel for c in candidate_configs(8, 128)} == {"gemv_mfma"}  # dot form: M <= 4
    assert {c.block_k for c in candidate_configs(8, 128)} == {128, 256, 512}
    # the stream form: block_m 4 for buckets up to 4, block_m 8 for the bucket of 8
    assert {c.block_m for c in candidate_configs(8, 128) if c.stream} == {8}
    assert {c.block_m for c in candidate_configs(4, 128) if c.stream} == {4}
    assert not any(c.stream for c in candidate_configs(16, 128))
    # the stream form is also tried with K split across workgroups; no other gemv kernel splits
    assert {c.split_k for c in candidate_configs(8, 128) if c.stream} == {1, 2, 4}
    assert {c.split_k for c in candidate_configs(8, 128) if not c.stream} == {1}
    GemmConfig("gemv_mfma", 8, 16, 512, 4, 16, 2).validate(128)
    assert {c.block_m for c in candidate_configs(4, 128) if c.kernel == "gemv_dot"} == {4}
    assert {c.block_m for c in candidate_configs(32, 128) if c.family == "gemv"} == {16, 32}


@pytest.mark.parametrize(
    ("kwargs", "match"),
    [
        ({"kernel": "gemv_triton", "block_m": 1, "block_n": 16, "block_k": 128}, "kernel"),
        ({"kernel": "gemv_mfma", "block_m": 48, "block_n": 16, "block_k": 128, "num_warps": 1, "num_stages": 1}, "compiled variant"),
        ({"kernel": "gemm_mfma", "block_m": 64, "block_n": 64, "block_k": 256}, "divide"),
        ({"kernel": "gemm_mfma", "block_m": 64, "block_n": 64, "block_k": 64, "split_k": 0}, "split_k"),
        ({"kernel": "gemv_mfma", "block_m": 16, "block_n": 16, "block_k": 128, "split_k": 2}, "split_k"),
        ({"kernel": "gemm_mfma", "block_m": 64, "block_n": 64, "block_k": 64, "num_warps": 3}, "num_warps"),
        ({"kernel": "gemm_mfma", "block_m": 64, "block_n": 64, "block_k": 64, "num_stages": 9}, "num_stages"),
    ],
)
def test_config_validation(kwargs: dict, match: str) -> None:
    with pytest.raises(ValueError, match=match):
        GemmConfig(**kwargs).validate(128)


def test_stream_form_rules() -> None:
    """The stream form serves buckets up to 4 (block_m 4) and the bucket of 8 (block_m 8); the
    heuristic default picks it where it applies under every epilogue and keeps the K-split GEMV
    elsewhere. The RMSNorm prologue runs on the block_m 4 form only."""
    from tokenforge.kernels.config import default_config, split_k_gemv_config, stream_form_applies

    s = GemmConfig("gemv_mfma", 4, 16, 512, 1, 8, 2)
    assert s.stream and s.family == "gemv"
    assert [b for b in M_BUCKETS if s.fits_bucket(b)] == [1, 2, 4]
    s8 = GemmConfig("gemv_mfma", 8, 16, 512, 1, 8, 2)
    assert s8.stream and [b for b in M_BUCKETS if s8.fits_bucket(b)] == [8]
    assert stream_form_applies(8, 37888, 3584, 8, max_m=8)
    assert stream_form_applies(5, 4608, 3584, 16, max_m=8)
    assert not stream_form_applies(8, 37888, 3584, 8, norm=True, max_m=8)  # the prologue: M <= 4
    assert not stream_form_applies(8, 3584, 18944, 8, max_m=8)  # x does not fit 96 KiB of LDS
    assert not stream_form_applies(9, 4608, 3584, 8, max_m=8)
    # K split across workgroups: each stages a slice of x (down_proj at M = 4 and 8)
    assert stream_form_applies(8, 3584, 18944, 16, max_m=8, split_k=4)
    assert stream_form_applies(4, 3584, 18944, 8, split_k=2)
    assert not stream_form_applies(8, 3584, 18944, 16, max_m=8, split_k=2)  # the slice does not fit
    assert not stream_form_applies(4, 4608, 3584, 8, split_k=4)  # 7 steps per slice for 8 waves
    assert not stream_form_applies(2, 4608, 3584, 8, norm=True, split_k=2)  # the prologue: no split
    assert stream_form_applies(2, 4608, 3584, 8, norm=True)
    # the op fuses the norm at M = 1 only, on the bucket's stream config with the ring at depth 4
    from tokenforge.kernels.config import norm_fused_config
    s1 = GemmConfig("gemv_mfma", 4, 16, 512, 1, 8, 2)
    assert norm_fused_config(s1, 1, 4608, 3584) == GemmConfig("gemv_mfma", 4, 16, 512, 1, 8, 4)
    assert norm_fused_config(GemmConfig("gemv_mfma", 4, 16, 512, 1, 16, 4), 1, 4608, 3584).num_stages == 4
    assert norm_fused_config(s1, 2, 4608, 3584) is None
    assert norm_fused_config(GemmConfig("gemv_mfma", 4, 16, 512, 2, 8, 2), 1, 4608, 3584) is None
    assert norm_fused_config(GemmConfig("gemv_mfma", 16, 16, 128, 1, 8, 2), 1, 4608, 3584) is None
    assert norm_fused_config(s1, 1, 4608, 12160) is None  # the prologue serves K <= 8192
    assert stream_form_applies(1, 37888, 3584, 8)
    assert stream_form_applies(2, 3584, 18944, 16)
    assert not stream_form_applies(4, 3584, 18944, 8)  # x does not fit 96 KiB of LDS
    assert not stream_form_applies(5, 4608, 3584, 8)
    assert not stream_form_applies(1, 48, 1024, 8)  # N % 32 == 16: SiLU*mul could not pair it
    assert not stream_form_applies(1, 200, 1024, 8)  # N % 16 == 8
    assert not stream_form_applies(1, 256, 1000, 1)  # K % 128 != 0
    assert not stream_form_applies(1, 256, 896, 8)  # 7 steps for 8 waves
    assert default_config(1, 37888, 3584, 128) == s
    assert default_config(4, 3584, 18944, 128) == split_k_gemv_config(3584, 18944)
    assert default_config(1, 200, 1024, 128) == split_k_gemv_config(200, 1024)
    assert not default_config(8, 4608, 3584, 128).stream


def test_config_from_dict_strict() -> None:
    good = GemmConfig("gemv_mfma", 16, 16, 128, 1, 1, 2).to_dict()
    assert GemmConfig.from_dict(good) == GemmConfig("gemv_mfma", 16, 16, 128, 1, 1, 2)
    with pytest.raises(ValueError, match="unknown"):
        GemmConfig.from_dict({**good, "block_q": 1})
    with pytest.raises(TypeError, match="integers"):
        GemmConfig.from_dict({**good, "split_k": True})
    with pytest.raises(TypeError, match="kernel"):
        GemmConfig.from_dict({**good, "kernel": 2})
    with pytest.raises(TypeError, match="object"):
        GemmConfig.from_dict([1, 2])


def test_variant_table_is_consistent() -> None:
    assert len(set(VARIANTS)) == len(VARIANTS)
    for kernel, bm, bn, bk, warps, stages in VARIANTS:
        GemmConfig(kernel, bm, bn, bk, 1, warps, stages).validate(128)
