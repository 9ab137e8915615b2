"""The tuner's fill split (config.fill_split): the K split that ends an LDS-tile GEMM launch in
the fewest K blocks per CU over whole rounds of workgroups, capped so that the fp32 partials
stay no larger than the packed weights; added to the tuner's candidates next to its
power-of-two splits."""

from __future__ import annotations

from tokenforge.kernels.config import GemmConfig, candidate_configs, fill_split, fill_split_candidates


def _brute(cfg: GemmConfig, m: int, n: int, k: int, cus: int) -> int:
    tiles = -(-m // cfg.block_m) * -(-n // cfg.block_n)
    blocks = k // cfg.block_k
    limit = max(1, min(16, blocks, k // (8 * m)))
    costs = {s: -(-tiles * s // cus) * -(-blocks // s) for s in range(1, limit + 1)}
    return min(costs, key=lambda s: (costs[s], s))


def test_known_shapes() -> None:
    down = GemmConfig("gemm_mfma", 256, 128, 64, 1, 8, 3)
    # 28 tiles x 296 blocks: split 9 gives 252 workgroups of 33 blocks (split 8: 37 blocks).
    assert fill_split(down, 256, 3584, 18944) == 9
    # gate_up 256 x 192 at M = 256: 198 tiles in one round; a split would add more partial
    # bytes than the weights (K / (8 M) < 2).
    assert fill_split(GemmConfig("gemm_mfma", 256, 192, 64, 1, 8, 3), 256, 37888, 3584) == 1
    # down at M = 1024: the cap K / (8 M) = 2.
    assert fill_split(GemmConfig("gemm_mfma", 256, 256, 64, 1, 8, 3), 1024, 3584, 18944) <= 2


def test_matches_brute_force() -> None:
    for bm, bn in ((64, 64), (128, 128), (256, 128), (256, 192), (128, 256)):
        cfg = GemmConfig("gemm_mfma", bm, bn, 64, 1, 8 if bm == 256 else 4, 3 if bm == 256 else 4)
        for m in (16, 64, 128, 256, 512, 1024):
            for n, k in ((4608, 3584), (3584, 3584), (37888, 3584), (3584, 18944)):
                for cus in (80, 256, 304):
                    assert fill_split(cfg, m, n, k, cus) == _brute(cfg, m, n, k, cus)


def test_candidates_add_only_new_splits_of_lds_tile_gemms() -> None:
    cands = candidate_configs(256, 128)
    extra = fill_split_candidates(cands, 256, 3584, 18944)
    have = {(c.kernel, c.block_m, c.block_n, c.block_k, c.num_warps, c.num_stages, c.split_k) for c in cands}
    assert extra, "down_proj at M = 256 has a fill split outside 1, 2, 4, 8"
    for c in extra:
        assert c.kernel == "gemm_mfma" and not c.skinny
        assert (c.kernel, c.block_m, c.block_n, c.block_k, c.num_warps, c.num_stages, c.split_k) not in have
        c.validate(128)
    assert GemmConfig("gemm_mfma", 256, 128, 64, 9, 8, 3) in extra
    assert fill_split_candidates(candidate_configs(256, 128), 256, 37888, 3584) == []
