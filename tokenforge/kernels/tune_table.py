"""Make the autotune table shipped for one GPU (``tokenforge/kernels/tuned/<gpu>-hip<abi>.json``).

    python -m tokenforge.kernels.tune_table [--out DIR] [--shape NxK ...] [--buckets 1,2,4,...] [--update]

Tunes every M bucket of every layer shape (by default the four Qwen2.5-7B decoder linears,
group 128) on the current GPU from an empty cache, then writes the cache document, which has
the cache's own format and checks, into ``--out`` (default: the package's ``tuned/``). With
``--update`` the entries tuned here replace theirs in the table already in ``--out`` and the
other entries stay (for retuning some shapes or buckets). The hot path's lookup reads a
user's cache first, then this table, then the heuristic default. Run on the GPU the table is
for; the file name carries that GPU's identity and the kernel ABI.
"""

from __future__ import annotations

import argparse
import os
import shutil
import sys
import tempfile
import time
from pathlib import Path

QWEN25_7B = ((4608, 3584), (3584, 3584), (37888, 3584), (3584, 18944))


def main(argv: list[str] | None = None) -> int:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--out", type=Path, default=Path(__file__).resolve().parent / "tuned")
    ap.add_argument("--shape", action="append", default=None, metavar="NxK")
    ap.add_argument("--buckets", type=str, default=None, help="comma-separated M buckets (default: all)")
    ap.add_argument("--group-size", type=int, default=128)
    ap.add_argument("--update", action="store_true", help="merge into the table already in --out")
    args = ap.parse_args(argv)

    import torch

    from tokenforge.kernels import autotune
    from tokenforge.kernels.config import M_BUCKETS
    from tokenforge.kernels.device import gpu_identity

    if not torch.cuda.is_available():
        print("tune_table needs the GPU the table is for", file=sys.stderr)
        return 1
    shapes = QWEN25_7B if not args.shape else tuple(tuple(int(v) for v in s.lower().split("x")) for s in args.shape)
    buckets = M_BUCKETS if not args.buckets else tuple(int(b) for b in args.buckets.split(","))
    dev = torch.device("cuda:0")
    gpu = gpu_identity(dev)
    with tempfile.TemporaryDirectory() as tmp:
        os.environ[autotune.CACHE_DIR_ENV] = tmp  # start from an empty cache
        for n, k in shapes:
            for bucket in buckets:
                t0 = time.perf_counter()
                won = autotune.tune_layer(n, k, args.group_size, device=dev, gpu=gpu, buckets=(bucket,))
                print(f"{n}x{k} M={bucket}: {won[bucket]} ({time.perf_counter() - t0:.1f}s)",
                      file=sys.stderr, flush=True)
        abi = autotune.hip_abi()
        src = autotune.cache_path(gpu, abi)
        args.out.mkdir(parents=True, exist_ok=True)
        dst = args.out / src.name
        if args.update and dst.exists():
            table = autotune._decode_document(dst.read_text(encoding="utf-8"), gpu, abi)
            table.update(autotune._decode_document(src.read_text(encoding="utf-8"), gpu, abi))
            autotune._replace_file(dst, autotune._encode_document(gpu, abi, table))
        else:
            shutil.copyfile(src, dst)
    print(dst)
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
