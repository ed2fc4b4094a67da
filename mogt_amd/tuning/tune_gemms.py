"""Regenerate the GEMM table of mogt_amd.gemm_tuning on the GPU it is for.

    python -m mogt_amd.tuning.tune_gemms [output.csv]

Runs the backbone benchmarks' forward and training steps (bench.py's
measure_backbone / measure_backbone_train: 4 layers with FFN 3072 and 2 layers
with the reference FFN, L = 8192 / 16384 / 32768) once each with TunableOp
tuning on, which times every hipBLASLt / rocBLAS solution per GEMM shape and
writes the fastest to the table.
"""
from __future__ import annotations

import sys
import time
from pathlib import Path

import torch

ROOT = Path(__file__).resolve().parents[2]


def main(out: str) -> None:
    sys.path.insert(0, str(ROOT))
    import bench

    torch.cuda.tunable.enable(True)
    torch.cuda.tunable.tuning_enable(True)
    torch.cuda.tunable.set_filename(out)
    torch.cuda.tunable.set_max_tuning_duration(30)
    torch.cuda.tunable.set_max_tuning_iterations(20)
    for L in (8192, 16384, 32768):
        for layers, ffn, vocab in ((4, 3072, 32000), (2, None, 4096)):
            t0 = time.time()
            bench.measure_backbone(torch, layers, ffn, vocab, L, 1, 1)
            bench.measure_backbone_train(torch, layers, ffn, vocab, L, 1, 1, fused=True)
            print(f"tuned L={L} layers={layers}: {time.time() - t0:.1f} s, "
                  f"{len(torch.cuda.tunable.get_results())} shapes", flush=True)
    # TunableOp writes the table when the process ends


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else str(ROOT / "mogt_amd" / "tuning" / "gemm_gfx950.csv"))
