# SPDX-License-Identifier: Apache-2.0
"""Make the GEMM solution table of the large-row prefill (kernels.prefill_gemm, library form).

The library form multiplies the rotated activations by the reconstructed weights with the process's BLAS
library (torch.matmul: an fp16 "NT" GEMM, (rows, k) x (n, k)^T). hipBLASLt's default heuristic does not pick
the fastest of its solutions for these shapes; PyTorch's TunableOp can time every hipBLASLt / rocBLAS
solution for a shape and record the fastest. This script does that for the 27B decoder's projection shapes
at a set of row counts and writes TunableOp's CSV table, which kernels.prefill_gemm then uses (tuning off)
when it is present:

    python omlx-exl3_amd/tune_gemm.py [--out omlx-exl3_amd/tuning/prefill_gemm_mi355x.csv] [--rows 512 4608]

It needs the GPU the table is for (MI355X) and the same PyTorch / ROCm / hipBLASLt versions: TunableOp
rejects a table whose version lines differ, and the prefill then uses the library's default solutions.
"""
from __future__ import annotations

import argparse
import os
import sys
import time

HERE = os.path.dirname(os.path.abspath(__file__))
DEFAULT_OUT = os.path.join(HERE, "tuning", "prefill_gemm_mi355x.csv")
# (k, n) of the 27B decoder's linear layers: q, k/v, o, gate/up, down
SHAPES = [(5120, 6144), (5120, 1024), (6144, 5120), (5120, 17408), (17408, 5120)]
ROWS = [16, 32, 48, 64, 96, 128, 256, 512, 1024, 2048, 4096, 4608]


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--out", default=DEFAULT_OUT)
    ap.add_argument("--rows", type=int, nargs="*", default=ROWS)
    ap.add_argument("--max-ms", type=int, default=30, help="tuning time per solution (ms)")
    args = ap.parse_args()

    import torch
    import torch.cuda.tunable as tunable

    if not torch.cuda.is_available():
        print("tune_gemm: no GPU", file=sys.stderr)
        return 1
    os.makedirs(os.path.dirname(os.path.abspath(args.out)), exist_ok=True)
    if os.path.exists(args.out):
        os.remove(args.out)
    tunable.set_filename(args.out, False)
    tunable.set_max_tuning_duration(args.max_ms)
    tunable.tuning_enable(True)
    tunable.enable(True)
    for rows in args.rows:
        for k, n in SHAPES:
            x = torch.randn(rows, k, dtype=torch.float16, device="cuda")
            wt = torch.randn(n, k, dtype=torch.float16, device="cuda") * 0.01
            t0 = time.time()
            torch.matmul(x, wt.t())
            torch.cuda.synchronize()
            print(f"tuned rows {rows:5d} k {k:5d} n {n:5d} in {time.time() - t0:5.1f} s", flush=True)
            del x, wt
    # TunableOp writes the table when the process ends (it is enabled, tuning is on and it holds new results)
    print(f"table: {args.out} (written at exit)", flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
