"""The vendor library's bf16 GEMM on the prompt GEMMs' shapes, timed for
comparison only: nothing on the product path calls it.

The 1600-token ingest runs five GEMM shapes (M = 1600 prompt rows): gate/up
(N = 2 x 12288, K = 4096), down (N = 4096, K = 12288), the GDN in_proj
(N = 12352 = q/k/v 8192 + z 4096 + a 32 + b 32, K = 4096), the attention
q/k/v (N = 10240, K = 4096) and out_proj / o_proj (N = 4096, K = 4096).
Each is timed through `torch.mm` (hipBLASLt on ROCm) on plain bf16 operands
-- no Q4 dequantisation and no fused epilogue -- in the two weight layouts a
caller can hand it: W[N, K] (rows of K, the layout the prompt GEMM reads) as
C[N, M] = W @ x^T, and W[K, N] as C[M, N] = x @ W. Every operand is
contiguous (no transposed views). Times are CUDA-event means over 20 calls
after 5 warm calls.

    python -m peregrine_amd.gemm_baseline
"""
from __future__ import annotations

import json

SHAPES = [("gate_up", 1600, 24576, 4096), ("down", 1600, 4096, 12288), ("in_proj", 1600, 12352, 4096),
          ("attn_qkv", 1600, 10240, 4096), ("out_proj", 1600, 4096, 4096)]


def _time_us(torch, fn, warm: int = 5, reps: int = 20) -> float:
    for _ in range(warm):
        fn()
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(reps):
        fn()
    end.record()
    torch.cuda.synchronize()
    return start.elapsed_time(end) / reps * 1e3


def library_gemms() -> list[dict]:
    import torch

    if not torch.cuda.is_available():
        raise RuntimeError("the library GEMM baseline needs a GPU")
    torch.manual_seed(0)
    rows = []
    for name, M, N, K in SHAPES:
        flop = 2.0 * M * N * K
        w_nk = torch.randn(N, K, device="cuda", dtype=torch.bfloat16) * 0.02
        x_t = torch.randn(K, M, device="cuda", dtype=torch.bfloat16)
        us_nk = _time_us(torch, lambda: torch.mm(w_nk, x_t))
        del w_nk, x_t
        x = torch.randn(M, K, device="cuda", dtype=torch.bfloat16)
        w_kn = torch.randn(K, N, device="cuda", dtype=torch.bfloat16) * 0.02
        us_kn = _time_us(torch, lambda: torch.mm(x, w_kn))
        del x, w_kn
        rows.append({"gemm": name, "M": M, "N": N, "K": K,
                     "us_w_nk": round(us_nk, 1), "tflops_w_nk": round(flop / us_nk / 1e6, 1),
                     "us_w_kn": round(us_kn, 1), "tflops_w_kn": round(flop / us_kn / 1e6, 1)})
    return rows


def main() -> int:
    for r in library_gemms():
        print(json.dumps(r), flush=True)
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
