"""The `nvfp4` encoded linear on gfx950: cozyq's counterpart of cozy-runtime's
`internal/nvfp4_linear.py`.

* **W4A16 GEMV, up to `GEMV_ROWS` rows** (`internal/nvfp4_linear.py:367-375`, which stops at
  `DECODE_ROWS`): the packed E2M1 codes and E4M3 block scales are decoded in registers onto the
  bf16/fp16 MFMA (`cozyq_nvfp4_gemv`), reading 0.56 bytes a weight, each decoded weight fed to
  one MFMA per 16 activation rows.
* **More rows** (`:376-385`): the weight is decoded once per 128-row chunk into the activation
  dtype with the second level folded in (`cozyq_decode`, the reference's `_dequant`), and the
  library GEMM multiplies it (`torch.nn.functional.linear`, hipBLASLt), as the reference's
  cuBLAS call does. The one-launch W4A16 GEMM (`cozyq_nvfp4_gemm`, W decoded exactly on the
  way to the MFMA, no transient) takes these rows when `gemm=True` is asked for: it is measured
  slower than decode + hipBLASLt at every shape tried, so it is not the default.

Activations stay 16-bit here, as in the reference's nvfp4 leaf. The W4A4 form, where the
activation is quantized to nvfp4 too, is svdq.nvfp4's (`cozyq.svdq_linear`): it decodes both
operands exactly to fp16 on the way to the MFMA. There is no eager lane: operands off the GPU
raise.
"""

from __future__ import annotations

from collections.abc import Callable
from typing import Any

from cozyq import decode as dec

Tensor = Any
Dtype = Any

#: The reference's GEMV limit (`internal/nvfp4_linear.py:60`).
DECODE_ROWS = 16
#: Up to this many rows the GEMV serves: the weight is read once, 0.56 bytes a weight. Measured
#: against decode + hipBLASLt on three weights (3072², 12288x3072, 14336x4096): 1.9-5.7x faster
#: at every M up to 64.
GEMV_ROWS = 64
#: The K multiple of the nvfp4 GEMM (one 64-element step); other shapes decode and call the
#: library GEMM.
GEMM_K = 64
#: The decode transient per row chunk (`internal/nvfp4_linear.py:54-55`).
_DECODE_CHUNK = 256 << 20
NVFP4_BLOCK = 16


def matmul(torch: Any, x: Tensor, weight: Tensor, blocked_scale: Tensor,
           linear_scale: Callable[[], Tensor] | None, scale_2: Tensor, out_dtype: Dtype,
           gemm: bool = False) -> Tensor:  # fmt: skip
    """`x @ W.T` for one stored nvfp4 weight (`internal/nvfp4_linear.py:338-403`): `weight` u8
    [N, K/2] (element 2k low), `blocked_scale` its E4M3 block scales in cuBLAS's 128x4 tiles as
    [rows padded to 128, K/16 padded to 4], `scale_2` the float32 [1] second level.
    `linear_scale` (the reference's eager path's row-major scales) is not used here. `gemm`
    takes rows past `GEMV_ROWS` through the one-launch W4A16 GEMM where its shape rule holds."""
    from cozyq.prebuilt import library

    rows_out, cols = int(weight.shape[0]), 2 * int(weight.shape[1])
    if not x.is_cuda or x.dtype not in (torch.bfloat16, torch.float16):
        raise ValueError(f"nvfp4 linear: bf16/fp16 activations on the GPU, not {x.dtype} on {x.device}")
    flat = x.reshape(-1, cols).contiguous()
    rows = int(flat.shape[0])
    ops = library(x.device.index or 0)
    weight = weight.view(torch.uint8)
    scales = blocked_scale.view(torch.uint8)
    second = scale_2.to(torch.float32).reshape(1)
    if rows <= GEMV_ROWS:
        out = ops.nvfp4_gemv(flat, weight, scales, second, x.dtype)
        return out.to(out_dtype).reshape(*x.shape[:-1], rows_out)
    if gemm and cols % GEMM_K == 0 and rows_out % 8 == 0:
        out = ops.nvfp4_gemm(flat, weight, scales, second, None, x.dtype)
        return out.to(out_dtype).reshape(*x.shape[:-1], rows_out)
    # 128-row chunks (whole scale tiles) bound the decoded transient.
    step = max(128, _DECODE_CHUNK // (2 * cols) // 128 * 128)
    parts = []
    for i in range(0, rows_out, step):
        n = min(step, rows_out - i)
        tiles = scales[i : i + -(-n // 128) * 128]  # the chunk's whole 128-row tiles
        decoded = torch.empty(n, cols, dtype=x.dtype, device=x.device)
        ops.decode_table(dec._CODE["u8"], weight[i : i + n], tiles, dec._NUM["f8_e4m3fn"], decoded,
                         n, cols, grid=dec.GRID_BLOCKS, block=NVFP4_BLOCK, tiled=True,
                         scale_2=second)  # fmt: skip
        parts.append(torch.nn.functional.linear(flat, decoded))
    out = parts[0] if len(parts) == 1 else torch.cat(parts, dim=-1)
    return out.to(out_dtype).reshape(*x.shape[:-1], rows_out)
