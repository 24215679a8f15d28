"""The target: one AMD Instinct MI355X (gfx950, CDNA4). Replaces the reference's chip module
(src/autokernel/v5e.py:28-80), whose VMEM/SMEM budgets and (8, 128) layout rules have no meaning here.

What the lowering plans against: 256 compute units in 8 XCDs (accelerator complex dies, each with its own
4 MiB L2), 160 KiB of LDS per CU, 64-wide wavefronts, 512 VGPRs + AGPRs per lane, bf16 MFMA shapes
32x32x16 and 16x16x32, 288 GB of HBM3E at ~8 TB/s. Peaks are the published dense figures.
"""

from __future__ import annotations

ARCH = "gfx950"
DEVICE_NAME = "AMD Instinct MI355X"
CUS = 256
XCDS = 8
WAVE = 64
LDS_BYTES = 160 * 1024  # per CU
LDS_BUDGET = 160 * 1024  # what one workgroup of a kernel may take
HBM_BYTES = 288 * 10**9

PEAK_BF16_FLOPS = 2.5e15  # dense MFMA
PEAK_FP32_FLOPS = 157.3e12
PEAK_HBM_BYTES_PER_S = 8.0e12

# bf16 MFMA instruction shapes (M, N, K) the lowering uses.
MFMA_32x32x16 = (32, 32, 16)
MFMA_16x16x32 = (16, 16, 32)

# Index arrays and step tables live in device memory read through the scalar cache; a kernel keeps the
# tables it walks below this many bytes (the reference's SMEM budget played this role: v5e.py).
TABLE_BUDGET = 64 * 2**20


def padded_bytes(shape, itemsize: int) -> int:
    n = itemsize
    for s in shape:
        n *= int(s)
    return n
