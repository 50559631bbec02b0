"""Writes the committed fixtures of tests/golden/.

  e4m3_of_bf16.npy  torch's float8_e4m3fn cast of every bf16 bit pattern (uint8[65536]): the
                    library routine the reference's casts use (engine/kernels/fp8.py:22, :56).
  small_cases.npz   a seeded small case (x [4,256], W [32,256] bf16 bits) with the oracle's
                    per-token / per-channel quantization and FP8 product (device scale
                    arithmetic), as a regression fixture for the oracle and the GPU tests.

Run from the repository root: python tests/golden/make_golden.py
"""

import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

from oracle import oracle as O  # noqa: E402


def main():
    bits = np.arange(65536, dtype=np.uint16)
    f = torch.from_numpy(bits.view(np.int16).copy()).view(torch.bfloat16).float()
    np.save(os.path.join(HERE, "e4m3_of_bf16.npy"), f.to(torch.float8_e4m3fn).view(torch.uint8).numpy())

    g = torch.Generator().manual_seed(123)
    x = torch.randn(4, 256, generator=g).to(torch.bfloat16)
    w = (torch.randn(32, 256, generator=g) * 0.02).to(torch.bfloat16)
    xb = x.view(torch.int16).numpy().view(np.uint16)
    wb = w.view(torch.int16).numpy().view(np.uint16)
    x8, xs = O.quant_rows(xb)
    w8, ws = O.quantize(wb)
    _, y = O.fp8_matmul(x8, xs, w8, ws)
    np.savez(os.path.join(HERE, "small_cases.npz"), x=xb, w=wb, x8=x8, xs=xs, w8=w8, ws=ws,
             y_bf16=O.f32_to_bf16(y.astype(np.float32)))


if __name__ == "__main__":
    main()
