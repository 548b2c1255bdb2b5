"""The library's fp32 -> 16-bit conversions (hk_to_lp_host; the kernels use
the same routine) against torch's casts, which CastLinear applies to its
weights, biases, inputs and outputs (example_model.py:82-95): round to
nearest even, fp16 overflow to infinity, subnormals, signed zeros, NaN."""

import numpy as np
import pytest
import torch

from hackathon_amd import weights

FMT = {"bf16": torch.bfloat16, "fp16": torch.float16}


def _values():
    rng = np.random.default_rng(0)
    parts = [rng.standard_normal(200_000).astype(np.float32) * s
             for s in (1e-7, 1e-5, 1e-3, 1.0, 300.0, 3e4, 7e4, 1e30)]
    # every 65537th fp32 bit pattern (all exponents, mantissa patterns)
    parts.append(np.arange(0, 2 ** 32, 65537, dtype=np.uint64).astype(np.uint32).view(np.float32))
    # ties and boundaries: fp16 max 65504, the overflow tie 65520, the
    # smallest subnormal 2^-24 and its half 2^-25 (a tie to zero), bf16 ties
    edge = [65504.0, 65519.996, 65520.0, -65520.0, 65536.0, 2.0 ** -24, 2.0 ** -25,
            3 * 2.0 ** -25, 2.0 ** -14, 6.0975552e-05, 1.0 + 2.0 ** -11, 1.0 + 3 * 2.0 ** -11,
            1.0 + 2.0 ** -8, 1.0 + 3 * 2.0 ** -8, 0.0, -0.0, np.inf, -np.inf,
            3.3895314e38, -3.3895314e38]
    parts.append(np.asarray(edge, dtype=np.float32))
    return np.concatenate(parts)


@pytest.mark.parametrize("fmt", ["bf16", "fp16"])
def test_to_lp_matches_torch_cast(fmt):
    x = torch.from_numpy(_values())
    got = weights.to_lp_bits(x, fmt)
    want = x.to(FMT[fmt]).view(torch.int16)
    finite = ~torch.isnan(x)
    assert torch.equal(got[finite], want[finite])
    # NaN stays NaN
    nan_in = torch.tensor([float("nan")])
    assert torch.isnan(weights.to_lp_bits(nan_in, fmt).view(FMT[fmt]).float()).all()
