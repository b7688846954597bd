"""Quantized projection modules: the module-swap boundary of the INT4-G32 path.

The reference installs quantized projections by registering packed buffers and flags on
the fused attention/MLP modules and branching on them in ``_attention``/``_mlp``
(``src/moss_tts/_runtime/calibrated_backend.py:41-54``, ``src/moss_tts/_runtime/llm.py:26-130``).
Here each quantized projection is an explicit ``nn.Module`` holding its row-packed weight
as buffers; ``forward`` picks the decode GEMV for one row, the prefill GEMM for more.
"""
from __future__ import annotations

import torch
from torch import nn

from . import bf16, w4g32
from .w4g32 import PackedW4G32, _require


class QuantLinearG32(nn.Module):
    """``y = x @ dequant(W)^T`` with W INT4, 32-input groups, bf16 activations and outputs.

    Replaces a bf16 ``nn.Linear(in_features=K, out_features=N, bias=False)``; the fused
    q||k||v (N=6144) and the O/down projections of the Qwen3-8B backbone use it
    (``src/moss_tts/_runtime/llm.py:140-144``).
    """

    def __init__(self, packed: PackedW4G32, *, dequant: int = w4g32.EXACT):
        super().__init__()
        self.in_features = packed.K
        self.out_features = packed.N
        self.dequant = dequant
        self.register_buffer("qw", packed.qw, persistent=True)
        self.register_buffer("scales", packed.scales, persistent=True)
        self.register_buffer("zeros", packed.zeros, persistent=True)

    @property
    def packed(self) -> PackedW4G32:
        return PackedW4G32(self.qw, self.scales, self.zeros)

    @classmethod
    def from_float(cls, weight: torch.Tensor, *, symmetric: bool = False, **kw) -> "QuantLinearG32":
        """Quantize a float weight ``[N, K]`` on its device: min-max RTN, or with ``symmetric`` the
        reference's static absmax/7 scales and round-to-nearest codes in [-7, 7]
        (``src/moss_tts/_runtime/calibrated_quant.py:36-38,74-77``)."""
        _require(weight.is_cuda and weight.ndim == 2, "a 2-D device weight [out, in] is required")
        w = weight.detach().float().contiguous()
        return cls(w4g32.quantize_symmetric(w) if symmetric else w4g32.quantize_minmax(w), **kw)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        _require(x.shape[-1] == self.in_features, f"expected {self.in_features} input features")
        rows = x.numel() // self.in_features
        if rows == 1:
            return w4g32.gemv(x.contiguous(), self.packed, dequant=self.dequant)
        return w4g32.gemm(x.contiguous(), self.packed)

    def extra_repr(self) -> str:
        return f"in_features={self.in_features}, out_features={self.out_features}, group=32"


class QuantGateUpG32(QuantLinearG32):
    """Fused gate||up projection (gate rows first) followed by ``bf16(silu(g)) * u``; the
    output has ``out_features // 2`` columns (``src/moss_tts/_runtime/llm.py:144``,
    epilogue ``src/moss_tts/_runtime/dp4a_scaled.py:64-68``)."""

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        _require(x.shape[-1] == self.in_features, f"expected {self.in_features} input features")
        rows = x.numel() // self.in_features
        if rows == 1:
            return w4g32.gateup_silu(x.contiguous(), self.packed, dequant=self.dequant)
        from . import pointwise

        return pointwise.silu_mul(w4g32.gemm(x.contiguous(), self.packed))


class Bf16Linear(nn.Module):
    """bf16 weight ``[N, K]`` applied to one row with the bf16 decode GEMV (fp32 accumulate): the
    reference's bf16 output heads (``src/moss_tts/_runtime/llm.py:188-191,270-279``).  The weight is
    held as given (a contiguous buffer, no copy)."""

    def __init__(self, weight: torch.Tensor):
        super().__init__()
        _require(isinstance(weight, torch.Tensor) and weight.ndim == 2 and weight.dtype == torch.bfloat16,
                 "a 2-D bf16 weight [out, in] is required")
        self.in_features = weight.shape[1]
        self.out_features = weight.shape[0]
        self.register_buffer("weight", weight.detach().contiguous(), persistent=True)

    @property
    def nbytes(self) -> int:
        return self.weight.numel() * self.weight.element_size()

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        _require(x.shape[-1] == self.in_features, f"expected {self.in_features} input features")
        _require(x.numel() == self.in_features, "the bf16 heads run on one row (the decode step's last token)")
        return bf16.gemv(x.contiguous(), self.weight)

    def extra_repr(self) -> str:
        return f"in_features={self.in_features}, out_features={self.out_features}, dtype=bf16"
