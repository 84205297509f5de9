"""Synthetic inputs for the benchmark configurations of the HSTU attention path (1-5 from the
baseline; 6 = configuration 2 with the reference's semi-local mask, 256 local + 256 full tail;
7 = 16 sequences of 4,096 history tokens, the kernel's steady state: two workgroups on every CU
from the start of the launch to its end).

Sequence lengths come from ``numpy.random.Generator(PCG64(seed))``; q, k, v (and the relative
attention bias) from ``torch.Generator().manual_seed(seed)`` on the CPU in the order q, k, v, rab.
Tensors are always generated on the CPU and copied to the device, never drawn from a device RNG,
so that the oracle, the CPU baseline and the kernel see identical values.
"""
from __future__ import annotations

from dataclasses import dataclass, field
from typing import Optional

import numpy as np
import torch


@dataclass
class Workload:
    name: str
    q: torch.Tensor  # [T,H,Dqk] float32 master copy (already rounded to `dtype` where that is bf16 or fp16)
    k: torch.Tensor
    v: torch.Tensor
    seq_offsets: torch.Tensor  # [B+1] int64
    num_targets: torch.Tensor  # [B] int64
    max_seq_len: int
    alpha: float
    dtype: str  # "fp32" | "bf16" | "fp16" | "fp8"
    contextual_seq_len: int = 0
    rab: Optional[torch.Tensor] = None  # [H, 2*max_seq_len-1] float32
    lengths: np.ndarray = field(default=None)  # [B] full sequence lengths (history + targets)
    max_attn_len: int = 0    # > 0: semi-local window over the history
    full_attn_size: int = 0  # > 0 (with max_attn_len > 0): the last rows keep full causal attention
    mask_type: str = "lower_triangular"  # any other string: the reference's mask on absolute distances

    @property
    def T(self) -> int:
        return int(self.q.shape[0])

    @property
    def B(self) -> int:
        return int(self.num_targets.shape[0])

    @property
    def H(self) -> int:
        return int(self.q.shape[1])

    def pairs(self) -> int:
        """Unmasked (query, key) pairs.  Causal mask: h(h+1)/2 + t(h+1) + c(c-1)/2 per sequence; in
        general, per query row: the diagonal, the visible history keys (all keys below the row's
        target-clamped position, or the last ``max_attn_len`` of them unless the row is in the
        full-attention tail) and the contextual keys not counted yet."""
        total = 0
        c = self.contextual_seq_len
        A, F = self.max_attn_len, self.full_attn_size
        for n, t in zip(self.lengths.tolist(), self.num_targets.tolist()):
            if n <= 0:
                continue
            cap = min(max(n - t, -1), n)
            m = np.arange(n, dtype=np.int64)
            idm = np.minimum(m, cap)
            pos = np.maximum(idm, 0)
            if A > 0:
                tail = (idm >= cap - F) if F > 0 else np.zeros(n, dtype=bool)
                lo = np.where(tail, 0, np.maximum(pos - A, 0))
            else:
                lo = np.zeros(n, dtype=np.int64)
            hist = pos - lo
            total += int(n + hist.sum())
            ce = min(c, n) if c > 0 else 0
            if ce > 0:
                in_ctx = np.maximum(np.minimum(pos, ce) - np.minimum(lo, ce), 0) + (m < ce)
                total += int((ce - in_ctx).sum())
        return total

    def flops(self) -> int:
        """Two contractions over the unmasked pairs; SiLU, mask and bias are not counted."""
        return self.H * (2 * self.q.shape[2] + 2 * self.v.shape[2]) * self.pairs()

    def algorithmic_bytes(self) -> int:
        """q, k, v read once and out written once, plus offsets, targets and the bias table."""
        T, H, Dqk = self.q.shape
        Dv = self.v.shape[2]
        qk_size = {"fp32": 4, "bf16": 2, "fp16": 2, "fp8": 1}[self.dtype]
        v_size = 4 if self.dtype == "fp32" else 2
        b = 2 * Dqk * H * T * qk_size + 2 * Dv * H * T * v_size
        b += 8 * (self.B + 1) + 8 * self.B
        if self.rab is not None:
            b += 4 * self.rab.numel()
        return b


def history_lengths(config: int, seed: int = 0) -> np.ndarray:
    rng = np.random.Generator(np.random.PCG64(seed))
    if config == 1:
        return np.full((4,), 16, dtype=np.int64)
    if config in (2, 3, 5, 6, 8, 9, 10):
        return rng.integers(256, 1985, size=32).astype(np.int64)
    if config == 4:
        return np.clip(rng.zipf(1.2, size=8), 128, 8064).astype(np.int64)
    if config == 7:
        return np.full((16,), 4096, dtype=np.int64)
    raise ValueError(f"unknown config {config}")


_SPEC = {
    # config: (num_targets, max_seq_len, H, D, dtype, alpha)
    1: (4, 20, 2, 32, "fp32", 1.0 / 32),
    2: (64, 2048, 4, 128, "bf16", 1.0 / 128),
    3: (64, 2048, 4, 128, "bf16", 1.0 / 128),
    4: (128, 8192, 4, 128, "bf16", 1.0 / 128),
    5: (64, 2048, 4, 128, "fp8", 1.0 / 128),
    6: (64, 2048, 4, 128, "bf16", 1.0 / 128),  # config 2 with the semi-local mask (256 local, 256 full tail)
    7: (0, 4096, 4, 128, "bf16", 1.0 / 128),   # steady state of the tiled kernel: 16 x 4,096, no targets
    8: (64, 2048, 8, 64, "bf16", 1.0 / 64),    # config 2's sequences at head dim 64, 8 heads (general MFMA kernels)
    9: (64, 2048, 4, 128, "fp16", 1.0 / 128),  # config 2 in fp16 (general MFMA kernels)
    10: (64, 2048, 8, 50, "bf16", 1.0 / 50),   # config 8 at head dim 50: rows of 100 bytes (general MFMA kernels for rows aligned to the element only)
}


def make_jagged(lengths, num_targets, H, Dqk, Dv, *, max_seq_len, alpha, dtype="fp32", seed=0,
                contextual_seq_len=0, with_rab=False, rab_std=0.02, tail_rows=0, name="custom",
                max_attn_len=0, full_attn_size=0, mask_type="lower_triangular"):
    """Build a workload from explicit full lengths (history + targets) and target counts."""
    lengths = np.asarray(lengths, dtype=np.int64)
    T = int(lengths.sum()) + int(tail_rows)
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(T, H, Dqk, generator=g)
    k = torch.randn(T, H, Dqk, generator=g)
    v = torch.randn(T, H, Dv, generator=g)
    rab = None
    if with_rab:
        rab = torch.randn(H, 2 * max_seq_len - 1, generator=g) * rab_std
    if dtype in ("bf16", "fp8"):
        q = q.bfloat16().float()
        k = k.bfloat16().float()
        v = v.bfloat16().float()
    if dtype == "fp16":
        q = q.half().float()
        k = k.half().float()
        v = v.half().float()
    off = np.concatenate([[0], np.cumsum(lengths)]).astype(np.int64)
    return Workload(name=name, q=q, k=k, v=v, seq_offsets=torch.from_numpy(off),
                    num_targets=torch.as_tensor(np.asarray(num_targets, dtype=np.int64)),
                    max_seq_len=int(max_seq_len), alpha=float(alpha), dtype=dtype,
                    contextual_seq_len=int(contextual_seq_len), rab=rab, lengths=lengths,
                    max_attn_len=int(max_attn_len), full_attn_size=int(full_attn_size), mask_type=str(mask_type))


def make_config(config: int, seed: int = 0) -> Workload:
    t, N, H, D, dtype, alpha = _SPEC[config]
    hist = history_lengths(config, seed)
    lengths = hist + t
    return make_jagged(lengths, np.full_like(hist, t), H, D, D, max_seq_len=N, alpha=alpha,
                       dtype=dtype, seed=seed, contextual_seq_len=8 if config == 3 else 0,
                       with_rab=(config == 3), name=f"config{config}",
                       max_attn_len=256 if config == 6 else 0, full_attn_size=256 if config == 6 else 0)
