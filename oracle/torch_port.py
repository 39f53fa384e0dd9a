"""torch_port.py -- torch restatement of the reference Viterbi (TEST INFRASTRUCTURE).

This is the timed CPU baseline reported beside the GPU numbers (kind "port")
and a second, independently written check of the C oracle.  It performs the
same tensor operations in the same step order as the reference's torch path
(quantize.py:218-320 viterbi with emit_mode="sq", quantize.py:323-354
quantize_seq_tailbite), batched over sequences, on the device X lives on: on
the CPU it is the reference's own CPU path; on the GPU the same elementwise
fp32 operations (no contraction across separate tensor ops) and torch's
min(dim)/argmin, whose first-index tie rule a test pins against the C oracle,
make it a full-scale checker of every tile.  Only tests/, the smoke check and
bench.py's CPU-baseline and bit-exact legs may import it.
"""
from __future__ import annotations

import torch


def viterbi(X: torch.Tensor, lut: torch.Tensor, K: int, L: int,
            overlap: torch.Tensor | None = None,
            back_from: int | None = None) -> torch.Tensor:
    """X [T, B] fp32 -> states [T, B] int64, or [B] when back_from is set."""
    T, B = X.shape
    S, NC, SP = 1 << L, 1 << K, 1 << (L - K)
    dev = X.device
    X = X.float()
    LUT = lut.float().to(dev).view(1, S)
    INF = float("inf")

    def emit(i):
        return (LUT - X[i].unsqueeze(-1)).square()          # [B, S]

    cost = emit(0)
    if overlap is not None:
        allow = (overlap.view(B, 1).long() << K) + torch.arange(NC, device=dev).view(1, NC)
        mask = torch.full((B, S), INF, device=dev)
        mask.scatter_(1, allow, 0.0)
        cost = cost + mask
    nkeep = T if back_from is None else max(0, T - 1 - back_from)
    fs_dtype = torch.uint8 if NC <= 256 else torch.int16
    from_state = torch.empty(nkeep, B, SP, dtype=fs_dtype, device=dev)
    for i in range(1, T):
        best = cost.view(B, NC, SP).min(dim=1)
        if back_from is None:
            from_state[i] = best.indices.to(fs_dtype)
        elif i > back_from:
            from_state[i - 1 - back_from] = best.indices.to(fs_dtype)
        e = emit(i)
        e.view(B, SP, NC).add_(best.values.unsqueeze(-1))
        cost = e
    if overlap is not None:
        allow = overlap.view(B, 1).long() + (torch.arange(NC, device=dev).view(1, NC) << (L - K))
        mask = torch.full((B, S), INF, device=dev)
        mask.scatter_(1, allow, 0.0)
        cost = cost + mask
    if back_from is not None:
        s = cost.argmin(dim=1)
        for i in range(T - 1, back_from, -1):
            j = s >> K
            w = from_state[i - 1 - back_from].gather(1, j.unsqueeze(1)).squeeze(1).long()
            s = j + w * SP
        return s
    states = torch.empty(T, B, dtype=torch.int64, device=dev)
    states[-1] = cost.argmin(dim=1)
    for i in range(T - 1, 0, -1):
        j = states[i] >> K
        w = from_state[i].gather(1, j.unsqueeze(1)).squeeze(1).long()
        states[i - 1] = j + w * SP
    return states


def tailbite(X: torch.Tensor, lut: torch.Tensor, K: int, L: int = 16,
             pivot: int | None = None, margin: int = 0) -> torch.Tensor:
    """X [T, B] -> states [T, B] int64 (two-pass QTIP tail-biting)."""
    T = X.shape[0]
    if pivot is None:
        pivot = T // 2
    roll = torch.roll(X, pivot, 0)
    if margin and pivot + margin < T:
        s_p = viterbi(roll[:pivot + margin], lut, K, L, back_from=pivot)
    else:
        s_p = viterbi(roll, lut, K, L)[pivot]
    ov = (s_p >> K).contiguous()
    return viterbi(X, lut, K, L, overlap=ov)
