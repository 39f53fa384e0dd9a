#!/usr/bin/env python3
"""quantize.py -- EXL3 trellis quantizer for one AMD Instinct MI355X (gfx950).

Drop-in host module for the reference quantizer's public API
(quantize/quantize.py of SergiioB/exl3xpu-mixedk): the same function names,
argument meanings, defaults where they still make sense, return values and
error behaviour.  The trellis work runs in hand-written HIP kernels
(libexl3vit.so, include/exl3_vit.h) called through ctypes on torch-ROCm device
tensors; there is no CPU Viterbi and no fallback -- every Viterbi, pack,
unpack and decode call raises if the library or a HIP device is missing.

Pipeline (reference citations are quantize.py:line):
  incoherence   random signs + block-128 Hadamard on both sides     121-182
  BlockLDLQ     block-LDL of the rotated damped Hessian, right-to-left
                16-row sweep with error feedback                    419-437, 631-746
  tail-biting   two-pass QTIP Viterbi per 16x16 tile (HIP)          323-354
  format        packed trellis [k/16, n/16, 16K] int16, decode      357-415

Orientation: public functions take nn.Linear W [out, in] and the input Gram
H [in, in] in the original basis; internally W_i is [k=in, n=out].

Backends: "hip" (default) runs the HIP kernels.  "torch" and "esimd", the
reference's backend names, are accepted as aliases of "hip" so existing call
sites keep working; the reference's per-launch "dual" comparator lives in the
test-suite (tests/test_gpu_quantize.py), which compares every launch against
the CPU oracle.  `compiled` and `batch` are accepted and ignored (the HIP path
has no torch.compile step and chunks batches itself).
"""
from __future__ import annotations

import math
import os
import sys
import threading
import time

import numpy as np
import torch

sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))
import hip_backend as _hb  # noqa: E402

BACKENDS = ("hip", "torch", "esimd")
# BlockLDLQ schedules: "block" is the reference's sweep (one tail-bite launch
# per 16-row block, feedback GEMMs in torch where W lives); "chain" runs the
# whole sweep as tile column chains in one persistent GPU launch with the
# feedback computed in the kernel; "auto" picks "chain" when W is on the GPU
# and "block" otherwise (so CPU-side runs reproduce the reference's torch
# arithmetic).
SCHEDULES = ("auto", "block", "chain")
DEFAULT_SCHEDULE = "auto"
_DUAL_STATS: dict = {}


# -------------------------------------------------------------- codebooks
def _f16(bits) -> np.ndarray:
    return np.asarray(bits).astype(np.uint16).view(np.float16)


_CODE_TABLES: dict = {}


def _code_table(name: str, L: int) -> np.ndarray:
    """fp32 decode table of a named V=1 code over all 2^L states
    (the codes of quantize.py:56-87), computed once per (code, L) and kept
    read-only (get_lut hands out copies)."""
    key = (name, int(L))
    t = _CODE_TABLES.get(key)
    if t is None:
        t = _code_table_compute(name, int(L))
        t.setflags(write=False)
        _CODE_TABLES[key] = t
    return t


def _code_table_compute(name: str, L: int) -> np.ndarray:
    s = np.arange(1 << L, dtype=np.uint64)
    if name == "exl3_mul1":
        h = (s * 0x83DCD12D) & 0xFFFFFFFF
        total = sum(((h >> sh) & 0xFF) for sh in (0, 8, 16, 24))
        c1 = float(_f16(0x1EEE))
        c2 = float(_f16(0xC931))
        return ((1024 + total).astype(np.float64) * c1 + c2).astype(np.float16).astype(np.float32)
    if name in ("exl3_3inst", "exl3_mcg"):
        h = (s * 89226354 + 64248484) if name == "exl3_3inst" else (s * 0xCBAC1FED)
        h = ((h & 0xFFFFFFFF) & 0x8FFF8FFF) ^ 0x3B603B60
        a = _f16(h & 0xFFFF).astype(np.float64)
        b = _f16(h >> 16).astype(np.float64)
        return (a + b).astype(np.float16).astype(np.float32)
    if name == "qtip_1mad":
        h = (s * 34038481 + 76625530) & 0xFFFFFFFF
        total = sum(((h >> sh) & 0xFF) for sh in (0, 8, 16, 24)).astype(np.float64)
        return ((total - 510.0) / 147.800537109375).astype(np.float32)
    raise KeyError(f"unknown local code {name!r}")


def get_lut(code: str, L: int = 16, device=None) -> torch.Tensor:
    """fp32 [2^L] decode table f(state) for the named code (quantize.py:90-97)."""
    lut = torch.from_numpy(_code_table(code, L).copy())
    return lut.to(device) if device is not None else lut


_LUT_IDS: dict = {}


def _kernel_code(lut: torch.Tensor, L: int) -> str:
    """Library code name for a decode table (the kernels hold the tables)."""
    if L != 16:
        raise NotImplementedError("the HIP trellis kernels use the 16-bit state (L=16)")
    lut = lut.detach().float().reshape(-1).cpu()
    for name in ("exl3_mul1", "exl3_3inst", "exl3_mcg", "qtip_1mad"):
        ref = _LUT_IDS.get(name)
        if ref is None:
            ref = _LUT_IDS[name] = get_lut(name, 16)
        if lut.shape == ref.shape and torch.equal(lut, ref):
            return name
    raise NotImplementedError(
        "the HIP trellis kernels run the V=1 codes exl3_mul1, exl3_3inst, exl3_mcg and "
        "qtip_1mad; this decode table is none of them")


# ------------------------------------------------------------ tile layout
def tensor_core_perm() -> torch.Tensor:
    """Sequence element t -> row-major position in the 16x16 [k, n] tile
    (quantize.py:101-118): groups of eight elements walk row pairs
    (r0, r0+1, r0+8, r0+9) in column c0 and then column c0+8."""
    t = torch.arange(256)
    g, e = t // 8, t % 8
    row = (g % 4) * 2 + (e % 2) + 8 * ((e // 2) % 2)
    col = g // 4 + 8 * (e // 4)
    return (row * 16 + col).long()


# ------------------------------------------------------------- incoherence
_H128: dict = {}


def hadamard128(device=None, dtype=torch.float32) -> torch.Tensor:
    """Normalised 128x128 Sylvester Hadamard matrix (symmetric, H H = I)."""
    key = (str(device), dtype)
    if key not in _H128:
        h = torch.ones(1, 1, dtype=torch.float64)
        while h.shape[0] < 128:
            h = torch.cat([torch.cat([h, h], 1), torch.cat([h, -h], 1)], 0)
        _H128[key] = (h / math.sqrt(128)).to(dtype=dtype, device=device)
    return _H128[key]


def had_left(w: torch.Tensor, h: torch.Tensor) -> torch.Tensor:
    """Block-128 Hadamard applied on the first (k) dim of w [k, n]
    (quantize.py:134-138).  GPU tensors go through the library's kernel,
    which accumulates every output in the order torch's CPU matmul does, so
    both devices give the reference's bits."""
    k, n = w.shape
    assert k % 128 == 0
    if w.is_cuda and w.dtype == torch.float32:
        return _hb.had128_left(w.contiguous(), h.to(w.device, torch.float32))
    return torch.matmul(h, w.view(k // 128, 128, n)).view(k, n)


def had_right(w: torch.Tensor, h: torch.Tensor) -> torch.Tensor:
    """Block-128 Hadamard applied on the last (n) dim of w [k, n]
    (quantize.py:141-145).  GPU tensors go through the library's kernel,
    which accumulates every output in the order torch's CPU matmul does."""
    k, n = w.shape
    assert n % 128 == 0
    if w.is_cuda and w.dtype == torch.float32:
        return _hb.had128_right(w.contiguous(), h.to(w.device, torch.float32))
    return torch.matmul(w.view(k, n // 128, 128), h).view(k, n)


def to_inner(w_orig: torch.Tensor, suh: torch.Tensor, svh: torch.Tensor,
             h: torch.Tensor) -> torch.Tensor:
    """W_orig [k, n] -> W_inner = B_k diag(1/suh) W diag(1/svh) B_n."""
    w = w_orig / suh.float().unsqueeze(1)
    w = w / svh.float().unsqueeze(0)
    return had_right(had_left(w, h), h)


def from_inner(w_inner: torch.Tensor, suh: torch.Tensor, svh: torch.Tensor,
               h: torch.Tensor) -> torch.Tensor:
    """W_inner -> W_orig = diag(suh) B_k W_i B_n diag(svh)."""
    w = had_left(w_inner, h) * suh.float().unsqueeze(1)
    return had_right(w, h) * svh.float().unsqueeze(0)


def rotate_hessian(H_x: torch.Tensor, suh: torch.Tensor, h: torch.Tensor) -> torch.Tensor:
    """Inner-basis input Gram G = B diag(suh) H_x diag(suh) B."""
    k = H_x.shape[0]
    a = H_x.float() * suh.float().unsqueeze(0) * suh.float().unsqueeze(1)
    return had_right(had_right(a.view(k, k), h).t().contiguous(), h)


_SIGNS: dict = {}


def sign_vec(n: int, seed: int, device=None) -> torch.Tensor:
    """Deterministic Rademacher vector from torch's CPU generator (drawn once
    per (n, seed); every call returns a tensor of its own)."""
    key = (int(n), int(seed))
    v = _SIGNS.get(key)
    if v is None:
        g = torch.Generator().manual_seed(seed)
        v = _SIGNS[key] = torch.where(torch.rand(n, generator=g) < 0.5, -1.0, 1.0)
    dev = torch.device(device) if device is not None else torch.device("cpu")
    return v.clone() if dev.type == "cpu" else v.to(dev)


# ------------------------------------------------------------------ Viterbi
def _check_viterbi_args(L: int, V: int, dtype, emit_mode: str):
    if V != 1:
        raise NotImplementedError("the HIP trellis kernels implement V=1 codes")
    if dtype not in (torch.float32, None):
        raise NotImplementedError("the bit-exact trellis path accumulates in float32")
    if emit_mode != "sq":
        raise NotImplementedError(
            "emit_mode must be 'sq' (the addmm emit of the reference is not bit-exact)")
    if L != 16:
        raise NotImplementedError("the HIP trellis kernels use the 16-bit state (L=16)")


_STAGE_BYTES = 32 << 20
_STAGE_MIN = 1 << 20
_STAGE: list = []
# the staging buffers serve one copy at a time (calls from several threads
# take turns)
_STAGE_LOCK = threading.Lock()


def _stage_buffers() -> list:
    if not _STAGE:
        _STAGE.extend(torch.empty(_STAGE_BYTES, dtype=torch.uint8, pin_memory=True)
                      for _ in range(2))
    return _STAGE


class _HostBuffers:
    """Host tensors of the given (shape, dtype) specs, allocated and every
    4 KiB page of them touched in a background thread.  The first-touch page
    faults of a fresh tensor otherwise set the pace of a large copy into it:
    c5's 356 MB fp32 W_hat took 11-20 ms from the staging buffers into fresh
    memory and 4.4 ms into touched memory, against 6.3 ms for the DMA.
    Started before the long device phase (its synchronous library calls
    release the interpreter lock), so the faults are taken while the host
    waits for the GPU."""

    def __init__(self, specs):
        specs = [(tuple(int(x) for x in shape), dtype) for shape, dtype in specs]
        self._bufs = [None] * len(specs)
        self._thread = threading.Thread(target=self._fill, args=(specs,), daemon=True)
        self._thread.start()

    def _fill(self, specs):
        for i, (shape, dtype) in enumerate(specs):
            t = torch.empty(shape, dtype=dtype)
            if t.numel():
                t.view(-1).view(torch.uint8)[::4096].zero_()
            self._bufs[i] = t

    def take(self, i: int):
        """Buffer i (None if the thread could not make it); each is handed
        out once."""
        self._thread.join()
        t, self._bufs[i] = self._bufs[i], None
        return t


def _to_host(t: torch.Tensor, out: torch.Tensor | None = None) -> torch.Tensor:
    """t.cpu() for device tensors of 1 MiB or more through two pinned staging
    buffers (allocated once per process): chunk i+1's device-to-host DMA runs
    while chunk i is copied into the (pageable) result -- `out` when given
    (a contiguous host tensor of t's shape and dtype, e.g. from
    _HostBuffers), else a new tensor.  Measured on the MI355X host: 126 MB
    in 3.9 ms, against 31 ms on the runtime's pageable path (~4 GB/s from
    64 MB up); 21 MB in 0.5 ms against 1.2 ms.  Smaller tensors and host
    tensors take t.cpu()."""
    if not t.is_cuda or t.numel() * t.element_size() < _STAGE_MIN:
        return t.cpu()
    src = t.contiguous().view(-1).view(torch.uint8)
    if (out is None or out.is_cuda or out.shape != t.shape or out.dtype != t.dtype
            or not out.is_contiguous()):
        out = torch.empty(t.shape, dtype=t.dtype)
    dst = out.view(-1).view(torch.uint8)
    n, C = src.numel(), _STAGE_BYTES
    offs = list(range(0, n, C))
    with _STAGE_LOCK, torch.cuda.device(t.device):
        stage = _stage_buffers()
        stream = torch.cuda.current_stream(t.device)
        ev = [torch.cuda.Event(), torch.cuda.Event()]

        def issue(i):
            o = offs[i]
            m = min(C, n - o)
            stage[i & 1][:m].copy_(src[o:o + m], non_blocking=True)
            ev[i & 1].record(stream)

        issue(0)
        for i, o in enumerate(offs):
            if i + 1 < len(offs):
                issue(i + 1)      # its buffer's previous chunk was copied out at i - 1
            ev[i & 1].synchronize()
            m = min(C, n - o)
            dst[o:o + m].copy_(stage[i & 1][:m])
    return out


def _to_device(t: torch.Tensor, dev: torch.device) -> torch.Tensor:
    """t.to(dev) for host tensors of 1 MiB or more through the two pinned
    staging buffers: chunk i is copied into buffer i & 1 while chunk i-1's
    host-to-device DMA runs; the call returns with every DMA complete (the
    buffers are free for the next copy).  Measured on the MI355X host:
    1.21 GB in 22 ms against 40 ms through the runtime's pageable path,
    67 MB in 1.6 ms against 2.3 ms.  Device tensors, CPU targets and smaller
    tensors take t.to(dev)."""
    dev = torch.device(dev)
    if (t.is_cuda or dev.type != "cuda"
            or t.numel() * t.element_size() < _STAGE_MIN):
        return t.to(dev)
    src = t.contiguous().view(-1).view(torch.uint8)
    out = torch.empty(t.shape, dtype=t.dtype, device=dev)
    dst = out.view(-1).view(torch.uint8)
    n, C = src.numel(), _STAGE_BYTES
    with _STAGE_LOCK, torch.cuda.device(dev):
        stage = _stage_buffers()
        stream = torch.cuda.current_stream(dev)
        ev = [torch.cuda.Event(), torch.cuda.Event()]
        for i, o in enumerate(range(0, n, C)):
            m = min(C, n - o)
            if i >= 2:
                ev[i & 1].synchronize()         # chunk i-2's DMA out of this buffer
            stage[i & 1][:m].copy_(src[o:o + m])
            dst[o:o + m].copy_(stage[i & 1][:m], non_blocking=True)
            ev[i & 1].record(stream)
        for e in ev:
            e.synchronize()
    return out


def _weight_fp32(W: torch.Tensor, dev: torch.device) -> torch.Tensor:
    """W as fp32 on dev.  fp16 and bf16 host weights cross in their own dtype
    (half the bytes) and are widened on the device, which gives the host
    conversion's bits for every bit pattern; other dtypes are converted
    where they are, as before the copy."""
    if W.dtype in (torch.float16, torch.bfloat16):
        return _to_device(W, dev).float()
    return _to_device(W.float(), dev)


def _on_gpu(X: torch.Tensor) -> torch.Tensor:
    if X.is_cuda:
        return X
    if not torch.cuda.is_available():
        raise RuntimeError("the trellis encoder needs a HIP device (none visible)")
    return X.cuda()


def viterbi(X: torch.Tensor, lut: torch.Tensor, K: int, L: int, V: int = 1,
            overlap: torch.Tensor = None, dtype: torch.dtype = torch.float32,
            back_from: int | None = None, compiled: bool = False,
            emit_mode: str = "sq"):
    """One trellis Viterbi run over X [T, B] (T <= 256), on the GPU.

    Returns states [T, B] int64, or with back_from the state at step
    back_from [B]; overlap [B] pins s_0 >> K and s_{T-1} mod 2^(L-K)
    (quantize.py:218-320).  Results land on X's device.
    """
    _check_viterbi_args(L, V, dtype, emit_mode)
    code = _hb.code_name(_kernel_code(lut, L))
    Xg = _on_gpu(X).float()
    st = _hb.viterbi(Xg.t().contiguous(), K, overlap=overlap, back_from=back_from,
                     code=code)
    st = st.long()
    st = st if back_from is not None else st.t().contiguous()
    return st.to(X.device)


def quantize_seq_tailbite(X: torch.Tensor, lut: torch.Tensor, K: int, L: int,
                          V: int = 1, dtype: torch.dtype = torch.float32,
                          pivot: int | None = None, margin: int = 0,
                          compiled: bool = False, emit_mode: str = "sq"):
    """QTIP tail-biting Viterbi of X [256, B] -> states [256, B] int64 on the
    GPU (quantize.py:323-354): pass 1 free on X rolled by pivot (truncated to
    pivot+margin steps when margin > 0), wrap bits ov = s_pivot >> K, pass 2
    pinned to ov."""
    _check_viterbi_args(L, V, dtype, emit_mode)
    T = X.shape[0]
    if T != 256:
        raise NotImplementedError("the HIP tail-biting encoder runs 256-step tiles")
    if pivot is None:
        pivot = T // 2
    assert 0 <= pivot < T
    code = _hb.code_name(_kernel_code(lut, L))
    Xg = _on_gpu(X).float().t().contiguous()
    st, _ = _hb.tailbite(Xg, K, int(pivot), int(margin), code=code)
    return st.long().t().contiguous().to(X.device)


# ------------------------------------------------------------ trellis format
def pack_states(states: torch.Tensor, K: int, V: int = 1) -> torch.Tensor:
    """states [ntiles, 256] -> int16 [ntiles, 16K] (quantize.py:360-378);
    symbol t = s_t mod 2^K at stream bits [tK, (t+1)K) MSB first, 32-bit
    words MSB first, stored as int16 halves, low half first."""
    if V != 1:
        raise NotImplementedError("V=1 only")
    st = _on_gpu(states).to(torch.int32).reshape(-1, 256)
    return _hb.pack(st, K).to(states.device)


def unpack_states(trellis: torch.Tensor, K: int, V: int = 1) -> torch.Tensor:
    """int16 [..., 16K] -> states [..., 256] int64 (quantize.py:381-402)."""
    if V != 1:
        raise NotImplementedError("V=1 only")
    st = _hb.unpack(_on_gpu(trellis).reshape(-1, 16 * K), K)
    return st.long().view(*trellis.shape[:-1], 256).to(trellis.device)


def decode_trellis(trellis: torch.Tensor, lut: torch.Tensor, K: int, k: int, n: int,
                   V: int = 1) -> torch.Tensor:
    """int16 [k/16, n/16, 16K] -> W_inner fp32 [k, n] (quantize.py:405-415)."""
    if V != 1:
        raise NotImplementedError("V=1 only")
    tk, tn, _ = trellis.shape
    assert (16 * tk, 16 * tn) == (k, n), (trellis.shape, k, n)
    code = _hb.code_name(_kernel_code(lut, 16))
    return _hb.decode(_on_gpu(trellis), K, code=code).to(trellis.device)


# ---------------------------------------------------------------- block LDL
# Device Cholesky from this order up runs on torch's MAGMA backend, when the
# build has it: measured on the MI355X (fp32) 4.7 / 6.6 / 7.8 / 35.5 ms at
# n = 3072 / 4096 / 5120 / 17408 against rocSOLVER's 9.4 / 12.9 / 16.3 /
# 81.4 ms; below it the two are even or rocSOLVER is faster.  Both are fp32
# factorizations (relative error of L against fp64 2e-5 vs 4e-6 at 17408;
# proxy loss of the quantized weight equal to 3e-4 relative).  The first
# MAGMA call in a process initialises it (~30 ms).
_MAGMA_CHOL_MIN = 3072


def _cholesky(H: torch.Tensor) -> torch.Tensor:
    """torch.linalg.cholesky, on MAGMA for large device matrices (torch's
    preferred linalg backend is switched for the call and restored)."""
    if H.is_cuda and H.shape[0] >= _MAGMA_CHOL_MIN and torch.cuda.has_magma:
        prev = torch.backends.cuda.preferred_linalg_library()
        torch.backends.cuda.preferred_linalg_library("magma")
        try:
            return torch.linalg.cholesky(H)
        finally:
            torch.backends.cuda.preferred_linalg_library(prev)
    return torch.linalg.cholesky(H)


def block_LDL(H: torch.Tensor, b: int):
    """QTIP block LDL (quantize.py:419-437): H = L D L^T with L unit-block
    lower triangular (b x b identity diagonal blocks) and D block diagonal.
    Raises torch's RuntimeError when H is not positive definite."""
    n = H.shape[0]
    assert n % b == 0
    m = n // b
    Lc = _cholesky(H)
    blocks = torch.diagonal(Lc.reshape(m, b, m, b), dim1=0, dim2=2).permute(2, 0, 1)
    D = blocks @ blocks.permute(0, 2, 1)
    inv = torch.linalg.inv(blocks)
    Lv = Lc.view(n, m, b)
    if Lc.is_cuda:
        # one batched product on the GPU (m launches of a 16-wide product
        # would dominate); each entry is the same length-b dot product
        Lv.copy_(torch.bmm(Lv.permute(1, 0, 2), inv).permute(1, 0, 2))
    else:
        for i in range(m):
            Lv[:, i, :] = Lv[:, i, :] @ inv[i]
    Lc = Lc.reshape(n, n).contiguous()
    idx = torch.arange(m, device=Lc.device)
    Lc.view(m, b, m, b)[idx, :, idx, :] = torch.eye(b, dtype=Lc.dtype, device=Lc.device)
    return Lc, D


# -------------------------------------------------------------- LDLQ sweep
def _tile_targets(rows: torch.Tensor, perm: torch.Tensor) -> torch.Tensor:
    """rows [16, n] of one 16-row block -> per-tile sequences [n/16, 256]
    with x_t = tile[perm[t]] (quantize.py:684-686)."""
    n = rows.shape[1]
    tiles = rows.view(16, n // 16, 16).permute(1, 0, 2).reshape(n // 16, 256)
    return tiles[:, perm].contiguous()


def _launch(X: torch.Tensor, K: int, code: str, pivot: int, margin: int):
    """One Viterbi launch: X [ntiles, 256] fp32 (device) -> (states int32,
    trellis int16), enqueued on the current stream without waiting (the sweep
    checks the NaN status once at its end).  Tests wrap this to compare each
    launch with the oracle."""
    return _hb.tailbite(X, K, pivot, margin, code=code, states=True, trellis=True,
                        sync=False)


def _lazy_cols(buf_cols) -> int:
    """Columns of the lazy feedback buffer: whole 16-column blocks, at least
    one, as the reference's buf_tiles = max(1, buf_cols // 16)
    (quantize.py:665) -- so buf_cols = 8 or 100 run as 16 and 96."""
    return 16 * max(1, int(buf_cols) // 16)


def ldlq_viterbi(Wq: torch.Tensor, Lfac: torch.Tensor | None, lut: torch.Tensor,
                 K: int, L: int, buf_cols: int = 128, V: int = 1,
                 batch: int = 0, dtype: torch.dtype = torch.float32,
                 pivot: int | None = None, margin: int = 0,
                 compiled: bool = False, progress=None,
                 code: str | None = None, backend: str = "hip",
                 schedule: str | None = None):
    """BlockLDLQ trellis quantization of W_i [k, n] (quantize.py:631-746).

    Sweeps the 16-row blocks right to left.  Block i's targets are
    W_i[rows i] + L[later, i]^T (W - What)[later] plus the lazily accumulated
    feedback of earlier buffers (every buf_cols/16 blocks); each 16x16 tile of
    the block is one tail-biting launch entry on the GPU.  Lfac None or all
    zeros gives plain Viterbi.  Returns (hatW [k, n] fp32, states int64
    [k/16, n/16, 256]) on Wq's device; the packed trellis of the sweep is left
    in ldlq_viterbi.last_trellis ([k/16, n/16, 16K] int16, GPU).

    schedule (default DEFAULT_SCHEDULE) picks the sweep's launch schedule
    (see SCHEDULES).  With "chain", ldlq_viterbi.keep_targets = True leaves
    every tile's targets in ldlq_viterbi.last_targets ([k/16, n/16, 256]
    fp32, sequence order, GPU).
    """
    if backend not in BACKENDS:
        raise ValueError(f"backend {backend!r} not in {BACKENDS}")
    schedule = DEFAULT_SCHEDULE if schedule is None else schedule
    if schedule not in SCHEDULES:
        raise ValueError(f"schedule {schedule!r} not in {SCHEDULES}")
    if schedule == "auto":
        schedule = "chain" if Wq.is_cuda else "block"
    _check_viterbi_args(L, V, dtype, "sq")
    k, n = Wq.shape
    assert k % 16 == 0 and n % 16 == 0
    dev = Wq.device
    gdev = _on_gpu(torch.empty(0)).device if not Wq.is_cuda else dev
    kcode = _hb.code_name(_kernel_code(lut, L))
    piv = 128 if pivot is None else int(pivot)
    perm = tensor_core_perm().to(dev)
    feedback = Lfac is not None and bool(Lfac.any())
    tk, tn = k // 16, n // 16
    ldlq_viterbi.last_targets = None
    ldlq_viterbi.last_groups = None
    if schedule == "chain":
        Wg = Wq.to(gdev, torch.float32).contiguous()
        Lg = Lfac.to(gdev, torch.float32).contiguous() if feedback else None
        hatW, states, trellis, xt = _hb.ldlq_chain(
            Wg, Lg, K, piv, int(margin), code=kcode, states=True,
            targets=bool(ldlq_viterbi.keep_targets), buf_cols=_lazy_cols(buf_cols))
        _chain_progress(progress, tk)
        ldlq_viterbi.last_trellis = trellis
        ldlq_viterbi.last_targets = xt
        return hatW.to(dev), states.long().to(dev)
    Lf = Lfac.to(dev, Wq.dtype) if feedback else None

    W_t = Wq.t().contiguous()                  # [n, k]
    hatW_t = torch.zeros_like(W_t)
    prod = torch.zeros(k, n, dtype=Wq.dtype, device=dev)
    states = torch.empty(tk, tn, 256, dtype=torch.int32, device=gdev)
    trellis = torch.empty(tk, tn, 16 * K, dtype=torch.int16, device=gdev)
    per_buf = _lazy_cols(buf_cols) // 16
    step_i = 0
    for cur in range(tk, 0, -per_buf):
        lo = max(0, cur - per_buf)
        for i in range(cur - 1, lo - 1, -1):
            c0, c1 = 16 * i, 16 * (i + 1)
            rows = W_t[:, c0:c1].t().contiguous()          # [16, n]
            if feedback:
                if c1 < 16 * cur:
                    err = (W_t[:, c1:16 * cur] - hatW_t[:, c1:16 * cur]).t()
                    rows = rows + Lf[c1:16 * cur, c0:c1].t() @ err
                rows = rows + prod[c0:c1, :]
            X = _tile_targets(rows, perm)
            st, tr = _launch(X.to(gdev), K, kcode, piv, int(margin))
            states[i] = st
            trellis[i] = tr
            step_i += 512
            if progress is not None:
                progress(i, step_i)
            # decoded block written back in [k, n] order: rows c0..c1 of What
            blk = _hb.decode(tr.view(1, tn, 16 * K), K, code=kcode)   # [16, n]
            hatW_t[:, c0:c1] = blk.to(dev).t()
        if feedback and lo > 0:
            err = (W_t[:, 16 * lo:16 * cur] - hatW_t[:, 16 * lo:16 * cur]).t()
            prod += Lf[16 * lo:16 * cur, :].t() @ err
    _hb.status(gdev)                 # NaN targets anywhere in the sweep raise here
    ldlq_viterbi.last_trellis = trellis
    return hatW_t.t().contiguous(), states.long().to(dev)


def _chain_progress(progress, tk: int):
    """The reference's per-block progress sequence (quantize.py:666,732-734):
    progress(i, 512 * blocks done) for the 16-row blocks i = tk-1 .. 0 in
    sweep order.  The column-chain schedule encodes all blocks in one launch,
    so the calls follow its completion."""
    if progress is None:
        return
    for d, i in enumerate(range(tk - 1, -1, -1), start=1):
        progress(i, 512 * d)


ldlq_viterbi.last_trellis = None
ldlq_viterbi.last_targets = None
ldlq_viterbi.last_groups = None
ldlq_viterbi.keep_targets = False


# ---------------------------------------------------------------- top level
def _factor_hessian(G: torch.Tensor):
    """block_LDL of the damped rotated Gram with the reference's failure
    policy (quantize.py:815-835): non-finite G raises; a non-SPD G is retried
    in fp64 with +0, +0.1, +1.0 x mean(diag) extra damping."""
    try:
        Lfac, _ = block_LDL(G.float(), 16)
        return Lfac
    except RuntimeError:
        if not torch.isfinite(G).all():
            raise
    Gd = G.double()
    for extra in (0.0, 0.1, 1.0):
        if extra:
            Gd.diagonal().add_(extra * Gd.diagonal().mean())
        try:
            Lfac, _ = block_LDL(Gd.clone(), 16)
            print(f"xtq_quant: block_LDL fallback used extra damping {extra} x mean diag",
                  flush=True)
            return Lfac
        except RuntimeError:
            if extra == 1.0:
                raise
    raise RuntimeError("unreachable")


def quantize_linear(W: torch.Tensor, H_x: torch.Tensor | None, code: str = "exl3_mul1",
                    K: int = 4, L: int = 16, V: int = 0, percdamp: float = 0.01,
                    su_seed: int = 20261011, buf_cols: int = 128,
                    use_ldlq: bool = True, device: str = "cpu",
                    batch: int = 0, dtype: torch.dtype = torch.float32,
                    margin: int = 0, compiled: bool = False, progress=None,
                    backend: str = "hip", channel_scales: bool = False,
                    reference_arithmetic: bool = False):
    """Quantize one nn.Linear weight (quantize.py:750-875).

    W [out, in]; H_x [in, in] undamped input Gram or None.  `device` is where
    the torch work (incoherence, block-LDL, LDLQ feedback) runs -- pass the
    GPU ("cuda") to keep the whole pipeline on the MI355X; the trellis
    kernels always run on the GPU.  Returns a dict with W_hat [out, in] fp32,
    trellis int16 [in/16, out/16, 16K], suh/svh fp16 and diagnostics.
    channel_scales=True applies EXL3 1.4.2's per-channel scaling order.

    On the GPU the Hadamard transforms and the LDLQ feedback already round as
    the reference's CPU arithmetic does; its reductions (channel RMS, Wscale,
    the damping mean) and the block-LDL factorisation (which the reference
    always runs on the CPU) round differently there.  reference_arithmetic=
    True runs those on the host CPU, as torch computes them for the
    reference, so that with device="cuda" every result equals the reference's
    device="cpu" result on the same host bit for bit.
    """
    return quantize_linear_group(
        [W], H_x, code=code, K=K, L=L, V=V, percdamp=percdamp, su_seed=su_seed,
        buf_cols=buf_cols, use_ldlq=use_ldlq, device=device, batch=batch, dtype=dtype,
        margin=margin, compiled=compiled, progress=progress, backend=backend,
        channel_scales=channel_scales, reference_arithmetic=reference_arithmetic)[0]


def quantize_linear_group(Ws, H_x: torch.Tensor | None, code: str = "exl3_mul1",
                          K=4, L: int = 16, V: int = 0, percdamp: float = 0.01,
                          su_seed: int = 20261011, buf_cols: int = 128,
                          use_ldlq: bool = True, device: str = "cpu",
                          batch: int = 0, dtype: torch.dtype = torch.float32,
                          margin: int = 0, compiled: bool = False, progress=None,
                          backend: str = "hip", channel_scales: bool = False,
                          reference_arithmetic: bool = False):
    """quantize_linear for several weights that read the same input (one
    H_x, e.g. the q/k/v or gate/up projections of a layer).  K is one bit
    width for all members or one per member (mixed-K, e.g. q at 5 and k/v
    at 7).

    The block-LDL factor is computed once and the members' inner weights are
    quantized side by side in one BlockLDLQ sweep: the sweep's feedback only
    mixes rows within an output column, so the members never interact.  With
    the column-chain schedule (GPU tensors) every result is bit-identical to
    a separate quantize_linear call; narrow members (out/16 below the GPU's
    compute-unit count) then share the GPU instead of leaving most of it
    idle, and members of different K run as concurrent launches over a split
    of the compute units.  Returns the list of quantize_linear result dicts,
    in order.  reference_arithmetic: see quantize_linear.
    """
    Ws = list(Ws)
    if not Ws:
        raise ValueError("quantize_linear_group needs at least one weight")
    Ks = [int(K)] * len(Ws) if isinstance(K, int) else [int(x) for x in K]
    if len(Ks) != len(Ws):
        raise ValueError(f"{len(Ks)} bit widths for {len(Ws)} weights")
    k_in = Ws[0].shape[1]
    for W in Ws:
        if W.dim() != 2 or W.shape[1] != k_in:
            raise ValueError(f"all weights must be [out, {k_in}], got {tuple(W.shape)}")
        assert k_in % 128 == 0 and W.shape[0] % 128 == 0, (W.shape, "need k%128, n%128")
    if backend not in BACKENDS:
        raise ValueError(f"backend {backend!r} not in {BACKENDS}")
    dev = torch.device(device)
    lut = get_lut(code, L).to(torch.float32)
    V = 1 if V == 0 else V
    lut_rms = lut.double().square().mean().sqrt().float()
    # the reference's reductions and factorisation on the host CPU
    host = bool(reference_arithmetic) and dev.type != "cpu"

    def red(t: torch.Tensor) -> torch.Tensor:
        """Where a reduction runs: the host CPU under reference_arithmetic."""
        return _to_host(t) if host else t

    suh0 = sign_vec(k_in, su_seed, dev).half()
    h = hadamard128(dev, torch.float32)
    members = []
    for W in Ws:
        m_out = W.shape[0]
        suh = suh0
        svh = sign_vec(m_out, su_seed + 1, dev).half()
        W32 = _weight_fp32(W, dev).t().contiguous()       # [k, n]
        mb = {"n": m_out}
        if channel_scales:
            su, sv = suh.float(), svh.float()
            r_out = red(W32).square().mean(dim=0).sqrt()
            rm = r_out.mean()
            if rm > 1e-30:
                r_out = r_out / rm
            zero_out = r_out.abs() < 1e-30
            r_out = torch.where(zero_out, torch.full_like(r_out, 0.1), r_out).to(dev)
            zero_out = zero_out.to(dev)
            w = had_right(W32 / (sv * r_out).unsqueeze(0), h)
            r_in = red(w).square().mean(dim=1).sqrt()
            r_in = torch.where(r_in.abs() < 1e-30, torch.full_like(r_in, 0.1), r_in).to(dev)
            W_i = had_left(w / (su * r_in).unsqueeze(1), h)
            svh_store = torch.where(zero_out, torch.zeros_like(r_out), r_out)
            mb.update(su=su, sv=sv, r_in=r_in, svh_store=svh_store)
        else:
            W_i = to_inner(W32, suh, svh, h)
        Wscale = (red(W_i).square().mean().sqrt() / lut_rms).to(dev)
        mb.update(Wq=W_i / Wscale, Wscale=Wscale, suh=suh, svh=svh)
        members.append(mb)
    Wq = members[0]["Wq"] if len(members) == 1 else \
        torch.cat([mb["Wq"] for mb in members], dim=1)

    Lfac = None
    if use_ldlq and H_x is not None:
        t0 = time.time()
        G = rotate_hessian(_to_device(H_x.float(), dev), suh0, h)
        if host:
            # the damping and the factorisation on a host copy of the whole
            # G, as the reference computes them (quantize.py:809-816): its
            # damping mean runs over the strided diagonal view of the [k, k]
            # matrix, and torch's CPU mean of a contiguous copy of that
            # diagonal can round differently
            G = _to_host(G)
        dead = G.diagonal() == 0
        if dead.any():
            G[dead, dead] = 1.0
        G.diagonal().add_(percdamp * G.diagonal().mean())
        # the reference factors on the CPU on every device (quantize.py:816)
        Lfac = _to_device(_factor_hessian(G).to(Wq.dtype), dev)
        del G
        if progress is not None:
            progress("hinv", time.time() - t0)

    # the results' host tensors (W_hat, trellis per member), paged in during
    # the sweep (after the factorisation, whose host side it would share the
    # cores with)
    outbufs = _HostBuffers([spec for W, Km in zip(Ws, Ks) for spec in (
        (W.shape, torch.float32),
        ((k_in // 16, W.shape[0] // 16, 16 * Km), torch.int16))]) if dev.type != "cpu" else None

    # runs of consecutive members with the same K: (first column, columns, K)
    runs = []
    for mb, Km in zip(members, Ks):
        if runs and runs[-1][2] == Km:
            runs[-1][1] += mb["n"]
        else:
            runs.append([sum(r[1] for r in runs), mb["n"], Km])
    sched = DEFAULT_SCHEDULE if DEFAULT_SCHEDULE != "auto" else \
        ("chain" if Wq.is_cuda else "block")
    if len(runs) == 1:
        hatWq, states = ldlq_viterbi(Wq, Lfac, lut, Ks[0], L, buf_cols=buf_cols, V=V,
                                     batch=batch, dtype=dtype, margin=margin,
                                     compiled=compiled, progress=progress,
                                     code=code, backend=backend)
        run_tr = [ldlq_viterbi.last_trellis]                      # GPU
    elif sched == "chain":
        # one call: a concurrent chain launch per run (xtq_ldlq_chain_multi_dev)
        _check_viterbi_args(L, V, dtype, "sq")
        gdev = _on_gpu(torch.empty(0)).device if not Wq.is_cuda else Wq.device
        feedback = Lfac is not None and bool(Lfac.any())
        hatWq, st, run_tr, xt = _hb.ldlq_chain(
            Wq.to(gdev, torch.float32).contiguous(),
            Lfac.to(gdev, torch.float32).contiguous() if feedback else None, None, 128,
            int(margin), code=_hb.code_name(_kernel_code(lut, L)), states=True,
            targets=bool(ldlq_viterbi.keep_targets), groups=[(r[1], r[2]) for r in runs],
            buf_cols=_lazy_cols(buf_cols))
        states = st.long().to(dev)
        hatWq = hatWq.to(dev)
        ldlq_viterbi.last_targets = xt
        ldlq_viterbi.last_trellis = None
        ldlq_viterbi.last_groups = [(r[0], r[1], r[2], t) for r, t in zip(runs, run_tr)]
        _chain_progress(progress, Wq.shape[0] // 16)
    else:
        hatWq = torch.empty_like(Wq)
        states = torch.empty(Wq.shape[0] // 16, Wq.shape[1] // 16, 256, dtype=torch.long,
                             device=dev)
        run_tr = []
        for c0, nc, Kr in runs:
            hw, stv = ldlq_viterbi(Wq[:, c0:c0 + nc].contiguous(), Lfac, lut, Kr, L,
                                   buf_cols=buf_cols, V=V, batch=batch, dtype=dtype,
                                   margin=margin, compiled=compiled, progress=progress,
                                   code=code, backend=backend)
            hatWq[:, c0:c0 + nc] = hw
            states[:, c0 // 16:(c0 + nc) // 16] = stv
            run_tr.append(ldlq_viterbi.last_trellis)
    # bit-exact self-checks of the format round trip (quantize.py:848-853),
    # compared where the trellis lives, per run of one K
    hatW_parts = []
    for (c0, nc, Kr), trellis in zip(runs, run_tr):
        st_rt = _hb.unpack(trellis.view(-1, 16 * Kr), Kr)
        st_ref = states[:, c0 // 16:(c0 + nc) // 16].reshape(-1, 256)
        assert torch.equal(st_rt, st_ref.to(st_rt.device, torch.int32)), \
            "pack/unpack round-trip broke state sequence"
        hw = _hb.decode(trellis, Kr, code=_hb.code_name(code))
        assert torch.equal(hw, hatWq[:, c0:c0 + nc].to(hw.device)), "decode != encoder output"
        hatW_parts.append(hw)
    out, off = [], 0
    for mi, (mb, Km) in enumerate(zip(members, Ks)):
        n = mb["n"]
        ri = max(i for i, r in enumerate(runs) if r[0] <= off)
        c0 = off - runs[ri][0]
        hatW_d = hatW_parts[ri][:, c0:c0 + n].contiguous().to(dev)
        tr = run_tr[ri][:, c0 // 16:(c0 + n) // 16].contiguous()
        off += n
        Wscale, suh, svh = mb["Wscale"], mb["suh"], mb["svh"]
        if channel_scales:
            suh = (mb["su"] * mb["r_in"] * Wscale).half()
            svh = (mb["sv"] * mb["svh_store"]).half()
            W_hat = from_inner(hatW_d, suh, svh, h).t().contiguous()
        else:
            W_hat = from_inner(hatW_d * Wscale, suh, svh, h).t().contiguous()
        out.append({
            "W_hat": _to_host(W_hat, outbufs.take(2 * mi) if outbufs else None),
            "trellis": _to_host(tr, outbufs.take(2 * mi + 1) if outbufs else None),
            "suh": suh.cpu(), "svh": svh.cpu(),
            "Wscale": float(Wscale), "lut_rms": float(lut_rms),
            "code": code, "K": Km, "L": L, "V": V, "use_ldlq": use_ldlq,
            "channel_scales": channel_scales,
        })
    return out


def hessian_weighted_err(W: torch.Tensor, W_hat: torch.Tensor, H_x: torch.Tensor) -> float:
    """Proxy loss tr(dW H dW^T) / tr(W H W^T), W [out, in] (quantize.py:878-885)."""
    dW = (W_hat - W).float()
    H = H_x.float()
    num = torch.einsum("ij,jk,ik->", dW, H, dW)
    den = torch.einsum("ij,jk,ik->", W.float(), H, W.float())
    return float(num / den)


def rel_mse(W: torch.Tensor, W_hat: torch.Tensor) -> float:
    d = W_hat.float() - W.float()
    return float(d.square().sum() / W.float().square().sum())


def quantize(W_transformed: torch.Tensor, U_upper: torch.Tensor | None,
             code: str, K: int, seed: int, L: int = 16,
             dtype: torch.dtype = torch.float32,
             backend: str = "hip", margin: int = 16, batch: int = 0,
             su_mag: torch.Tensor | None = None,
             sv_mag: torch.Tensor | None = None,
             reference_arithmetic: bool = False):
    """Harness entry point (quantize.py:894-966).

    W_transformed [out, in] fp32 already in the inner (incoherent) domain;
    U_upper [in, in] the GPTQ-convention factor with U^T U = G^-1 (or None
    for plain tail-biting Viterbi); seed picks the pass-1 pivot (seed mod 256).
    su_mag/sv_mag fold per-channel magnitudes out before quantization and back
    into W_hat.  Runs on W_transformed's device; the U -> L conversion runs on
    U_upper's.  Returns (W_hat [out, in] fp32, packed int16 [in/16, out/16,
    16K], scale) with decode(packed) * scale == W_hat bit for bit (before the
    magnitude refold).

    On the GPU the sweep's feedback already rounds as the reference's CPU
    arithmetic does; the scale (a mean over the weight) and, for a device
    U_upper, the U -> L conversion round differently there.
    reference_arithmetic=True runs both on the host CPU, as torch computes
    them for the reference, so that every output equals the reference's
    CPU result bit for bit.
    """
    m_out, k_in = W_transformed.shape
    assert k_in % 16 == 0 and m_out % 16 == 0, W_transformed.shape
    lut = get_lut(code, L).float()
    lut_rms = lut.double().square().mean().sqrt().float()
    Wt = W_transformed.float()
    folded = su_mag is not None or sv_mag is not None
    if folded:
        su_m = (torch.ones(k_in, dtype=Wt.dtype, device=Wt.device) if su_mag is None
                else su_mag.float().to(Wt.device))
        sv_m = (torch.ones(m_out, dtype=Wt.dtype, device=Wt.device) if sv_mag is None
                else sv_mag.float().to(Wt.device))
        Wt = Wt / (sv_m.unsqueeze(1) * su_m.unsqueeze(0))
    Wq = Wt.t().contiguous()
    host = bool(reference_arithmetic) and Wq.device.type != "cpu"
    scale = ((_to_host(Wq) if host else Wq).square().mean().sqrt() / lut_rms).to(Wq.device)
    Wq = Wq / scale
    Lfac = None
    if U_upper is not None:
        Uu = (_to_host(U_upper) if reference_arithmetic else U_upper).double()
        eye = torch.eye(Uu.shape[0], dtype=Uu.dtype, device=Uu.device)
        Ui = torch.linalg.solve_triangular(Uu, eye, upper=True)     # U^-1
        Lfac, _ = block_LDL(Ui @ Ui.t(), 16)                         # G = U^-1 U^-T
        Lfac = Lfac.float()
    pivot = int(seed) % 256
    hatWq, states = ldlq_viterbi(Wq, Lfac, lut, K, L, dtype=dtype, pivot=pivot,
                                 margin=margin, code=code, backend=backend, batch=batch)
    packed = ldlq_viterbi.last_trellis
    st_rt = _hb.unpack(packed.view(-1, 16 * K), K)
    assert torch.equal(st_rt, states.reshape(-1, 256).to(st_rt.device, torch.int32)), \
        "pack/unpack round-trip broke state sequence"
    W_hat = (hatWq * scale).t().contiguous()
    hatW_rt = decode_trellis(packed, lut, K, k_in, m_out).to(hatWq.device) * scale
    assert torch.equal(hatW_rt.t().contiguous(), W_hat), "decode != encoder"
    if folded:
        W_hat = W_hat * (sv_m.unsqueeze(1) * su_m.unsqueeze(0))
    return W_hat, packed.to(W_transformed.device), float(scale)


def prepare_incoherence(W: torch.Tensor, H_x: torch.Tensor | None = None,
                        su_seed: int = 20261011,
                        sv_seed: int | None = None,
                        su_sign: torch.Tensor | None = None,
                        sv_sign: torch.Tensor | None = None,
                        channel_scales: bool = True,
                        device: str = "cpu") -> dict:
    """Incoherence transform in pieces for a harness that owns damping and the
    U build (quantize.py:969-1058).  Returns Wt [out, in] (magnitudes folded,
    Wscale not), the sign-only rotated undamped Gram G, signed magnitudes
    suh/svh, raw magnitudes su_mag/sv_mag and the dead-output mask."""
    m_out, k_in = W.shape
    assert k_in % 128 == 0 and m_out % 128 == 0, (W.shape, "need %128 dims")
    dev = torch.device(device)
    h = hadamard128(dev, torch.float32)
    su_s = (sign_vec(k_in, su_seed, dev).half() if su_sign is None
            else su_sign.to(dev).half())
    sv_s = (sign_vec(m_out, (su_seed + 1) if sv_seed is None else sv_seed, dev).half()
            if sv_sign is None else sv_sign.to(dev).half())
    W32 = _weight_fp32(W, dev).t().contiguous()
    if channel_scales:
        su, sv = su_s.float(), sv_s.float()
        sv_mag = W32.square().mean(dim=0).sqrt()
        rm = sv_mag.mean()
        if rm > 1e-30:
            sv_mag = sv_mag / rm
        zero_out = sv_mag.abs() < 1e-30
        sv_mag = torch.where(zero_out, torch.full_like(sv_mag, 0.1), sv_mag)
        w = had_right(W32 / (sv * sv_mag).unsqueeze(0), h)
        su_mag = w.square().mean(dim=1).sqrt()
        su_mag = torch.where(su_mag.abs() < 1e-30, torch.full_like(su_mag, 0.1), su_mag)
        W_i = had_left(w / (su * su_mag).unsqueeze(1), h)
        suh = su * su_mag
        svh = sv * torch.where(zero_out, torch.zeros_like(sv_mag), sv_mag)
    else:
        W_i = to_inner(W32, su_s, sv_s, h)
        suh, svh = su_s.float(), sv_s.float()
        su_mag = torch.ones(k_in, device=dev)
        sv_mag = torch.ones(m_out, device=dev)
        zero_out = torch.zeros(m_out, dtype=torch.bool, device=dev)
    G = _to_host(rotate_hessian(_to_device(H_x.float(), dev), su_s, h)) \
        if H_x is not None else None
    return {"Wt": W_i.t().contiguous().cpu(), "G": G,
            "suh": suh.cpu(), "svh": svh.cpu(),
            "su_mag": su_mag.cpu(), "sv_mag": sv_mag.cpu(),
            "zero_out": zero_out.cpu(), "channel_scales": channel_scales}
