"""hip_backend.py -- ctypes binding of libexl3vit.so (include/exl3_vit.h).

The MI355X counterpart of the reference's ESIMD transport
(quantize.py:441-628): the same C-ABI conventions (int status, caller-owned
buffers, library-owned scratch), but the encoder runs on torch-ROCm device
tensors in place, so the LDLQ sweep never round-trips targets through the
host.  There is no fallback: if the library is missing or the tensors are not
on a HIP device, the calls raise.
"""
from __future__ import annotations

import ctypes
import os

import torch

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.environ.get(
    "XTQ_VIT_LIB",
    os.path.normpath(os.path.join(_HERE, "..", "lib", "libexl3vit.so")))

_LIB = None

# Codebook names accepted by the library (fp16-exact V=1 codes).
CODE_NAMES = {"exl3_mul1": "mul1", "exl3_3inst": "3inst", "exl3_mcg": "mcg",
              "qtip_1mad": "1mad",
              "mul1": "mul1", "3inst": "3inst", "mcg": "mcg", "1mad": "1mad"}


class HipViterbiError(RuntimeError):
    """A non-zero status from libexl3vit.so."""

    def __init__(self, fn: str, rc: int):
        msg = lib().xtq_vit_strerror(rc).decode() if _LIB is not None else "?"
        super().__init__(f"{fn} rc={rc} ({msg})")
        self.rc = rc


def lib():
    """Load libexl3vit.so once; raises if it has not been built."""
    global _LIB
    if _LIB is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(
                f"libexl3vit.so not found at {LIB_PATH}; build it with "
                "`make -C exl3xpu-mixedk_amd` (or __graft_entry__.build())")
        L = ctypes.CDLL(LIB_PATH)
        vp, i32, i64 = ctypes.c_void_p, ctypes.c_int, ctypes.c_int64
        cp = ctypes.c_char_p
        L.xtq_vit_init.argtypes = []
        L.xtq_vit_run.argtypes = [vp, i32, cp, i32, i32, vp]
        L.xtq_vit_run_k.argtypes = [vp, i32, i32, cp, i32, i32, vp]
        L.xtq_vit_tailbite_dev.argtypes = [vp, i32, i32, cp, i32, i32, vp, vp, vp]
        L.xtq_vit_tailbite_dev_async.argtypes = [vp, i32, i32, cp, i32, i32, vp, vp, vp]
        L.xtq_vit_tailbite_dev_noalloc.argtypes = [vp, i32, i32, cp, i32, i32, vp, vp, vp]
        L.xtq_vit_status_dev.argtypes = [vp]
        L.xtq_ldlq_chain_dev.argtypes = [vp, vp, i32, i32, i32, cp, i32, i32, i32, vp, vp, vp,
                                         vp, vp]
        L.xtq_ldlq_chain_multi_dev.argtypes = [vp, vp, i32, i32, i32, vp, vp, cp, i32, i32,
                                               i32, vp, vp, vp, vp, vp]
        L.xtq_vit_viterbi_dev.argtypes = [vp, i32, i32, i32, cp, vp, i32, vp, vp]
        L.xtq_trellis_decode_dev.argtypes = [vp, i32, i32, i32, cp, vp, vp, vp]
        L.xtq_trellis_pack_dev.argtypes = [vp, i32, i32, vp, vp]
        L.xtq_trellis_unpack_dev.argtypes = [vp, i32, i32, vp, vp]
        L.xtq_vit_get_lut.argtypes = [cp, vp]
        L.xtq_had128_left_dev.argtypes = [vp, vp, vp, i32, i32, vp]
        L.xtq_had128_right_dev.argtypes = [vp, vp, vp, i32, i32, vp]
        L.xtq_vit_scratch_per_seq.argtypes = [i32]
        L.xtq_vit_scratch_per_seq.restype = i64
        L.xtq_vit_chunk_seqs.argtypes = [i32, i32, ctypes.POINTER(ctypes.c_int)]
        L.xtq_vit_chunk_seqs.restype = i32
        L.xtq_vit_prof_enable.argtypes = [i32]
        L.xtq_vit_prof_enable.restype = i32
        dp = ctypes.POINTER(ctypes.c_double)
        lp = ctypes.POINTER(ctypes.c_int64)
        L.xtq_vit_prof_read.argtypes = [dp, lp, dp, dp, lp]
        L.xtq_vit_prof_read.restype = i32
        L.xtq_vit_strerror.argtypes = [i32]
        L.xtq_vit_strerror.restype = cp
        for fn in ("xtq_vit_init", "xtq_vit_run", "xtq_vit_run_k", "xtq_vit_tailbite_dev",
                   "xtq_vit_tailbite_dev_async", "xtq_vit_tailbite_dev_noalloc", "xtq_vit_status_dev", "xtq_vit_viterbi_dev",
                   "xtq_ldlq_chain_dev", "xtq_ldlq_chain_multi_dev",
                   "xtq_trellis_decode_dev", "xtq_trellis_pack_dev",
                   "xtq_trellis_unpack_dev", "xtq_vit_get_lut", "xtq_had128_left_dev",
                   "xtq_had128_right_dev"):
            getattr(L, fn).restype = i32
        _LIB = L
    return _LIB


def _check(fn: str, rc: int):
    if rc:
        raise HipViterbiError(fn, rc)


def code_name(code: str) -> str:
    try:
        return CODE_NAMES[code]
    except KeyError:
        raise NotImplementedError(
            f"code {code!r} has no HIP trellis kernel (supported: "
            f"{sorted(set(CODE_NAMES))})") from None


def _dev_tensor(t: torch.Tensor, dtype: torch.dtype, name: str) -> torch.Tensor:
    if not t.is_cuda:
        raise ValueError(f"{name} must be a HIP device tensor, got {t.device}")
    if t.dtype != dtype:
        raise ValueError(f"{name} must be {dtype}, got {t.dtype}")
    return t.contiguous()


def _stream(dev: torch.device) -> int:
    return torch.cuda.current_stream(dev).cuda_stream


def tailbite(X: torch.Tensor, K: int, pivot: int, margin: int, code: str = "mul1",
             states: bool = True, trellis: bool = False, sync: bool = True):
    """Tail-biting encode of X [nseq, 256] fp32 (device).

    Returns (states int32 [nseq, 256] or None, trellis int16 [nseq, 16K] or
    None), both on X's device.  Bit-exact with quantize_seq_tailbite
    (quantize.py:323-354) given the same targets, pivot and margin.
    sync=False only enqueues the work on the current stream; a NaN target is
    then reported by the next status() call instead of raising here.
    """
    X = _dev_tensor(X, torch.float32, "X")
    if X.dim() != 2 or X.shape[1] != 256:
        raise ValueError(f"X must be [nseq, 256], got {tuple(X.shape)}")
    nseq = X.shape[0]
    st = torch.empty(nseq, 256, dtype=torch.int32, device=X.device) if states else None
    tr = torch.empty(nseq, 16 * K, dtype=torch.int16, device=X.device) if trellis else None
    if nseq == 0:
        return st, tr
    fn = "xtq_vit_tailbite_dev" if sync else "xtq_vit_tailbite_dev_async"
    with torch.cuda.device(X.device):
        rc = getattr(lib(), fn)(
            X.data_ptr(), nseq, int(K), code_name(code).encode(), int(margin), int(pivot),
            st.data_ptr() if st is not None else None,
            tr.data_ptr() if tr is not None else None, _stream(X.device))
    _check(fn, rc)
    return st, tr


def status(device=None):
    """Wait for the current stream of `device` and raise HipViterbiError
    (rc 11) if a stream-ordered encode met a NaN target since the last check."""
    dev = torch.device("cuda") if device is None else torch.device(device)
    with torch.cuda.device(dev):
        _check("xtq_vit_status_dev", lib().xtq_vit_status_dev(_stream(dev)))


def ldlq_chain(W: torch.Tensor, L: torch.Tensor | None, K, pivot: int, margin: int,
               code: str = "mul1", states: bool = True, targets: bool = False,
               groups=None, buf_cols: int = 128):
    """BlockLDLQ sweep of W [k, n] fp32 (inner domain, device) with the
    block-LDL factor L [k, k] (or None: no feedback) as column chains on the
    GPU (xtq_ldlq_chain_dev), the feedback summed in the order of the
    reference's ldlq_viterbi with lazy buffers of buf_cols columns.  Returns
    (What [k, n] fp32, states int32 [k/16, n/16, 256] or None, trellis int16
    [k/16, n/16, 16K], targets fp32 [k/16, n/16, 256] or None), all on W's
    device.

    groups: None (all columns at K), or a list of (ncols, K) that splits W's
    columns into consecutive groups encoded at their own K
    (xtq_ldlq_chain_multi_dev); the trellis is then a list with one
    [k/16, ncols/16, 16K] tensor per group."""
    W = _dev_tensor(W, torch.float32, "W")
    if W.dim() != 2 or W.shape[0] % 16 or W.shape[1] % 16:
        raise ValueError(f"W must be [k, n] with k, n multiples of 16, got {tuple(W.shape)}")
    k, n = W.shape
    if L is not None:
        L = _dev_tensor(L, torch.float32, "L")
        if L.shape != (k, k) or L.device != W.device:
            raise ValueError(f"L must be [{k}, {k}] on {W.device}")
    single = groups is None
    if single:
        groups = [(n, int(K))]
    groups = [(int(c), int(kk)) for c, kk in groups]
    if sum(c for c, _ in groups) != n or any(c <= 0 or c % 16 for c, _ in groups):
        raise ValueError(f"group widths {[c for c, _ in groups]} must be multiples of 16 "
                         f"summing to {n}")
    tk, tn = k // 16, n // 16
    dev = W.device
    hatW = torch.empty(k, n, dtype=torch.float32, device=dev)
    st = torch.empty(tk, tn, 256, dtype=torch.int32, device=dev) if states else None
    trs = [torch.empty(tk, c // 16, 16 * kk, dtype=torch.int16, device=dev) for c, kk in groups]
    xt = torch.empty(tk, tn, 256, dtype=torch.float32, device=dev) if targets else None
    ng = len(groups)
    ncols = (ctypes.c_int * ng)(*[c for c, _ in groups])
    ks = (ctypes.c_int * ng)(*[kk for _, kk in groups])
    ptrs = (ctypes.c_void_p * ng)(*[t.data_ptr() for t in trs])
    with torch.cuda.device(dev):
        rc = lib().xtq_ldlq_chain_multi_dev(
            W.data_ptr(), L.data_ptr() if L is not None else None, k, n, ng, ncols, ks,
            code_name(code).encode(), int(margin), int(pivot), int(buf_cols), hatW.data_ptr(),
            st.data_ptr() if st is not None else None, ptrs,
            xt.data_ptr() if xt is not None else None, _stream(dev))
    _check("xtq_ldlq_chain_multi_dev", rc)
    return hatW, st, (trs[0] if single else trs), xt


def viterbi(X: torch.Tensor, K: int, overlap: torch.Tensor | None = None,
            back_from: int | None = None, code: str = "mul1") -> torch.Tensor:
    """One Viterbi run over X [nseq, T] fp32 (device), T <= 256.

    Free run, or pinned to overlap [nseq] (s_0 >> K and s_{T-1} mod 2^(16-K));
    returns int32 states [nseq, T], or [nseq] (the state at back_from).
    Bit-exact with viterbi() (quantize.py:218-320) for V = 1, L = 16.
    """
    X = _dev_tensor(X, torch.float32, "X")
    if X.dim() != 2 or not 1 <= X.shape[1] <= 256:
        raise ValueError(f"X must be [nseq, T<=256], got {tuple(X.shape)}")
    nseq, T = X.shape
    bf = -1 if back_from is None else int(back_from)
    if not -1 <= bf < T:
        raise ValueError(f"back_from {back_from} outside [0, {T})")
    ov = None
    if overlap is not None:
        ov = overlap.to(device=X.device, dtype=torch.int32).contiguous()
        if ov.shape != (nseq,):
            raise ValueError(f"overlap must be [{nseq}], got {tuple(ov.shape)}")
        if nseq and (int(ov.min()) < 0 or int(ov.max()) >= (1 << (16 - K))):
            raise ValueError("overlap values must lie in [0, 2^(16-K))")
    out = torch.empty((nseq,) if bf >= 0 else (nseq, T), dtype=torch.int32, device=X.device)
    if nseq == 0:
        return out
    with torch.cuda.device(X.device):
        rc = lib().xtq_vit_viterbi_dev(
            X.data_ptr(), nseq, T, int(K), code_name(code).encode(),
            ov.data_ptr() if ov is not None else None, bf, out.data_ptr(),
            _stream(X.device))
    _check("xtq_vit_viterbi_dev", rc)
    return out


def decode(trellis: torch.Tensor, K: int, code: str = "mul1",
           dtype: torch.dtype = torch.float32) -> torch.Tensor:
    """int16 [tk, tn, 16K] (device) -> W_inner [16 tk, 16 tn] (quantize.py:405-415)."""
    tr = _dev_tensor(trellis, torch.int16, "trellis")
    tk, tn, w = tr.shape
    if w != 16 * K:
        raise ValueError(f"trellis last dim {w} != 16*K = {16 * K}")
    if dtype not in (torch.float32, torch.float16):
        raise ValueError("decode dtype must be float32 or float16")
    out = torch.empty(16 * tk, 16 * tn, dtype=dtype, device=tr.device)
    if tk == 0 or tn == 0:
        return out
    with torch.cuda.device(tr.device):
        rc = lib().xtq_trellis_decode_dev(
            tr.data_ptr(), tk, tn, int(K), code_name(code).encode(),
            out.data_ptr() if dtype == torch.float32 else None,
            out.data_ptr() if dtype == torch.float16 else None, _stream(tr.device))
    _check("xtq_trellis_decode_dev", rc)
    return out


def had128_left(w: torch.Tensor, h: torch.Tensor) -> torch.Tensor:
    """blockdiag(h) @ w for w [k, n] fp32 (device, k a multiple of 128) and
    any 128x128 h on the same device (the reference applies the normalised
    Sylvester matrix): each output one fused multiply-add chain in ascending
    order, as torch's CPU sgemm evaluates the reference's matmul
    (xtq_had128_left_dev, which takes the multipliers by input row, h^T)."""
    w = _dev_tensor(w, torch.float32, "w")
    h = _dev_tensor(h, torch.float32, "h")
    if w.dim() != 2 or w.shape[0] % 128 or h.shape != (128, 128) or h.device != w.device:
        raise ValueError(f"had128_left needs w [128m, n] and h [128, 128] on one device, got "
                         f"{tuple(w.shape)}, {tuple(h.shape)}")
    out = torch.empty_like(w)
    if w.numel() == 0:
        return out
    with torch.cuda.device(w.device):
        ht = h.t().contiguous()
        rc = lib().xtq_had128_left_dev(ht.data_ptr(), w.data_ptr(), out.data_ptr(), w.shape[0],
                                       w.shape[1], _stream(w.device))
    _check("xtq_had128_left_dev", rc)
    return out


def had128_right(w: torch.Tensor, h: torch.Tensor) -> torch.Tensor:
    """w @ blockdiag(h) for w [k, n] fp32 (device, n a multiple of 128) and
    any 128x128 h on the same device: each output one fused multiply-add
    chain in ascending order, as torch's CPU sgemm evaluates the reference's
    matmul (xtq_had128_right_dev)."""
    w = _dev_tensor(w, torch.float32, "w")
    h = _dev_tensor(h, torch.float32, "h")
    if w.dim() != 2 or w.shape[1] % 128 or h.shape != (128, 128) or h.device != w.device:
        raise ValueError(f"had128_right needs w [k, 128m] and h [128, 128] on one device, got "
                         f"{tuple(w.shape)}, {tuple(h.shape)}")
    out = torch.empty_like(w)
    if w.numel() == 0:
        return out
    with torch.cuda.device(w.device):
        hc = h.contiguous()
        rc = lib().xtq_had128_right_dev(hc.data_ptr(), w.data_ptr(), out.data_ptr(), w.shape[0],
                                        w.shape[1], _stream(w.device))
    _check("xtq_had128_right_dev", rc)
    return out


def pack(states: torch.Tensor, K: int) -> torch.Tensor:
    """int32 states [nt, 256] (device) -> int16 trellis [nt, 16K]."""
    st = _dev_tensor(states, torch.int32, "states")
    nt = st.shape[0]
    out = torch.empty(nt, 16 * K, dtype=torch.int16, device=st.device)
    if nt:
        with torch.cuda.device(st.device):
            rc = lib().xtq_trellis_pack_dev(st.data_ptr(), nt, int(K), out.data_ptr(),
                                            _stream(st.device))
        _check("xtq_trellis_pack_dev", rc)
    return out


def unpack(trellis: torch.Tensor, K: int) -> torch.Tensor:
    """int16 trellis [nt, 16K] (device) -> int32 states [nt, 256]."""
    tr = _dev_tensor(trellis, torch.int16, "trellis").view(-1, 16 * K)
    nt = tr.shape[0]
    out = torch.empty(nt, 256, dtype=torch.int32, device=tr.device)
    if nt:
        with torch.cuda.device(tr.device):
            rc = lib().xtq_trellis_unpack_dev(tr.data_ptr(), nt, int(K), out.data_ptr(),
                                              _stream(tr.device))
        _check("xtq_trellis_unpack_dev", rc)
    return out


def get_lut(code: str = "mul1") -> torch.Tensor:
    """fp32 [65536] decode table as the library computes it (host)."""
    out = torch.empty(65536, dtype=torch.float32)
    _check("xtq_vit_get_lut", lib().xtq_vit_get_lut(code_name(code).encode(), out.data_ptr()))
    return out


def scratch_per_seq(K: int) -> int:
    return int(lib().xtq_vit_scratch_per_seq(int(K)))


def chunk_seqs(nseq: int, K: int):
    """(sequences per scratch chunk, deferred-argmin encode?) the library
    would use for a tail-bite of nseq sequences at K on the current device
    (xtq_vit_chunk_seqs)."""
    d = ctypes.c_int()
    n = lib().xtq_vit_chunk_seqs(int(nseq), int(K), ctypes.byref(d))
    if n < 0:
        raise HipViterbiError("xtq_vit_chunk_seqs", -n)
    return n, bool(d.value)


def prof_enable(on: bool = True):
    """Bracket every forward/traceback launch with HIP events (benchmarks)."""
    lib().xtq_vit_prof_enable(1 if on else 0)


def prof_read() -> dict:
    """Totals since the last read: forward ms/launches/sequence-steps and
    traceback ms/launches (xtq_vit_prof_read)."""
    fm, ss, tm = ctypes.c_double(), ctypes.c_double(), ctypes.c_double()
    fl, tl = ctypes.c_int64(), ctypes.c_int64()
    lib().xtq_vit_prof_read(ctypes.byref(fm), ctypes.byref(fl), ctypes.byref(ss),
                            ctypes.byref(tm), ctypes.byref(tl))
    return {"fwd_ms": fm.value, "fwd_launches": fl.value, "fwd_seq_steps": ss.value,
            "tb_ms": tm.value, "tb_launches": tl.value}
