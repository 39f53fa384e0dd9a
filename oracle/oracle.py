"""oracle.py -- CPU oracle for the EXL3 trellis Viterbi path (TEST INFRASTRUCTURE).

Only tests/, the smoke check in __graft_entry__.py and the CPU-baseline leg of
bench.py may import this module, and only as the checker.  The product path
(the HIP library and exl3xpu-mixedk_amd/quantize) never imports it.

Contents
  * ctypes bindings to liboracle.so (viterbi_oracle.c): the scalar fp32
    restatement of quantize.py:218-415 (viterbi, quantize_seq_tailbite,
    pack/unpack/decode, tensor_core_perm).
  * numpy restatements of the codebook tables, following
    quantize.py:56-87 (_local_code_lut) operation for operation.
  * small pure-Python brute-force helpers for tiny trellises (L <= 8), used
    to pin the DP and its tie rule independently of the recurrence.
"""
from __future__ import annotations

import ctypes
import itertools
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB = None


def build(force: bool = False) -> str:
    """Compile liboracle.so with the committed Makefile (gcc, no fast-math)."""
    so = os.path.join(_HERE, "liboracle.so")
    if force or not os.path.exists(so):
        subprocess.run(["make", "-s", "-C", _HERE], check=True)
    return so


def lib():
    global _LIB
    if _LIB is None:
        so = os.path.join(_HERE, "liboracle.so")
        if not os.path.exists(so):
            build()
        L = ctypes.CDLL(so)
        c_i32p = ctypes.POINTER(ctypes.c_int32)
        c_f32p = ctypes.POINTER(ctypes.c_float)
        c_i16p = ctypes.POINTER(ctypes.c_int16)
        L.orc_viterbi.argtypes = [c_f32p, ctypes.c_int, ctypes.c_int, c_f32p,
                                  ctypes.c_int, ctypes.c_int, c_i32p,
                                  ctypes.c_int, c_i32p, ctypes.c_int]
        L.orc_tailbite.argtypes = [c_f32p, ctypes.c_int, ctypes.c_int, c_f32p,
                                   ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                   ctypes.c_int, c_i32p, c_i32p, ctypes.c_int]
        L.orc_tensor_core_perm.argtypes = [c_i32p]
        L.orc_tensor_core_perm.restype = None
        L.orc_pack.argtypes = [c_i32p, ctypes.c_int, ctypes.c_int, c_i16p]
        L.orc_unpack.argtypes = [c_i16p, ctypes.c_int, ctypes.c_int, c_i32p]
        L.orc_decode.argtypes = [c_i16p, ctypes.c_int, ctypes.c_int,
                                 ctypes.c_int, c_f32p, c_f32p]
        L.orc_path_cost.argtypes = [c_f32p, c_i32p, ctypes.c_int, c_f32p]
        L.orc_path_cost.restype = ctypes.c_float
        for fn in ("orc_viterbi", "orc_tailbite", "orc_pack", "orc_unpack",
                   "orc_decode"):
            getattr(L, fn).restype = ctypes.c_int
        _LIB = L
    return _LIB


def _p(a, ct):
    return a.ctypes.data_as(ctypes.POINTER(ct))


# ------------------------------------------------------------ codebook tables
def _f16_from_bits(u):
    return np.asarray(u).astype(np.uint16).view(np.float16)


def code_lut(name: str = "exl3_mul1", L: int = 16) -> np.ndarray:
    """fp32 [2^L] decode table; restates quantize.py:56-87 step for step."""
    s = np.arange(1 << L, dtype=np.uint64)
    if name in ("exl3_3inst", "exl3_mcg"):
        if name == "exl3_3inst":
            x = (s * 89226354 + 64248484) & 0xFFFFFFFF
        else:
            x = (s * 0xCBAC1FED) & 0xFFFFFFFF
        x = (x & 0x8FFF8FFF) ^ 0x3B603B60
        lo = _f16_from_bits(x & 0xFFFF).astype(np.float64)
        hi = _f16_from_bits(x >> 16).astype(np.float64)
        return (lo + hi).astype(np.float16).astype(np.float32)
    if name == "exl3_mul1":
        x = (s * 0x83DCD12D) & 0xFFFFFFFF
        bsum = ((x & 0xFF) + ((x >> 8) & 0xFF) + ((x >> 16) & 0xFF)
                + ((x >> 24) & 0xFF))
        h = (1024 + bsum).astype(np.float64)
        inv = float(_f16_from_bits(np.array([0x1EEE]))[0])
        bias = float(_f16_from_bits(np.array([0xC931]))[0])
        return (h * inv + bias).astype(np.float16).astype(np.float32)
    if name == "qtip_1mad":
        x = (s * 34038481 + 76625530) & 0xFFFFFFFF
        y = ((x & 255) + ((x >> 8) & 255) + ((x >> 16) & 255)
             + ((x >> 24) & 255)).astype(np.float64)
        return ((y - 510.0) / 147.800537109375).astype(np.float32)
    raise KeyError(f"unknown code {name!r}")


def tensor_core_perm() -> np.ndarray:
    perm = np.empty(256, dtype=np.int32)
    lib().orc_tensor_core_perm(_p(perm, ctypes.c_int32))
    return perm


# ------------------------------------------------------------------ Viterbi
def viterbi(X: np.ndarray, lut: np.ndarray, K: int, L: int,
            overlap: np.ndarray | None = None, back_from: int | None = None,
            nthreads: int = 0) -> np.ndarray:
    """X [nseq, T] fp32 -> states [nseq, T] int32 (or [nseq] with back_from)."""
    X = np.ascontiguousarray(X, dtype=np.float32)
    lut = np.ascontiguousarray(lut, dtype=np.float32)
    nseq, T = X.shape
    assert lut.shape == (1 << L,)
    ov = None
    if overlap is not None:
        ov = np.ascontiguousarray(overlap, dtype=np.int32)
        assert ov.shape == (nseq,)
    bf = -1 if back_from is None else int(back_from)
    out = np.empty((nseq,) if bf >= 0 else (nseq, T), dtype=np.int32)
    rc = lib().orc_viterbi(_p(X, ctypes.c_float), nseq, T,
                           _p(lut, ctypes.c_float), K, L,
                           None if ov is None else _p(ov, ctypes.c_int32), bf,
                           _p(out, ctypes.c_int32), nthreads)
    if rc:
        raise RuntimeError(f"orc_viterbi rc={rc}")
    return out


def tailbite(X: np.ndarray, lut: np.ndarray, K: int, L: int = 16,
             pivot: int | None = None, margin: int = 0, nthreads: int = 0,
             return_ov: bool = False):
    """X [nseq, T] fp32 -> states [nseq, T] int32 (quantize.py:323-354)."""
    X = np.ascontiguousarray(X, dtype=np.float32)
    lut = np.ascontiguousarray(lut, dtype=np.float32)
    nseq, T = X.shape
    if pivot is None:
        pivot = T // 2
    out = np.empty((nseq, T), dtype=np.int32)
    ov = np.empty(nseq, dtype=np.int32)
    rc = lib().orc_tailbite(_p(X, ctypes.c_float), nseq, T,
                            _p(lut, ctypes.c_float), K, L, int(pivot),
                            int(margin), _p(out, ctypes.c_int32),
                            _p(ov, ctypes.c_int32), nthreads)
    if rc:
        raise RuntimeError(f"orc_tailbite rc={rc}")
    return (out, ov) if return_ov else out


def pack(states: np.ndarray, K: int) -> np.ndarray:
    st = np.ascontiguousarray(states, dtype=np.int32).reshape(-1, 256)
    out = np.empty((st.shape[0], 16 * K), dtype=np.int16)
    rc = lib().orc_pack(_p(st, ctypes.c_int32), st.shape[0], K,
                        _p(out, ctypes.c_int16))
    if rc:
        raise RuntimeError(f"orc_pack rc={rc}")
    return out


def unpack(trellis: np.ndarray, K: int) -> np.ndarray:
    tr = np.ascontiguousarray(trellis, dtype=np.int16).reshape(-1, 16 * K)
    out = np.empty((tr.shape[0], 256), dtype=np.int32)
    rc = lib().orc_unpack(_p(tr, ctypes.c_int16), tr.shape[0], K,
                          _p(out, ctypes.c_int32))
    if rc:
        raise RuntimeError(f"orc_unpack rc={rc}")
    return out


def decode(trellis: np.ndarray, lut: np.ndarray, K: int) -> np.ndarray:
    """int16 [tk, tn, 16K] -> fp32 [16 tk, 16 tn]."""
    tr = np.ascontiguousarray(trellis, dtype=np.int16)
    tk, tn, _ = tr.shape
    lut = np.ascontiguousarray(lut, dtype=np.float32)
    out = np.empty((16 * tk, 16 * tn), dtype=np.float32)
    rc = lib().orc_decode(_p(tr, ctypes.c_int16), tk, tn, K,
                          _p(lut, ctypes.c_float), _p(out, ctypes.c_float))
    if rc:
        raise RuntimeError(f"orc_decode rc={rc}")
    return out


def path_cost(x: np.ndarray, states: np.ndarray, lut: np.ndarray) -> float:
    x = np.ascontiguousarray(x, dtype=np.float32)
    st = np.ascontiguousarray(states, dtype=np.int32)
    lut = np.ascontiguousarray(lut, dtype=np.float32)
    return float(lib().orc_path_cost(_p(x, ctypes.c_float),
                                     _p(st, ctypes.c_int32), x.shape[0],
                                     _p(lut, ctypes.c_float)))


# ------------------------------------------------------ tiny-trellis brute force
def _f32(v):
    return np.float32(v)


def brute_force_viterbi(x: np.ndarray, lut: np.ndarray, K: int, L: int):
    """Exhaustive search over all state paths of a tiny trellis.

    Returns (best_cost, states) where best_cost is the minimum of the fp32
    path cost accumulated in the DP's order, and states is the path selected
    by the reference tie rule: the lowest final state among the optimal ones,
    then, walking back, the lowest predecessor index w whose exact prefix
    optimum equals the best over all predecessors (quantize.py:288-319).
    Prefix optima C_i(s) are computed by enumerating every path that ends at
    s at step i, so this never uses the DP recurrence itself.
    """
    S, NC, SP = 1 << L, 1 << K, 1 << (L - K)
    T = len(x)
    xs = [_f32(v) for v in x]
    lf = [_f32(v) for v in lut]
    # C[i][s] = min over all paths (s_0..s_i=s) of the fp32 prefix cost
    C = [[np.float32(np.inf)] * S for _ in range(T)]
    for s0 in range(S):
        for vs in itertools.product(range(NC), repeat=T - 1):
            st = s0
            d = lf[st] - xs[0]
            c = d * d
            if c < C[0][st]:
                C[0][st] = c
            for t in range(1, T):
                st = ((st << K) | vs[t - 1]) & (S - 1)
                d = lf[st] - xs[t]
                c = d * d + c
                if c < C[t][st]:
                    C[t][st] = c
    best = min(C[T - 1])
    s = min(i for i in range(S) if C[T - 1][i] == best)
    path = [0] * T
    path[T - 1] = s
    for i in range(T - 1, 0, -1):
        j = s >> K
        preds = [j + w * SP for w in range(NC)]
        pb = min(C[i - 1][p] for p in preds)
        w = min(w for w in range(NC) if C[i - 1][preds[w]] == pb)
        s = preds[w]
        path[i - 1] = s
    return float(best), np.array(path, dtype=np.int32)
