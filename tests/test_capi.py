"""The C-ABI library loads on any host, exports every symbol declared in
include/exl3_vit.h, and rejects invalid arguments with the documented status
codes before touching a device (quantize/viterbi_esimd.cpp:970-1005 codes)."""
import ctypes
import os
import re
import subprocess

import numpy as np
import pytest

from conftest import PKG, ROOT, load_golden

HEADER = os.path.join(ROOT, "include", "exl3_vit.h")


@pytest.fixture(scope="module")
def lib():
    so = os.path.join(PKG, "lib", "libexl3vit.so")
    if not os.path.exists(so):
        subprocess.run(["make", "-s", "-C", PKG], check=True)
    import hip_backend
    return hip_backend.lib()


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(xtq_\w+)\s*\(", text)))


def test_exports_every_declared_symbol(lib):
    names = declared_functions()
    assert len(names) >= 11
    for name in names:
        assert hasattr(lib, name), name
    out = subprocess.run(["nm", "-D", "--defined-only", os.path.join(PKG, "lib", "libexl3vit.so")],
                         capture_output=True, text=True, check=True).stdout
    for name in names:
        assert re.search(rf"\bT {name}\b", out), name


def test_lut_export(lib):
    out = np.empty(65536, np.float32)
    assert lib.xtq_vit_get_lut(b"mul1", out.ctypes.data_as(ctypes.c_void_p)) == 0
    np.testing.assert_array_equal(out, load_golden("lut_mul1.npz")["lut"])
    assert lib.xtq_vit_get_lut(b"ih2x2", out.ctypes.data_as(ctypes.c_void_p)) == 8
    # the other codes' device tables equal the reference's get_lut tables
    import hashlib
    g = load_golden("codes.npz")
    for short, name in (("3inst", "exl3_3inst"), ("mcg", "exl3_mcg"), ("1mad", "qtip_1mad"),
                        ("qtip_1mad", "qtip_1mad")):
        assert lib.xtq_vit_get_lut(short.encode(), out.ctypes.data_as(ctypes.c_void_p)) == 0
        assert hashlib.sha256(out.tobytes()).digest() == g[f"sha256_{name}"].tobytes(), short


def test_status_codes_without_device(lib):
    X = np.zeros((2, 256), np.float32)
    st = np.zeros((2, 256), np.int32)
    xp = X.ctypes.data_as(ctypes.c_void_p)
    sp = st.ctypes.data_as(ctypes.c_void_p)
    assert lib.xtq_vit_run(xp, 2, b"ih2x2", 0, 128, sp) == 8
    assert lib.xtq_vit_run(xp, 2, b"bogus", 0, 128, sp) == 8
    assert lib.xtq_vit_run(None, 2, b"mul1p", 0, 128, sp) == 12
    assert lib.xtq_vit_run(xp, 0, b"mul1p", 0, 128, sp) == 6
    assert lib.xtq_vit_run(xp, 2, b"mul1p", 0, 256, sp) == 10
    assert lib.xtq_vit_run(xp, 2, b"mul1p", 0, -1, sp) == 10
    assert lib.xtq_vit_run_k(xp, 2, 4, b"mul1", -1, 0, sp) == 10
    assert lib.xtq_vit_run_k(xp, 2, 8, b"mul1", 0, 0, sp) == 9
    assert lib.xtq_vit_run_k(xp, 2, 1, b"mul1", 0, 0, sp) == 9
    fake = ctypes.c_void_p(16)          # never dereferenced: rejected first
    assert lib.xtq_vit_tailbite_dev(fake, 4, 9, b"mul1", 0, 0, fake, None, None) == 9
    assert lib.xtq_vit_tailbite_dev(fake, 4, 4, b"mul1", 0, 300, fake, None, None) == 10
    assert lib.xtq_vit_tailbite_dev(fake, 4, 4, b"mul1", 0, 0, None, None, None) == 12
    assert lib.xtq_vit_tailbite_dev(fake, 4, 4, b"qtip", 0, 0, fake, None, None) == 8
    assert lib.xtq_vit_tailbite_dev_async(fake, 4, 9, b"mul1", 0, 0, fake, None, None) == 9
    assert lib.xtq_vit_tailbite_dev_async(fake, 0, 4, b"mul1", 0, 0, fake, None, None) == 6
    assert lib.xtq_vit_tailbite_dev_async(None, 4, 4, b"mul1", 0, 0, fake, None, None) == 12
    assert lib.xtq_vit_viterbi_dev(fake, 4, 300, 4, b"mul1", None, -1, fake, None) == 10
    assert lib.xtq_vit_viterbi_dev(fake, 4, 256, 4, b"mul1", None, 256, fake, None) == 10
    assert lib.xtq_trellis_decode_dev(fake, 1, 1, 8, b"mul1", fake, None, None) == 9
    assert lib.xtq_trellis_pack_dev(fake, 1, 3, None, None) == 12
    ch = lib.xtq_ldlq_chain_dev
    mis = ctypes.c_void_p(20)           # not 16-byte aligned
    assert ch(fake, fake, 64, 64, 8, b"mul1", 0, 128, 128, fake, None, fake, None, None) == 9
    assert ch(fake, fake, 64, 64, 4, b"mul1", 0, 256, 128, fake, None, fake, None, None) == 10
    assert ch(fake, fake, 64, 64, 4, b"qtip", 0, 128, 128, fake, None, fake, None, None) == 8
    assert ch(None, fake, 64, 64, 4, b"mul1", 0, 128, 128, fake, None, fake, None, None) == 12
    assert ch(fake, fake, 64, 64, 4, b"mul1", 0, 128, 128, fake, None, None, None, None) == 12
    assert ch(fake, mis, 64, 64, 4, b"mul1", 0, 128, 128, fake, None, fake, None, None) == 12
    assert ch(fake, fake, 72, 64, 4, b"mul1", 0, 128, 128, fake, None, fake, None, None) == 6
    assert ch(fake, None, 64, 0, 4, b"mul1", 0, 128, 128, fake, None, fake, None, None) == 6
    assert ch(fake, None, 64, 64, 4, b"mul1", 0, 128, 24, fake, None, fake, None, None) == 6
    assert ch(fake, None, 64, 64, 4, b"mul1", 0, 128, 0, fake, None, fake, None, None) == 6
    chm = lib.xtq_ldlq_chain_multi_dev
    i2 = (ctypes.c_int * 2)
    tp2 = (ctypes.c_void_p * 2)(16, 16)
    tp1 = (ctypes.c_void_p * 2)(16, None)
    args = (b"mul1", 0, 128, 128, fake, None)
    assert chm(fake, None, 64, 64, 2, i2(32, 32), i2(4, 9), *args, tp2, None, None) == 9
    assert chm(fake, None, 64, 64, 2, i2(32, 24), i2(4, 7), *args, tp2, None, None) == 6
    assert chm(fake, None, 64, 64, 2, i2(32, 16), i2(4, 7), *args, tp2, None, None) == 6
    assert chm(fake, None, 64, 64, 0, i2(64, 0), i2(4, 7), *args, tp2, None, None) == 6
    assert chm(fake, None, 64, 64, 9, i2(32, 32), i2(4, 7), *args, tp2, None, None) == 6
    assert chm(fake, None, 64, 64, 2, i2(32, 32), i2(4, 7), *args, tp1, None, None) == 12
    assert chm(fake, None, 64, 64, 2, None, i2(4, 7), *args, tp2, None, None) == 12
    # block-128 Hadamard entries: pointers and shapes are checked before any launch
    fake2 = ctypes.c_void_p(48)
    hl, hr = lib.xtq_had128_left_dev, lib.xtq_had128_right_dev
    assert hl(None, fake, fake2, 128, 64, None) == 12
    assert hl(fake, fake, fake, 128, 64, None) == 12          # in place
    assert hl(fake, fake, fake2, 100, 64, None) == 6          # rows not a multiple of 128
    assert hl(fake, fake, fake2, 128, 0, None) == 6
    assert hr(fake, None, fake2, 64, 128, None) == 12
    assert hr(fake, fake, fake, 64, 128, None) == 12          # in place
    assert hr(fake, fake, fake2, 64, 100, None) == 6          # cols not a multiple of 128
    assert hr(fake, fake, fake2, 0, 128, None) == 6
    assert hr(fake, fake, fake2, 2_097_121, 128, None) == 6   # one row past the documented maximum
    assert lib.xtq_vit_strerror(11) == b"NaN target"
    assert lib.xtq_vit_strerror(13) == b"synchronous entry given a stream under graph capture"
    assert lib.xtq_vit_strerror(99) == b"unknown status"


def test_host_entry_bounds(lib, monkeypatch):
    """xtq_vit_run keeps the reference's bounds and their order
    (viterbi_esimd.cpp:924-933,973-982): nseq <= XTQ_VIT_MAXSEQ (default
    4096) else 6, then nseq * 1,317,888 B <= XTQ_VIT_MAXBYTES (default 6 GiB)
    else 5, both read on every call; all before any device work."""
    for v in ("XTQ_VIT_MAXSEQ", "XTQ_VIT_MAXBYTES"):
        monkeypatch.delenv(v, raising=False)
    X = np.zeros((1, 256), np.float32)
    st = np.zeros((1, 256), np.int32)
    xp = X.ctypes.data_as(ctypes.c_void_p)
    sp = st.ctypes.data_as(ctypes.c_void_p)
    assert lib.xtq_vit_run(xp, 4097, b"mul1p", 0, 128, sp) == 6
    assert lib.xtq_vit_run_k(xp, 4097, 4, b"mul1", 0, 128, sp) == 6
    assert lib.xtq_vit_run(xp, -3, b"mul1p", 0, 128, sp) == 6
    monkeypatch.setenv("XTQ_VIT_MAXSEQ", "100000")
    # 5000 * 1,317,888 B = 6.14 GiB > 6 GiB
    assert lib.xtq_vit_run(xp, 5000, b"mul1p", 0, 128, sp) == 5
    monkeypatch.setenv("XTQ_VIT_MAXBYTES", str(1317888 * 3 - 1))
    assert lib.xtq_vit_run(xp, 3, b"mul1p", 0, 128, sp) == 5
    monkeypatch.setenv("XTQ_VIT_MAXSEQ", "2")
    assert lib.xtq_vit_run(xp, 3, b"mul1p", 0, 128, sp) == 6      # 6 is checked first


def test_probe_library_is_separate(lib):
    """The VALU probe is a benchmark helper in its own library: the encoder
    library exports no probe symbol, the probe library rejects bad input."""
    out = subprocess.run(["nm", "-D", "--defined-only", os.path.join(PKG, "lib", "libexl3vit.so")],
                         capture_output=True, text=True, check=True).stdout
    assert "xtq_valu_probe" not in out
    sys_path = os.path.join(PKG, "probe")
    import sys
    if sys_path not in sys.path:
        sys.path.insert(0, sys_path)
    import valu_probe
    pl = valu_probe.lib()
    v = ctypes.c_double()
    assert pl.xtq_valu_probe(13, ctypes.byref(v)) == 8
    assert pl.xtq_valu_probe(-1, ctypes.byref(v)) == 8
    assert pl.xtq_valu_probe(0, None) == 12


def test_scratch_sizes(lib):
    per = [lib.xtq_vit_scratch_per_seq(k) for k in range(2, 8)]
    # 255 stored steps x (backpointer bytes per step)
    assert per == [255 * 4096, 255 * 4096, 255 * 2048, 255 * 2048, 255 * 1024, 255 * 512]
    assert lib.xtq_vit_scratch_per_seq(8) == -1
