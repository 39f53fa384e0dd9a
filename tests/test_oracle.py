"""Pins of the CPU oracle (oracle/viterbi_oracle.c, oracle/oracle.py).

The oracle is only trusted as the GPU checker once it reproduces:
  * the reference's own golden vectors (tests/golden/, written from
    quantize/quantize.py on CPU by tests/golden/make_golden.py);
  * closed forms and known answers (codebook values, perm, bit layout);
  * exhaustive search on tiny trellises, including the tie rule;
  * invariants (tail-bite wrap, pack/unpack round trip, MSE bound);
and it agrees with the independent torch restatement (oracle/torch_port.py).
A planted mistake (wrong tie order, dropped roll, flipped bit order) fails
at least one of these.
"""
import itertools

import numpy as np
import pytest
import torch

from conftest import load_golden

PIVOTS = (0, 128, 147, 255)
MARGINS = (0, 16)


# --------------------------------------------------------------- codebooks
def test_mul1_known_answers(oracle_mod):
    lut = oracle_mod.code_lut("exl3_mul1")
    np.testing.assert_array_equal(
        lut[:4], np.array([-3.453125, 0.64111328125, -0.448486328125, 0.1944580078125],
                          dtype=np.float32))
    assert lut.min() == np.float32(-3.453125) and lut.max() == np.float32(3.34765625)
    assert len(np.unique(lut)) == 913
    assert abs(np.sqrt((lut.astype(np.float64) ** 2).mean()) - 1.0003120703268706) < 1e-15
    # every entry is an fp16 value (the kernels keep the table as fp16)
    assert np.array_equal(lut.astype(np.float16).astype(np.float32), lut)


def test_mul1_closed_form_fp32_path(oracle_mod):
    """The fp64 formula of the reference (quantize.py:73-81) and an fp32
    evaluation rounded once to fp16 give the same table for every byte sum."""
    lut = oracle_mod.code_lut("exl3_mul1")
    s = np.arange(65536, dtype=np.uint64)
    x = (s * 0x83DCD12D) & 0xFFFFFFFF
    bs = sum(((x >> sh) & 0xFF) for sh in (0, 8, 16, 24))
    c1 = np.float32(np.array([0x1EEE], np.uint16).view(np.float16)[0])
    c2 = np.float32(np.array([0xC931], np.uint16).view(np.float16)[0])
    v32 = (np.float32(1024) + bs.astype(np.float32)) * c1 + c2
    np.testing.assert_array_equal(v32.astype(np.float16).astype(np.float32), lut)


def test_lut_golden(oracle_mod):
    g = load_golden("lut_mul1.npz")
    np.testing.assert_array_equal(oracle_mod.code_lut("exl3_mul1"), g["lut"])


# ------------------------------------------------------------------ layout
def test_perm_known_answers(oracle_mod):
    perm = oracle_mod.tensor_core_perm()
    assert perm[:16].tolist() == [0, 16, 128, 144, 8, 24, 136, 152,
                                  32, 48, 160, 176, 40, 56, 168, 184]
    assert sorted(perm.tolist()) == list(range(256))
    np.testing.assert_array_equal(perm, load_golden("lut_mul1.npz")["perm"])


def test_pack_hand_vectors(oracle_mod):
    K = 4
    st = np.zeros((1, 256), np.int32)
    st[0, 0] = 0xB                       # symbol 1011 at stream bits 0..3
    P = oracle_mod.pack(st, K)
    # word 0 = 1011 << 28; stored low half first
    assert P[0, 0] == 0 and np.uint16(P[0, 1]) == 0xB000
    assert (P[0, 2:] == 0).all()
    ones = np.full((1, 256), (1 << K) - 1, np.int32)
    assert (oracle_mod.pack(ones, K).view(np.uint16) == 0xFFFF).all()
    # last symbol lands in the low bits of the last word's low half
    st = np.zeros((1, 256), np.int32)
    st[0, 255] = 0x5
    P = oracle_mod.pack(st, K)
    assert np.uint16(P[0, 16 * K - 2]) == 0x0005 and (P[0, :16 * K - 2] == 0).all()


@pytest.mark.parametrize("K", range(2, 8))
def test_pack_unpack_roundtrip(oracle_mod, K):
    """Random wrap-consistent state sequences survive pack -> unpack
    (the reference's own round-trip test, test_quantize.py:73-108)."""
    rng = np.random.default_rng(K)
    st = np.empty((9, 256), np.int64)
    for b in range(9):
        v = rng.integers(0, 1 << K, 256)
        s = int(rng.integers(0, 1 << 16))
        seq = [s]
        for t in range(1, 256):
            s = ((s << K) | int(v[t])) & 0xFFFF
            seq.append(s)
        wrap = seq[-1] & ((1 << (16 - K)) - 1)
        s = (wrap << K) | (seq[0] & ((1 << K) - 1))
        seq = [s]
        for t in range(1, 256):
            s = ((s << K) | int(v[t])) & 0xFFFF
            seq.append(s)
        st[b] = seq
    np.testing.assert_array_equal(oracle_mod.unpack(oracle_mod.pack(st, K), K), st)


# ------------------------------------------------------- golden (reference)
@pytest.mark.parametrize("K", range(2, 8))
def test_oracle_vs_reference_golden(oracle_mod, mul1_lut, K):
    g = load_golden("tailbite.npz")
    X = g[f"X_K{K}"]
    for m in MARGINS:
        for p in PIVOTS:
            st = oracle_mod.tailbite(X, mul1_lut, K, 16, pivot=p, margin=m)
            np.testing.assert_array_equal(st, g[f"S_K{K}_m{m}_p{p}"], err_msg=f"m={m} p={p}")
    np.testing.assert_array_equal(oracle_mod.viterbi(X, mul1_lut, K, 16), g[f"V_K{K}"])
    np.testing.assert_array_equal(
        oracle_mod.viterbi(X[:, :150], mul1_lut, K, 16, back_from=100), g[f"VB_K{K}"])
    np.testing.assert_array_equal(
        oracle_mod.viterbi(X, mul1_lut, K, 16, overlap=g[f"VPov_K{K}"]), g[f"VP_K{K}"])
    P = oracle_mod.pack(g[f"S_K{K}_m0_p128"], K)
    np.testing.assert_array_equal(P, g[f"P_K{K}"])
    np.testing.assert_array_equal(oracle_mod.unpack(P, K), g[f"U_K{K}"])
    np.testing.assert_array_equal(oracle_mod.decode(P.reshape(2, 3, 16 * K), mul1_lut, K),
                                  g[f"D_K{K}"])


TIE_CASES = ((128, 0), (147, 16), (0, 0), (255, 16))


@pytest.mark.parametrize("name", ("exl3_3inst", "exl3_mcg", "qtip_1mad"))
def test_other_code_tables_golden(oracle_mod, name):
    """The other V=1 decode tables restated by the oracle equal the
    reference's get_lut tables byte for byte (quantize.py:56-97)."""
    import hashlib
    g = load_golden("codes.npz")
    t = oracle_mod.code_lut(name)
    assert t.dtype == np.float32 and t.shape == (65536,)
    np.testing.assert_array_equal(t[:64], g[f"head_{name}"])
    assert hashlib.sha256(t.tobytes()).digest() == g[f"sha256_{name}"].tobytes()


@pytest.mark.parametrize("K", (2, 4, 7))
def test_oracle_1mad_vs_reference_golden(oracle_mod, K):
    """Tail-bite with the QTIP 1MAD table (fp32 values, not fp16-exact) on
    Gaussian and tie-forcing targets equals the reference's states."""
    g = load_golden("codes.npz")
    lut = oracle_mod.code_lut("qtip_1mad")
    X = g[f"mad_X_K{K}"]
    for p, m in ((128, 0), (147, 16)):
        np.testing.assert_array_equal(oracle_mod.tailbite(X, lut, K, 16, pivot=p, margin=m),
                                      g[f"mad_S_K{K}_m{m}_p{p}"], err_msg=f"p={p} m={m}")


@pytest.mark.parametrize("K", range(2, 8))
def test_oracle_vs_reference_ties(oracle_mod, mul1_lut, K):
    """The reference's outputs on 24 tie-forcing sequences per K (ties.npz):
    the C oracle and the torch restatement reproduce every state."""
    import torch
    from oracle import torch_port
    g = load_golden("ties.npz")
    X = g[f"X_K{K}"]
    for p, m in TIE_CASES:
        want = g[f"S_K{K}_m{m}_p{p}"]
        np.testing.assert_array_equal(oracle_mod.tailbite(X, mul1_lut, K, 16, pivot=p, margin=m),
                                      want, err_msg=f"oracle m={m} p={p}")
        got = torch_port.tailbite(torch.from_numpy(X.T.copy()), torch.from_numpy(mul1_lut), K,
                                  16, pivot=p, margin=m).t().numpy()
        np.testing.assert_array_equal(got, want, err_msg=f"torch port m={m} p={p}")
    np.testing.assert_array_equal(
        oracle_mod.viterbi(X, mul1_lut, K, 16, overlap=g[f"VPov_K{K}"]), g[f"VP_K{K}"])
    np.testing.assert_array_equal(
        oracle_mod.viterbi(X[:, :200], mul1_lut, K, 16, back_from=60), g[f"VB_K{K}"])


@pytest.mark.parametrize("K", (2, 4, 7))
def test_ties_fixture_pins_the_tie_rule(mul1_lut, K):
    """A planted 'last index wins' rule (the torch restatement with the
    candidate order reversed in every min and in the final argmin) changes
    most tie-forcing sequences of the fixture: the fixture pins the first-index
    rule at L=16 on its own."""
    import torch
    g = load_golden("ties.npz")
    X = torch.from_numpy(g[f"X_K{K}"].T.copy())
    lut = torch.from_numpy(mul1_lut)
    S, NC, SP = 1 << 16, 1 << K, 1 << (16 - K)
    T, B = X.shape

    def last_index_viterbi(x):
        def emit(i):
            return (lut.view(1, S) - x[i].unsqueeze(-1)).square()
        cost = emit(0)
        bps = []
        for i in range(1, T):
            rev = cost.view(B, NC, SP).flip(1).min(dim=1)
            bps.append(NC - 1 - rev.indices)
            e = emit(i)
            e.view(B, SP, NC).add_(rev.values.unsqueeze(-1))
            cost = e
        s = S - 1 - cost.flip(1).argmin(dim=1)
        st = [s]
        for i in range(T - 1, 0, -1):
            j = s >> K
            s = j + bps[i - 1].gather(1, j.unsqueeze(1)).squeeze(1) * SP
            st.append(s)
        return torch.stack(st[::-1]).t().numpy()

    planted = last_index_viterbi(X)
    from oracle import torch_port
    want = torch_port.viterbi(X, lut, K, 16).t().numpy()
    differ = int((planted != want).any(axis=1).sum())
    print(f"K={K}: the planted rule changes {differ} of {B} sequences")
    assert differ >= 10, f"only {differ} of {B} sequences separate the tie rules"


# ------------------------------------------------------------- brute force
@pytest.mark.parametrize("L,K,T,seed", [(4, 2, 6, 1), (4, 1, 7, 2), (6, 2, 5, 3),
                                        (6, 3, 4, 4)])
def test_brute_force_random(oracle_mod, L, K, T, seed):
    """Tiny trellises: the DP optimum, and the exact path chosen by the tie
    rule, equal exhaustive search (test_quantize.py:111-138 pins only cost)."""
    rng = np.random.default_rng(seed)
    lut = rng.standard_normal(1 << L).astype(np.float32)
    X = rng.standard_normal((3, T)).astype(np.float32)
    st = oracle_mod.viterbi(X, lut, K, L)
    for q in range(3):
        best, path = oracle_mod.brute_force_viterbi(X[q], lut, K, L)
        assert oracle_mod.path_cost(X[q], st[q], lut) == np.float32(best)
        np.testing.assert_array_equal(st[q], path)


@pytest.mark.parametrize("L,K,T,seed", [(4, 2, 6, 5), (6, 2, 5, 6), (6, 3, 4, 7)])
def test_brute_force_ties(oracle_mod, L, K, T, seed):
    """Tie-heavy tiny trellises: duplicated codebook values and targets on
    the codebook make many exactly equal path costs; the oracle must still
    pick the reference's path (lowest final state, lowest predecessor)."""
    rng = np.random.default_rng(seed)
    vals = np.array([-1.0, 0.0, 0.5, 1.0], np.float32)
    lut = vals[rng.integers(0, 4, 1 << L)]
    X = vals[rng.integers(0, 4, (4, T))]
    st = oracle_mod.viterbi(X, lut, K, L)
    for q in range(4):
        best, path = oracle_mod.brute_force_viterbi(X[q], lut, K, L)
        np.testing.assert_array_equal(st[q], path)


def test_brute_force_detects_wrong_tie_rule(oracle_mod):
    """A planted 'last index wins' tie rule disagrees with the brute-force
    path on a tie-heavy case (so the brute force really pins the rule)."""
    L, K, T = 4, 2, 5
    lut = np.zeros(1 << L, np.float32)
    X = np.zeros((1, T), np.float32)
    best, path = oracle_mod.brute_force_viterbi(X[0], lut, K, L)
    assert (path == 0).all()                   # all ties -> lowest everywhere
    st = oracle_mod.viterbi(X, lut, K, L)
    np.testing.assert_array_equal(st[0], path)


# -------------------------------------------------------------- invariants
@pytest.mark.parametrize("K", (2, 4, 7))
def test_tailbite_wrap_invariant(oracle_mod, mul1_lut, K):
    X = np.random.default_rng(2).standard_normal((4, 256)).astype(np.float32)
    st = oracle_mod.tailbite(X, mul1_lut, K, 16)
    SP = 1 << (16 - K)
    assert ((st[:, 0] >> K) == (st[:, -1] & (SP - 1))).all()
    np.testing.assert_array_equal(oracle_mod.unpack(oracle_mod.pack(st, K), K), st)


@pytest.mark.parametrize("K", (2, 4))
@pytest.mark.parametrize("code", ("exl3_mul1", "qtip_1mad"))
def test_gaussian_mse_bound(oracle_mod, code, K):
    """MSE < 3 * 2^-2K on rms-matched Gaussian targets, for both codes
    (test_quantize.py:183-202)."""
    lut = oracle_mod.code_lut(code)
    rng = np.random.default_rng(3)
    X = rng.standard_normal((16, 256)).astype(np.float32)
    lut_rms = np.sqrt((lut.astype(np.float64) ** 2).mean())
    X = (X / np.sqrt((X.astype(np.float64) ** 2).mean()) * lut_rms).astype(np.float32)
    st = oracle_mod.tailbite(X, lut, K, 16)
    mse = ((lut[st] - X) ** 2).mean() / (X ** 2).mean()
    assert mse < 3.0 * 2.0 ** (-2 * K)


def test_torch_port_agrees(oracle_mod, mul1_lut):
    from oracle import torch_port
    X = np.random.default_rng(9).standard_normal((3, 256)).astype(np.float32)
    X[1] = mul1_lut[np.random.default_rng(10).integers(0, 65536, 256)]
    for K, p, m in ((3, 128, 0), (5, 147, 16), (7, 0, 16)):
        want = oracle_mod.tailbite(X, mul1_lut, K, 16, pivot=p, margin=m)
        got = torch_port.tailbite(torch.from_numpy(X.T.copy()), torch.from_numpy(mul1_lut),
                                  K, 16, pivot=p, margin=m).t().numpy()
        np.testing.assert_array_equal(got, want)


def test_margin_truncation_changes_nothing_past_window(oracle_mod, mul1_lut):
    """margin >= 256 - pivot runs the full pass 1 (quantize.py:344-351)."""
    X = np.random.default_rng(12).standard_normal((3, 256)).astype(np.float32)
    a = oracle_mod.tailbite(X, mul1_lut, 4, 16, pivot=200, margin=56)
    b = oracle_mod.tailbite(X, mul1_lut, 4, 16, pivot=200, margin=0)
    np.testing.assert_array_equal(a, b)
