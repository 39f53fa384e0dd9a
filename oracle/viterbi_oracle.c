/*
 * viterbi_oracle.c -- CPU restatement of the reference trellis Viterbi path.
 *
 * TEST INFRASTRUCTURE ONLY.  Nothing in the product (the HIP library or the
 * Python host package) may link, load or call this file; only tests/, the
 * smoke check and the benchmark's CPU-baseline leg use it, as the checker.
 *
 * It restates, in scalar C with IEEE fp32 arithmetic and no FMA contraction,
 * the torch implementation that defines the bit-exact contract:
 *   quantize/quantize.py:218-320  viterbi()              (one DP run)
 *   quantize/quantize.py:323-354  quantize_seq_tailbite() (two-pass QTIP wrap)
 *   quantize/quantize.py:360-378  pack_states()
 *   quantize/quantize.py:381-402  unpack_states()
 *   quantize/quantize.py:405-415  decode_trellis()
 *   quantize/quantize.py:101-118  tensor_core_perm()
 * The state width L is a parameter so that tiny trellises (L=4..8) can be
 * checked against exhaustive search.  V (states per symbol) is 1 throughout:
 * the mul1 code the path covers is a V=1 code.
 *
 * Semantics kept from the reference (each line cites where it comes from):
 *   emit      e[s] = fl(fl(lut[s] - x)^2)                     quantize.py:257
 *   step      c_i[s] = fl(e_i[s] + b_i[s >> K])                quantize.py:293-295
 *   reduce    b_i[j] = min_w c_{i-1}[j + w*SP], first w wins   quantize.py:288-292
 *   pins      +inf masks on the first and last step            quantize.py:265-270,298-303
 *   argmin    lowest state index among equal minima            quantize.py:306,315
 *   backtrace s_{i-1} = (s_i >> K) + bp_i[s_i >> K] * SP       quantize.py:316-319
 *
 * Build: see oracle/Makefile (gcc -O3 -mavx2 -ffp-contract=off, no fast-math:
 * vectorised, but every element sees the same IEEE fp32 operations).
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#ifdef _OPENMP
#include <omp.h>
#endif

#define ORC_OK 0
#define ORC_EARG 1
#define ORC_ENOMEM 2

/*
 * One DP step: bn[j] = b_i[j] = min_w c_{i-1}[j + w*SP] and bw[j] = the
 * first w attaining it, where
 *   c_{i-1}[s] = fl(fl(fl(lut[s] - xp)^2) + b[s >> K])
 * and (j + w*SP) >> K = (j >> K) + w*Q; the first w wins ties (ascending w,
 * only a strictly smaller cost replaces).  Blocks of groups stay in L1; the
 * innermost loop runs over the NC groups sharing one predecessor minimum,
 * so it vectorises with that minimum broadcast.  dp_step_k is instantiated
 * for K >= 4 so the innermost trip count is a constant.
 */
static inline __attribute__((always_inline)) void
dp_step_k(const int K, const int L, const float *lut, const float *b, float xp,
          float *bn, int32_t *bw)
{
    const int NC = 1 << K, SP = 1 << (L - K), Q = SP >> K;
    enum { JB = 256 };
    for (int j0 = 0; j0 < SP; j0 += JB) {
        const int jn = SP - j0 < JB ? SP - j0 : JB;
        float *bb = bn + j0;
        int32_t *ww = bw + j0;
        for (int a = 0; a < (jn >> K); ++a) {       /* w = 0 */
            const float pb = b[(j0 >> K) + a];
            const float *lw = lut + j0 + (a << K);
            for (int r = 0; r < NC; ++r) {
                float d = lw[r] - xp;
                float e = d * d;
                bb[(a << K) + r] = e + pb;
                ww[(a << K) + r] = 0;
            }
        }
        for (int w = 1; w < NC; ++w) {
            const float *lw = lut + (size_t)w * SP + j0;
            const float *bp = b + (size_t)w * Q + (j0 >> K);
            for (int a = 0; a < (jn >> K); ++a) {
                const float pb = bp[a];
                float *bq = bb + (a << K);
                int32_t *wq = ww + (a << K);
                const float *lq = lw + (a << K);
                for (int r = 0; r < NC; ++r) {
                    float d = lq[r] - xp;
                    float e = d * d;
                    float v = e + pb;
                    const int lt = v < bq[r];
                    bq[r] = lt ? v : bq[r];
                    wq[r] = lt ? w : wq[r];
                }
            }
        }
    }
}

static void dp_step(int K, int L, const float *lut, const float *b, float xp,
                    float *bn, int32_t *bw)
{
    if (L == 16) {
        switch (K) {
        case 4: dp_step_k(4, 16, lut, b, xp, bn, bw); return;
        case 5: dp_step_k(5, 16, lut, b, xp, bn, bw); return;
        case 6: dp_step_k(6, 16, lut, b, xp, bn, bw); return;
        case 7: dp_step_k(7, 16, lut, b, xp, bn, bw); return;
        case 8: dp_step_k(8, 16, lut, b, xp, bn, bw); return;
        default: break;
        }
    }
    /* K = 2, 3 (their short innermost loops vectorise better with a
     * run-time trip count) and the small test trellises */
    dp_step_k(K, L, lut, b, xp, bn, bw);
}

/* ---------------------------------------------------------------- one run */
/*
 * One Viterbi run over x[0..T-1] on the 2^L-state shift-register trellis,
 * K bits per step (quantize.py:218-320 with V=1, emit_mode="sq").
 *   overlap  <0: free start and end; otherwise pin s_0>>K == overlap and
 *            s_{T-1} mod 2^(L-K) == overlap (quantize.py:265-270,298-303).
 *   back_from <0: full traceback into states[0..T-1];
 *            otherwise keep links only for steps > back_from and return the
 *            state at step back_from in states[0] (quantize.py:305-312).
 * Scratch is passed in so batch drivers can reuse it per thread.
 */
static __attribute__((noinline)) int
viterbi_run(const float *x, int T, const float *lut, int K, int L, int overlap,
            int back_from, int32_t *states, float *cost, float *best, int32_t *bw,
            uint8_t *from_state)
{
    const int S = 1 << L, SP = 1 << (L - K);
    const float INF = INFINITY;
    /* b holds the group minima b_i (SP floats), cost doubles as the buffer
     * of b_{i+1} while it is being formed, and finally holds c_{T-1}.
     * b_0 is the start mask: 0 (free) or 0 / +inf (pinned to overlap), so
     * c_0[s] = fl(e_0[s] + b_0[s >> K]) is e_0[s] or +inf, as the
     * reference's e + m (quantize.py:264-270). */
    float *b = best, *bn = cost;
    for (int g = 0; g < SP; ++g)
        b[g] = (overlap < 0 || g == overlap) ? 0.0f : INF;
    for (int i = 1; i < T; ++i) {
        int keep = (back_from < 0) || (i > back_from);
        uint8_t *fs = NULL;
        if (keep)
            fs = from_state + (size_t)(back_from < 0 ? i : i - 1 - back_from) * SP;
        const float xp = x[i - 1];
        dp_step(K, L, lut, b, xp, bn, bw);
        if (fs)
            for (int j = 0; j < SP; ++j) fs[j] = (uint8_t)bw[j];
        float *t = b; b = bn; bn = t;
    }
    /* c_{T-1}[s] = fl(e_{T-1}[s] + b_{T-1}[s >> K]) (+ the pinned end mask,
     * quantize.py:298-303), then the lowest index among the minima. */
    const float xl = x[T - 1];
    int am = 0;
    float mv = 0.0f;
    for (int s = 0; s < S; ++s) {
        float d = lut[s] - xl;
        float e = d * d;
        float v = e + b[s >> K];
        if (overlap >= 0)
            v = v + (((s & (SP - 1)) == overlap) ? 0.0f : INF);
        if (s == 0 || v < mv) { mv = v; am = s; }
    }
    if (back_from >= 0) {
        int s = am;
        for (int i = T - 1; i > back_from; --i) {
            int j = s >> K;
            int w = from_state[(size_t)(i - 1 - back_from) * SP + j];
            s = j + w * SP;
        }
        states[0] = s;
        return ORC_OK;
    }
    states[T - 1] = am;
    for (int i = T - 1; i > 0; --i) {
        int j = states[i] >> K;
        int w = from_state[(size_t)i * SP + j];
        states[i - 1] = j + w * SP;
    }
    return ORC_OK;
}

static int check_args(int T, int K, int L)
{
    if (L < 2 || L > 16 || K < 1 || 2 * K > L || K > 8 || T < 1 || T > 4096)
        return ORC_EARG;
    return ORC_OK;
}

/* Scratch for one sequence: cost S + best SP floats, from_state T*SP bytes. */
typedef struct { float *cost, *best; int32_t *bw; uint8_t *fs; int32_t *tmp; } scratch_t;

static int scratch_alloc(scratch_t *w, int T, int L, int K)
{
    const int S = 1 << L, SP = 1 << (L - K);
    w->cost = (float *)malloc(sizeof(float) * S);
    w->best = (float *)malloc(sizeof(float) * SP);
    w->bw = (int32_t *)malloc(sizeof(int32_t) * SP);
    w->fs = (uint8_t *)malloc((size_t)T * SP);
    w->tmp = (int32_t *)malloc(sizeof(int32_t) * T);
    if (!w->cost || !w->best || !w->bw || !w->fs || !w->tmp) return ORC_ENOMEM;
    return ORC_OK;
}

static void scratch_free(scratch_t *w)
{
    free(w->cost); free(w->best); free(w->bw); free(w->fs); free(w->tmp);
}

/*
 * Public: batch of independent Viterbi runs, X [nseq][T] -> states.
 * overlap may be NULL (free) or [nseq].  With back_from >= 0, out is [nseq].
 */
int orc_viterbi(const float *X, int nseq, int T, const float *lut, int K, int L,
                const int32_t *overlap, int back_from, int32_t *out,
                int nthreads)
{
    int rc = check_args(T, K, L);
    if (rc) return rc;
    if (back_from >= T) return ORC_EARG;
    int err = 0;
#ifdef _OPENMP
    if (nthreads <= 0) nthreads = omp_get_max_threads();
    #pragma omp parallel num_threads(nthreads) reduction(| : err)
#endif
    {
        scratch_t w;
        if (scratch_alloc(&w, T, L, K)) {
            err |= ORC_ENOMEM;
        } else {
#ifdef _OPENMP
            #pragma omp for schedule(dynamic, 1)
#endif
            for (int q = 0; q < nseq; ++q) {
                int ov = overlap ? overlap[q] : -1;
                int32_t *o = back_from >= 0 ? out + q : out + (size_t)q * T;
                viterbi_run(X + (size_t)q * T, T, lut, K, L, ov, back_from, o,
                            w.cost, w.best, w.bw, w.fs);
            }
        }
        scratch_free(&w);
    }
    (void)nthreads;
    return err;
}

/*
 * Public: QTIP tail-biting Viterbi (quantize.py:323-354), X [nseq][T] ->
 * states [nseq][T].  pivot in [0,T); margin >= 0.  Pass 1 runs free on the
 * sequence rolled right by pivot (torch.roll(X, pivot)), truncated to
 * pivot+margin steps when 0 < margin and pivot+margin < T; the wrap bits are
 * ov = s_pivot >> K; pass 2 runs pinned to ov on the unrolled sequence.
 * If ov_out is non-NULL it receives the per-sequence ov.
 */
int orc_tailbite(const float *X, int nseq, int T, const float *lut, int K,
                 int L, int pivot, int margin, int32_t *out, int32_t *ov_out,
                 int nthreads)
{
    int rc = check_args(T, K, L);
    if (rc) return rc;
    if (pivot < 0 || pivot >= T || margin < 0) return ORC_EARG;
    int err = 0;
#ifdef _OPENMP
    if (nthreads <= 0) nthreads = omp_get_max_threads();
    #pragma omp parallel num_threads(nthreads) reduction(| : err)
#endif
    {
        scratch_t w;
        float *roll = (float *)malloc(sizeof(float) * T);
        if (scratch_alloc(&w, T, L, K) || !roll) {
            err |= ORC_ENOMEM;
        } else {
#ifdef _OPENMP
            #pragma omp for schedule(dynamic, 1)
#endif
            for (int q = 0; q < nseq; ++q) {
                const float *x = X + (size_t)q * T;
                for (int t = 0; t < T; ++t)
                    roll[t] = x[((t - pivot) % T + T) % T];
                int s_p;
                if (margin > 0 && pivot + margin < T) {
                    int32_t sp1;
                    viterbi_run(roll, pivot + margin, lut, K, L, -1, pivot,
                                &sp1, w.cost, w.best, w.bw, w.fs);
                    s_p = sp1;
                } else {
                    viterbi_run(roll, T, lut, K, L, -1, -1, w.tmp, w.cost,
                                w.best, w.bw, w.fs);
                    s_p = w.tmp[pivot];
                }
                int ov = s_p >> K;
                if (ov_out) ov_out[q] = ov;
                viterbi_run(x, T, lut, K, L, ov, -1, out + (size_t)q * T,
                            w.cost, w.best, w.bw, w.fs);
            }
        }
        free(roll);
        scratch_free(&w);
    }
    (void)nthreads;
    return err;
}

/* -------------------------------------------------- tile <-> sequence layout */
/* tensor_core_perm (quantize.py:101-118): element t -> row-major 16x16 index. */
void orc_tensor_core_perm(int32_t *perm)
{
    for (int t = 0; t < 32; ++t) {
        int r0 = (t % 4) * 2, c0 = t / 4;
        int r1 = r0 + 1, r2 = r0 + 8, r3 = r0 + 9, c1 = c0 + 8;
        perm[t * 8 + 0] = r0 * 16 + c0;
        perm[t * 8 + 1] = r1 * 16 + c0;
        perm[t * 8 + 2] = r2 * 16 + c0;
        perm[t * 8 + 3] = r3 * 16 + c0;
        perm[t * 8 + 4] = r0 * 16 + c1;
        perm[t * 8 + 5] = r1 * 16 + c1;
        perm[t * 8 + 6] = r2 * 16 + c1;
        perm[t * 8 + 7] = r3 * 16 + c1;
    }
}

/*
 * pack_states (quantize.py:360-378): states [nt][256] -> int16 [nt][16K].
 * Symbol v_t = s_t mod 2^K occupies stream bits [tK, (t+1)K), MSB first;
 * stream bit b lives in 32-bit word b/32 at bit 31-(b%32); each word is
 * stored as two int16 halves, low half first.
 */
int orc_pack(const int32_t *states, int nt, int K, int16_t *out)
{
    if (K < 1 || K > 8) return ORC_EARG;
    const int nwords = 8 * K;              /* 256*K bits / 32 */
    for (int q = 0; q < nt; ++q) {
        const int32_t *s = states + (size_t)q * 256;
        uint32_t words[64];
        memset(words, 0, sizeof(words));
        for (int t = 0; t < 256; ++t) {
            uint32_t v = (uint32_t)s[t] & ((1u << K) - 1u);
            for (int k = 0; k < K; ++k) {
                uint32_t bit = (v >> (K - 1 - k)) & 1u;
                int b = t * K + k;
                words[b >> 5] |= bit << (31 - (b & 31));
            }
        }
        int16_t *o = out + (size_t)q * 16 * K;
        for (int wd = 0; wd < nwords; ++wd) {
            o[2 * wd] = (int16_t)(uint16_t)(words[wd] & 0xFFFFu);
            o[2 * wd + 1] = (int16_t)(uint16_t)(words[wd] >> 16);
        }
    }
    return ORC_OK;
}

/*
 * unpack_states (quantize.py:381-402): s_t = the 16-bit circular window of
 * the stream whose last bit is stream bit (t+1)K-1 (window start
 * (tK + K - 16) mod 256K), read MSB first.
 */
int orc_unpack(const int16_t *trellis, int nt, int K, int32_t *states)
{
    if (K < 1 || K > 8) return ORC_EARG;
    const int nbits = 256 * K;
    for (int q = 0; q < nt; ++q) {
        const int16_t *tr = trellis + (size_t)q * 16 * K;
        uint32_t words[64];
        for (int wd = 0; wd < 8 * K; ++wd)
            words[wd] = ((uint32_t)(uint16_t)tr[2 * wd]) |
                        ((uint32_t)(uint16_t)tr[2 * wd + 1] << 16);
        for (int t = 0; t < 256; ++t) {
            int b0 = ((t * K + K - 16) % nbits + nbits) % nbits;
            uint32_t v = 0;
            for (int k = 0; k < 16; ++k) {
                int b = (b0 + k) % nbits;
                uint32_t bit = (words[b >> 5] >> (31 - (b & 31))) & 1u;
                v = (v << 1) | bit;
            }
            states[(size_t)q * 256 + t] = (int32_t)v;
        }
    }
    return ORC_OK;
}

/*
 * decode_trellis (quantize.py:405-415): int16 [tk][tn][16K] -> fp32 [k][n]
 * with W[16a+r][16b+c] = lut[s_t] where perm[t] = 16r + c.
 */
int orc_decode(const int16_t *trellis, int tk, int tn, int K, const float *lut,
               float *out)
{
    if (K < 1 || K > 8 || tk <= 0 || tn <= 0) return ORC_EARG;
    int32_t perm[256];
    orc_tensor_core_perm(perm);
    int32_t st[256];
    const int n = tn * 16;
    for (int a = 0; a < tk; ++a)
        for (int b = 0; b < tn; ++b) {
            orc_unpack(trellis + ((size_t)a * tn + b) * 16 * K, 1, K, st);
            for (int t = 0; t < 256; ++t) {
                int r = perm[t] >> 4, c = perm[t] & 15;
                out[(size_t)(16 * a + r) * n + 16 * b + c] = lut[st[t]];
            }
        }
    return ORC_OK;
}

/*
 * Path cost of a state sequence in the DP's own accumulation order:
 * c = e_0; c = fl(e_t + c) for t = 1..T-1 (quantize.py:264,293-295).
 */
float orc_path_cost(const float *x, const int32_t *states, int T,
                    const float *lut)
{
    float c = 0.0f;
    for (int t = 0; t < T; ++t) {
        float d = lut[states[t]] - x[t];
        float e = d * d;
        c = (t == 0) ? e : e + c;
    }
    return c;
}
