/*
 * exl3_vit.h -- C-ABI of the MI355X (gfx950) EXL3 trellis encoder library
 * (libexl3vit.so).
 *
 * The library encodes 16x16 weight tiles (256-step sequences) with the QTIP
 * two-pass tail-biting Viterbi on the 16-bit-state EXL3 trellis, K = 2..7 bits
 * per weight, and decodes trellis streams back to weights.  Results are
 * bit-exact with the reference torch path (quantize/quantize.py:218-415).
 *
 * Conventions (kept from quantize/viterbi_esimd.cpp:924-1005):
 *   - every entry point returns an int status, 0 on success; nothing throws
 *     across the ABI; diagnostics go to stderr;
 *   - the caller owns all input and output buffers; the library owns a
 *     per-device, grow-only device scratch it never frees (and, for the
 *     host-pointer entries, a grow-only pinned host buffer of the last
 *     call's states, nseq * 1 KiB);
 *   - one caller at a time per process (calls are serialised internally by a
 *     mutex, but concurrent callers gain nothing);
 *   - X is [nseq][256] fp32, C-contiguous, one sequence per tile in the
 *     sequence order x_t = tile[perm[t]] (quantize.py:684-686).
 *
 * Status codes (1-6 keep the reference's numbers and meaning):
 *   0  ok
 *   1  initialisation failed (no HIP device, HIP error during init)
 *   2  device allocation failed
 *   3  XTQ_VIT_DEVIDX names no device
 *   4  HIP runtime error during a run
 *   5  host-pointer entries: nseq * 1,317,888 B > XTQ_VIT_MAXBYTES (the
 *      reference's check); any entry: library-owned device bytes would
 *      exceed XTQ_VIT_DEV_MAXBYTES
 *   6  nseq <= 0, or nseq > XTQ_VIT_MAXSEQ on the host-pointer entries;
 *      bad shapes on the device entries
 *   8  unsupported code (e.g. "ih2x2"; the V=1 codebooks run: "mul1",
 *      "3inst", "mcg" and "1mad")
 *   9  K outside 2..7 (or K != 4 for the K=4-only reference codes)
 *  10  pivot outside [0,256), or margin < 0 on the entries the reference
 *      has no counterpart for (xtq_vit_run treats margin < 0 as 0, as the
 *      reference kernel does; the reference reads outside X for such a
 *      pivot, its torch path asserts)
 *  11  a target is NaN
 *  12  null or misaligned pointer argument
 *  13  a synchronous entry was given a stream that is being captured into a
 *      HIP graph (nothing was enqueued; the capture is left intact)
 *
 * Environment (read on every call):
 *   XTQ_VIT_DEVIDX   device index for the host-pointer entries (default: the
 *                    calling thread's current HIP device)
 *   XTQ_VIT_MAXSEQ   upper bound on nseq per host-pointer call (default
 *                    4096, the reference's)
 *   XTQ_VIT_MAXBYTES bound on nseq * 1,317,888 B per host-pointer call
 *                    (default 6 GiB, the reference's accounting)
 *   XTQ_VIT_DEV_MAXBYTES upper bound on library-owned device bytes (default
 *                    64 GiB; no reference counterpart)
 *   XTQ_VIT_SCRATCH  backpointer scratch budget in bytes; larger batches are
 *                    processed in chunks (default 8 GiB)
 *   XTQ_VIT_DEFER    1: run the deferred-argmin encode for K >= 4 (opt-in);
 *                    unset or any other value: never
 *   XTQ_VIT_DEFER_SCRATCH  scratch budget of the deferred-argmin encode's
 *                    minima rows (default 48 GiB, at most half of the free
 *                    device memory)
 *   XTQ_VIT_GROUP    force 1, 2, 4 or 8 sequences per forward workgroup
 *                    (testing; default chosen from the batch size)
 *   XTQ_VIT_TB_LANES smallest batch whose tracebacks run one lane per sequence
 *                    (0: always, -1: never; default 2048)
 *   XTQ_VIT_FUSED    0: always run the two tail-biting passes as separate
 *                    launches; 1: always as one fused launch (testing);
 *                    default: fused for batches under 4 sequences per CU
 */
#ifndef EXL3_VIT_H
#define EXL3_VIT_H

#include <stdint.h>

/* The library is built with hidden symbol visibility; only these entry
 * points are exported. */
#if defined(__GNUC__) || defined(__clang__)
#define XTQ_API __attribute__((visibility("default")))
#else
#define XTQ_API
#endif

#ifdef __cplusplus
extern "C" {
#endif

/*
 * Replaces quantize/viterbi_esimd.cpp:935 xtq_vit_init (bound by
 * quantize.py:497-503).  Selects the device (XTQ_VIT_DEVIDX) and uploads the
 * codebook tables.  Idempotent.
 */
XTQ_API int xtq_vit_init(void);

/*
 * Replaces quantize/viterbi_esimd.cpp:970 xtq_vit_run (bound by
 * quantize.py:499-501,604-606).  Host pointers, synchronous.
 *   X     [nseq][256] fp32 host
 *   code  "mul1p", "mul1" or "mul1t" (the reference's K=4 mul1 kernels; all
 *         three give identical results); "ih2x2" returns 8
 *   out   [nseq][256] int32 host: the pass-2 states
 * Bounds as the reference's: nseq <= XTQ_VIT_MAXSEQ (default 4096, else 6),
 * nseq * 1,317,888 <= XTQ_VIT_MAXBYTES (default 6 GiB, else 5); margin < 0
 * runs pass 1 over the whole sequence, as margin 0.
 */
XTQ_API int xtq_vit_run(const float* X, int nseq, const char* code, int margin, int pivot,
                int32_t* out);

/*
 * K-aware host-pointer variant of xtq_vit_run (no reference counterpart: the
 * reference kernel is K=4 only, viterbi_esimd.cpp:83,352; the torch path it
 * generalises is quantize.py:323-354).  code: "mul1", "3inst", "mcg" (the
 * EXL3 codes, fp16 values) or "1mad" (QTIP's 1MAD code, fp32 values); the
 * exl3_/qtip_ prefixed names of quantize.py are accepted too.
 */
XTQ_API int xtq_vit_run_k(const float* X, int nseq, int K, const char* code, int margin,
                  int pivot, int32_t* out);

/*
 * Device-pointer tail-biting encoder: the HIP counterpart of
 * quantize_seq_tailbite (quantize.py:323-354) for torch-ROCm tensors.
 * Stream-ordered on `stream` (a hipStream_t, 0 = default stream) and
 * synchronous on return (the NaN check reads a device flag).
 *   dX        [nseq][256] fp32 device
 *   d_states  [nseq][256] int32 device, or NULL
 *   d_trellis [nseq][16K] int16 device (EXL3 trellis slices, pack_states
 *             layout quantize.py:360-378), or NULL
 */
XTQ_API int xtq_vit_tailbite_dev(const float* dX, int nseq, int K, const char* code,
                         int margin, int pivot, int32_t* d_states,
                         int16_t* d_trellis, void* stream);

/*
 * Stream-ordered variant of xtq_vit_tailbite_dev (no reference counterpart:
 * the reference's run is synchronous, viterbi_esimd.cpp:970-1005).  Returns
 * once the work is enqueued on `stream`; the outputs are valid in stream
 * order.  A NaN target is not reported here: it sets a per-device flag that
 * xtq_vit_status_dev reads.  For the BlockLDLQ sweep, which issues one
 * encode per 16-row block and must not wait on the host between blocks.
 * Calls on different streams are ordered among themselves by the library
 * (they share its backpointer scratch).
 */
XTQ_API int xtq_vit_tailbite_dev_async(const float* dX, int nseq, int K, const char* code,
                               int margin, int pivot, int32_t* d_states,
                               int16_t* d_trellis, void* stream);

/*
 * xtq_vit_tailbite_dev without any device allocation.  No reference
 * counterpart: for callers that cannot allocate device memory (tight serving
 * loops, harnesses that forbid hipMalloc).  It is synchronous -- it ends by
 * reading its status word back and waiting for `stream` -- so it cannot be
 * recorded into a HIP graph: on a stream under capture it returns 13 before
 * enqueuing anything, and the capture stays valid.
 * The caller passes inputs and outputs as for xtq_vit_tailbite_dev; the
 * backpointers and per-sequence words live in a fixed 256 MiB array in the
 * library's code object (one copy per device, held until the process ends),
 * so one call takes at most 257 sequences at K=2 or 3, 513 at K=4 or 5,
 * 1,027 at K=6 and 2,055 at K=7 (status 5 beyond that; split the batch).
 * The device must have been set up by xtq_vit_init (or by any other entry
 * point) first, else status 1.  Synchronous; calls are serialised by the
 * library's lock, and since each returns only after its work has finished,
 * calls on one GPU never overlap (each process has its own array).
 * Results equal xtq_vit_tailbite_dev's bit for bit.
 */
XTQ_API int xtq_vit_tailbite_dev_noalloc(const float* dX, int nseq, int K, const char* code,
                                         int margin, int pivot, int32_t* d_states,
                                         int16_t* d_trellis, void* stream);

/*
 * Waits for `stream` and reports the NaN flag that stream-ordered encodes
 * set since the last status or synchronous call: 0, or 11 (the flag is then
 * cleared), or 4 on a HIP error.
 */
XTQ_API int xtq_vit_status_dev(void* stream);

/*
 * The whole BlockLDLQ sweep (ldlq_viterbi, quantize.py:631-746) on the
 * device, as column chains in one persistent launch: tile (i, j)'s targets
 * are W[16i+r][16j+c] + sum_{m >= 16(i+1)} L[m][16i+r] (W - What)[m][16j+c],
 * so each output column of tiles is an independent chain and the GPU is
 * never idle at the end of a 16-row block.  No reference counterpart for
 * the launch itself (the reference issues one tail-bite per 16-row block
 * with torch GEMMs for the feedback); each tile's encode is bit-exact for
 * its targets, which d_targets exposes.  The feedback is summed in the
 * reference's own order (quantize.py:662-686,743-744 with buf_cols, its
 * GEMMs evaluated as torch's CPU sgemm does: one fp32 fused multiply-add
 * chain per output over the rows of each buffer, buffers added in sweep
 * order), so the targets, and hence W_hat and the trellis, equal the
 * reference's ldlq_viterbi on the same W and L for buf_cols up to 128 (a
 * wider buffer is one chain here too, while the host BLAS may split that
 * inner dimension).  Synchronous on return.
 *   d_W       [k][n] fp32 device, inner domain (k, n multiples of 16)
 *   d_L       [k][k] fp32 device block-LDL factor (row-major, 16-byte
 *             aligned), or NULL for no feedback
 *   buf_cols  ldlq_viterbi's lazy-feedback buffer width (a multiple of 16;
 *             the reference's default is 128), else status 6
 *   d_hatW    [k][n] fp32 device (out): the decoded tiles
 *   d_states  [k/16 * n/16][256] int32 device (out), or NULL
 *   d_trellis [k/16][n/16][16K] int16 device (out)
 *   d_targets [k/16 * n/16][256] fp32 device (out: every tile's targets in
 *             sequence order), or NULL
 */
XTQ_API int xtq_ldlq_chain_dev(const float* d_W, const float* d_L, int k, int n, int K,
                               const char* code, int margin, int pivot, int buf_cols,
                               float* d_hatW, int32_t* d_states, int16_t* d_trellis,
                               float* d_targets, void* stream);

/*
 * xtq_ldlq_chain_dev for weights quantized side by side at different K
 * (e.g. a layer's q/k/v projections, which share one input Hessian): W's
 * columns are ngroups consecutive groups of h_ncols[g] columns (multiples
 * of 16, summing to n) encoded at h_K[g] bits, group g's trellis going to
 * h_trellis[g] ([k/16][h_ncols[g]/16][16 h_K[g]] int16 device).  The groups
 * run as concurrent launches over a split of the compute units; every tile
 * encodes exactly as in a single-group call.  No reference counterpart (the
 * reference quantizes one weight at a time).  At most 8 groups.
 */
XTQ_API int xtq_ldlq_chain_multi_dev(const float* d_W, const float* d_L, int k, int n,
                                     int ngroups, const int* h_ncols, const int* h_K,
                                     const char* code, int margin, int pivot, int buf_cols,
                                     float* d_hatW, int32_t* d_states,
                                     int16_t* const* h_trellis, float* d_targets,
                                     void* stream);

/*
 * Device-pointer single Viterbi run: the HIP counterpart of viterbi()
 * (quantize.py:218-320) with V = 1 and L = 16.
 *   dX         [nseq][T] fp32 device, 1 <= T <= 256
 *   d_overlap  [nseq] int32 device pin values in [0, 2^(16-K)), or NULL for a
 *              free run; a pinned run pins s_0 >> K and s_{T-1} mod 2^(16-K)
 *   back_from  -1: d_out is [nseq][T] int32, the full state sequence;
 *              0 <= back_from < T: d_out is [nseq], the state at back_from
 *              (links kept only after back_from, quantize.py:273-277,305-312)
 * Synchronous on return, like xtq_vit_tailbite_dev.
 */
XTQ_API int xtq_vit_viterbi_dev(const float* dX, int nseq, int T, int K, const char* code,
                        const int32_t* d_overlap, int back_from, int32_t* d_out,
                        void* stream);

/*
 * Device-pointer trellis decode: the HIP counterpart of decode_trellis
 * (quantize.py:405-415) and of exl3xpu's reconstruct (patch 0001:60-75).
 *   d_trellis [tk][tn][16K] int16 device
 *   d_out_f32 [16tk][16tn] fp32 device, or NULL
 *   d_out_f16 [16tk][16tn] fp16 (bit patterns) device, or NULL: the table
 *             value rounded to fp16 (exact for the EXL3 codes; "1mad"'s fp32
 *             values round)
 * Stream-ordered: returns once the kernel is enqueued on `stream` (as do
 * the pack and unpack entries below).
 */
XTQ_API int xtq_trellis_decode_dev(const int16_t* d_trellis, int tk, int tn, int K,
                           const char* code, float* d_out_f32, uint16_t* d_out_f16,
                           void* stream);

/* Device-pointer pack_states / unpack_states (quantize.py:360-402). */
XTQ_API int xtq_trellis_pack_dev(const int32_t* d_states, int nt, int K, int16_t* d_trellis,
                         void* stream);
XTQ_API int xtq_trellis_unpack_dev(const int16_t* d_trellis, int nt, int K, int32_t* d_states,
                           void* stream);

/*
 * Device-pointer block-128 transform on the first dimension: the HIP
 * counterpart of had_left (quantize.py:134-138).  d_ht holds the [128][128]
 * multipliers by input row, d_ht[t][r] the weight of input row t in output
 * row r, so d_out = blockdiag(d_ht^T) @ d_in for [rows][cols] fp32 row-major
 * buffers (rows a multiple of 128, d_out not d_in).  For had_left(w, h) pass
 * h^T; the normalised Sylvester matrix of hadamard128 (quantize.py:123-131)
 * is symmetric, so it is passed as it is.  Each output is one fp32 fused
 * multiply-add chain over the 128 products in ascending order, as torch's
 * CPU sgemm evaluates the reference's matmul, so results equal the
 * reference's CPU results bit for bit.  Stream-ordered.
 */
XTQ_API int xtq_had128_left_dev(const float* d_ht, const float* d_in, float* d_out, int rows,
                                int cols, void* stream);

/*
 * Device-pointer block-128 transform on the last dimension: the HIP
 * counterpart of had_right (quantize.py:141-145).  d_h holds the [128][128]
 * multipliers, d_h[t][c] the weight of input column t in output column c,
 * so d_out = d_in @ blockdiag(d_h) for [rows][cols] fp32 row-major buffers
 * (cols a multiple of 128, rows up to 2,097,120, d_out not d_in).  Each
 * output is one fp32 fused multiply-add chain over the 128 products in
 * ascending order, as torch's CPU sgemm evaluates the reference's matmul
 * (the products and order of xtq_had128_left_dev on the transpose), so
 * results equal the reference's CPU results bit for bit.  Stream-ordered.
 */
XTQ_API int xtq_had128_right_dev(const float* d_h, const float* d_in, float* d_out, int rows,
                                 int cols, void* stream);

/*
 * Copies the fp32 decode table of `code` (65536 entries) into host memory
 * (the values get_lut returns, quantize.py:90-97).
 */
XTQ_API int xtq_vit_get_lut(const char* code, float* out);

/* Backpointer scratch bytes per sequence for K (sizing information). */
XTQ_API int64_t xtq_vit_scratch_per_seq(int K);

/*
 * Sizing information (no reference counterpart): the sequences per scratch
 * chunk a tail-bite of nseq sequences at K would run in on the current
 * device with the current environment, and in *deferred (nullable) 1 when
 * it would take the deferred-argmin encode (group minima rows in HBM, the
 * argmin recomputed by the traceback; only with XTQ_VIT_DEFER=1 and
 * K >= 4), else 0.  Returns minus a status code on error.  Sets the device
 * up like any other entry point.
 */
XTQ_API int xtq_vit_chunk_seqs(int nseq, int K, int* deferred);

/*
 * Kernel timing for benchmarks (no reference counterpart; the reference
 * times whole calls with steady_clock, viterbi_esimd.cpp:869-880).  While
 * enabled, every forward-DP and traceback launch is bracketed with HIP events
 * on the stream it runs on.  xtq_vit_prof_read returns and resets the totals:
 * forward milliseconds, forward launches, forward sequence-steps (sum of
 * sequences x steps over the launches), traceback milliseconds and launches.
 */
XTQ_API int xtq_vit_prof_enable(int on);
XTQ_API int xtq_vit_prof_read(double* fwd_ms, int64_t* fwd_launches, double* fwd_seq_steps,
                      double* tb_ms, int64_t* tb_launches);

/* Static description of a status code. */
XTQ_API const char* xtq_vit_strerror(int rc);

#ifdef __cplusplus
}
#endif

#endif /* EXL3_VIT_H */
