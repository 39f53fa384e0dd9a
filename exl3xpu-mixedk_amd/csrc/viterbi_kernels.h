// viterbi_kernels.h -- internal launch interface of the gfx950 trellis kernels.
//
// Not part of the C-ABI: the exported entry points live in exl3_vit_capi.hip
// and are declared in include/exl3_vit.h.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stddef.h>

namespace xtq {

// Threads per forward workgroup; one workgroup advances T (1, 2, 4 or 8)
// 256-step sequences in lockstep, 64 trellis states per thread per sequence.
constexpr int kFwdThreads = 1024;
// Threads per traceback workgroup.
constexpr int kTbThreads = 256;
// Number of trellis steps per sequence (16x16 tile).
constexpr int kSteps = 256;
// Backpointer slots stored per sequence: steps 1..255 of a pass.
constexpr int kSlots = kSteps - 1;

// Bytes of backpointers one sequence writes per step, for K bits per weight.
size_t bp_step_bytes(int K);
// Bytes of backpointer scratch one sequence needs for a whole pass.
inline size_t bp_tile_bytes(int K) { return (size_t)kSlots * bp_step_bytes(K); }

// Sequences per forward workgroup chosen for a launch of nseq sequences on a
// device with ncu compute units (LDS bounds it by K; small launches use 1).
int forward_group(int K, int nseq, int ncu);

// Forward DP of one Viterbi run for nseq sequences.
//   X, xstride, xlen  targets: row q holds xlen fp32 values at X + q*xstride
//   lut     [65536] fp32 codebook values f(state) (device)
//   roll    step i reads target (i - roll) mod xlen (roll != 0 needs xlen 256)
//   nsteps  steps of the run (<= xlen when roll == 0)
//   store_lo first step whose backpointers are kept (steps store_lo..nsteps-2)
//   ov_in   [nseq] pin values, or NULL for a free run; a pinned run pins
//           s_0 >> K == ov and s_last mod 2^(16-K) == ov (quantize.py:265-303)
//   bp      backpointer scratch, bp_tile_bytes(K) per sequence (device)
//   send    [nseq] final state of the run (device, out)
//   err     device word, OR-ed with 1 when a target is NaN
hipError_t launch_forward(int K, const float* X, int xstride, int xlen, int nseq,
                          const float* lut, int roll, int nsteps, int store_lo,
                          const int32_t* ov_in, void* bp, int32_t* send, uint32_t* err,
                          int group, hipStream_t stream);

// launch_forward for K=3 (same arguments); defined in the K=3 translation
// unit (viterbi_kernels.hip built with XTQ_FWD_K3_TU).
hipError_t launch_forward_k3(const float* X, int xstride, int xlen, int nseq,
                             const float* lut, int roll, int nsteps, int store_lo,
                             const int32_t* ov_in, void* bp, int32_t* send, uint32_t* err,
                             int group, hipStream_t stream);

// The forward DP with the argmin deferred to the traceback (K >= 4): same
// arguments as launch_forward, but instead of packed backpointers it writes
// the group minima b_r of steps r = max(store_lo, 1) .. nsteps-2 to bm, one
// row of 2^(16-K) floats per step, defer_tile_bytes(K) per sequence.
size_t defer_tile_bytes(int K);
hipError_t launch_forward_defer(int K, const float* X, int xstride, int xlen, int nseq,
                                const float* lut, int roll, int nsteps, int store_lo,
                                const int32_t* ov_in, void* bm, int32_t* send, uint32_t* err,
                                int group, hipStream_t stream);

// Traceback of launch_forward_defer's run from send down to step `stop`
// (one lane per sequence), recomputing each link's argmin from the minima
// rows, the codebook and the targets (X, xstride, xlen, roll as the forward
// read them; ov_in the run's pins or NULL).  Outputs as launch_traceback.
hipError_t launch_traceback_defer(int K, const void* bm, const float* X, int xstride, int xlen,
                                  int roll, const float* lut, int nseq,
                                  const int32_t* send, const int32_t* ov_in, int nsteps,
                                  int stop, int shift, int32_t* sout, int32_t* states,
                                  int16_t* trellis, hipStream_t stream);

// Both tail-biting passes of nseq sequences (256-step targets X [nseq][256])
// in one launch of 2*nseq workgroups (see tailbite_fused_kernel): pass 1
// free on X rolled by pivot for n1 steps, traced back in-kernel to
// ov = s_pivot >> K (ovbuf), pass 2 pinned to ov; send receives the pass-2
// final states and bp the pass-2 backpointers (trace them back with
// launch_traceback(K, bp, nseq, send, 256, 0, ...)).  flags [nseq] must hold
// values != epoch on entry (epoch increases per launch; zero-filled memory
// and epoch >= 1 work); counter is one device word.  err |= 2 when a pass-2
// wait expires after spin_limit polls, |= 4 on a task outside the launch.
hipError_t launch_tailbite_fused(int K, const float* X, int nseq, const float* lut,
                                 int pivot, int n1, void* bp, int32_t* send, int32_t* ovbuf,
                                 uint32_t* flags, int32_t* counter, uint32_t epoch,
                                 int spin_limit, uint32_t* err, hipStream_t stream);

// Writes the block-LDL factor L [k][k] (row-major, k a multiple of 16) into
// Lq (k*k floats) in the chain feedback's quad layout (see
// lfac_quads_kernel; only the part below the diagonal blocks).
hipError_t launch_lfac_quads(const float* L, int k, float* Lq, hipStream_t stream);

// out = blockdiag(ht^T) @ in for in, out [rows][cols] fp32 row-major (rows a
// multiple of 128, in != out), ht[t][r] the weight of input row t in output
// row r: each output one fp32 fused multiply-add chain in ascending order.
hipError_t launch_had_left(const float* ht, const float* in, float* out, int rows, int cols,
                           hipStream_t stream);

// out = in @ blockdiag(h) for in, out [rows][cols] fp32 row-major (cols a
// multiple of 128, in != out), h[t][c] the weight of input column t in
// output column c: each output one fp32 fused multiply-add chain in
// ascending order (the products and order of launch_had_left on the
// transpose).
hipError_t launch_had_right(const float* h, const float* in, float* out, int rows, int cols,
                            hipStream_t stream);

// The BlockLDLQ sweep of the column tiles jc0 .. jc0+tnl-1 of W [k][n]
// (inner domain, row-major, k and n multiples of 16) as one persistent
// launch of nwg workgroups over their column chains (see ldlq_chain_kernel).
// Lq: the factor from launch_lfac_quads (NULL: no feedback, plain
// tail-biting of every tile).  Writes hatW [k][n] (decoded tiles), Eq (k*n
// floats of scratch: W - hatW in the quad layout, which the kernel reads
// for the feedback), states [tk*tn][256] (nullable) and trellis
// [tk][tnl][16K] of the launch's tiles.  bp: nwg backpointer slots of
// bp_tile_bytes(K); xbuf: the targets, [nwg][256] scratch, or with xdump
// [tk*tn][256] holding every tile's targets afterwards.  flags [tk*tn] hold
// values != epoch on entry; counter is one device word per launch.  Launches
// over disjoint column ranges may run concurrently (they share Lq, Eq,
// hatW, states and flags).  err |= 1 on a NaN target, |= 2 when a wait
// expires after spin_limit polls, |= 4 on a runaway task loop.  buf_cols
// (a multiple of 16) is the reference sweep's lazy-feedback buffer width,
// which fixes the order the feedback is summed in.
hipError_t launch_ldlq_chain(int K, const float* W, const float* Lq, int k, int n, int jc0,
                             int tnl, const float* lut, int pivot, int n1, void* bp,
                             int nwg, float* xbuf, int xdump, float* hatW, float* Eq,
                             int32_t* states, int16_t* trellis, uint32_t* flags,
                             int32_t* counter, uint32_t epoch, int spin_limit, uint32_t* err,
                             int buf_cols, hipStream_t stream);

// Traceback of one run from send (the state at step nsteps-1) down to step
// `stop`.  Writes sout[q] = s_stop >> shift (nullable), the nsteps states
// (states [nseq][nsteps], nullable; needs stop == 0) and/or the packed EXL3
// trellis (trellis [nseq][16K] int16, nullable; needs stop == 0 and
// nsteps == 256).  lanes: one lane per sequence reading single backpointer
// units (large batches) instead of one workgroup per sequence staging whole
// rows through LDS (small batches).
hipError_t launch_traceback(int K, const void* bp, int nseq, const int32_t* send,
                            int nsteps, int stop, int shift, int32_t* sout,
                            int32_t* states, int16_t* trellis, bool lanes,
                            hipStream_t stream);

// Trellis decode: int16 [tk][tn][16K] -> [16tk][16tn] (fp32 or fp16 bits).
hipError_t launch_decode(int K, const int16_t* trellis, int tk, int tn,
                         const float* lut, float* out_f32,
                         uint16_t* out_f16, hipStream_t stream);

// Pack / unpack between int32 states [nt][256] and int16 trellis [nt][16K].
hipError_t launch_pack(int K, const int32_t* states, int nt, int16_t* trellis,
                       hipStream_t stream);
hipError_t launch_unpack(int K, const int16_t* trellis, int nt, int32_t* states,
                         hipStream_t stream);

// p[0..n) = v on `stream` (a kernel, so that it may be captured in a graph).
hipError_t launch_fill_u32(uint32_t* p, uint32_t n, uint32_t v, hipStream_t stream);

}  // namespace xtq
