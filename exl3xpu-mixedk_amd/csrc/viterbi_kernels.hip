// viterbi_kernels.hip -- gfx950 kernels for the EXL3 tail-biting trellis encoder.
//
// Contract (bit-exact with the reference torch Viterbi, quantize.py:218-354):
//   emit      e[s] = fl(fl(f[s] - x)^2)           (no FMA contraction)
//   step      c_i[s] = fl(e_i[s] + b_i[s >> K])
//   reduce    b_{i+1}[j] = min_w c_i[j + w*SP], lowest w on ties
//   end       lowest state index among equal minima (free end); pinned end
//             keeps only states with s mod SP == ov
//
// Work decomposition (16-bit state, K bits per step, NC = 2^K predecessors,
// SP = 2^(16-K) groups):
//   * one 1024-thread workgroup (16 waves, one per CU at 4 waves/SIMD)
//     advances T = 1, 2, 4 or 8 sequences in lockstep;
//   * thread t owns the C = SP/1024 consecutive groups j = t*C .. t*C+C-1
//     (K=7: half of group t/2) and the candidate states of each,
//     s = j + w*SP, i.e. 64 states per thread for every K; their codebook
//     values (the fp32 table of the reference's get_lut: fp16 values for
//     the EXL3 codes, (bytesum - 510) / 147.8 rounded to fp32 for
//     qtip_1mad) stay in 64 fp32 VGPRs for the whole kernel, shared by the
//     T sequences, so that fl(f - x) is one v_add_f32 of -x, an instruction
//     gfx950 issues on its fast path (the packed fp16 pairs plus
//     v_fma_mix_f32 of earlier versions took 32 VGPRs but a full 4 cycles);
//   * the per-group minima b (SP floats per sequence) are the only state
//     carried between steps; they live in LDS, double buffered, one barrier
//     per step for all T sequences;
//   * min and first-index argmin fold into one v_min_f64 per candidate: the
//     cost (non-negative fp32) is the high dword and the predecessor index
//     the low dword of a 64-bit key, so the fp64 order of the keys is the
//     lexicographic order (cost, index) -- the reference's tie rule;
//   * backpointers are K bits per group, packed per thread and written
//     coalesced to HBM; a separate traceback kernel stages them through LDS.
//
// Built twice: as the library's kernels, and with XTQ_FWD_K3_TU defined as
// the translation unit of K=3's batched forward alone (launch_forward_k3),
// which is compiled under the max-ilp scheduling strategy (faster for that
// kernel only; every other kernel measured slower under it).
#include "viterbi_kernels.h"

#pragma clang fp contract(off)


namespace xtq {
namespace {


template <int K>
struct Geom {
    static constexpr int NC = 1 << K;                 // predecessors per group
    static constexpr int SP = 1 << (16 - K);          // groups
    static constexpr int Q = 1 << (16 - 2 * K);       // NC x NC blocks per step
    static constexpr bool HALF = (SP < kFwdThreads);  // K=7: two lanes per group
    static constexpr int C = HALF ? 1 : SP / kFwdThreads;  // groups per thread
    static constexpr int W = HALF ? NC / 2 : NC;      // candidates per group/thread
    static constexpr int NCH = W < 16 ? W : 16;       // candidates per chunk
    static constexpr int NCHUNK = W / NCH;
    static constexpr int NB = C > NC ? C / NC : 1;    // blocks per thread
    static constexpr int CB = C / NB;                 // groups per block
    static constexpr int NSTATE = C * W;              // states per thread
    static constexpr int BITS = C * K;                // backpointer bits/thread
    static constexpr int UNIT = HALF ? 1 : BITS <= 8 ? 1 : BITS <= 16 ? 2 : 4;
    // Bytes per step: one unit per thread, or one byte per group when two
    // lanes share a group.
    static constexpr int BPSTEP = HALF ? SP : kFwdThreads * UNIT;
    // LDS slots per b buffer.  With two lanes per group (K=7) the even and
    // odd lanes of a wave read b at addresses 256 groups apart -- the same
    // bank -- so group j lives at slot j + (j >> 8): one pad slot moves the
    // upper half to the next bank (padded to keep rows 16-byte aligned).
    static constexpr int SPL = HALF ? SP + 4 : SP;
    static_assert(NSTATE == 64, "64 states per thread");
    static_assert(BITS <= 32, "backpointer unit");
    static_assert(BPSTEP % 16 == 0, "staging granularity");
};

// LDS slot of group j in a b buffer (see Geom::SPL).
template <int K>
__device__ __forceinline__ int bslot(int j) {
    return Geom<K>::HALF ? j + (j >> 8) : j;
}

template <int N> struct UnitT;
template <> struct UnitT<1> { typedef uint8_t type; };
template <> struct UnitT<2> { typedef uint16_t type; };
template <> struct UnitT<4> { typedef uint32_t type; };

// 64-bit key: high dword = cost bits, low dword = tag (index in the low byte).
__device__ __forceinline__ double key_of(uint32_t lo, float c) {
    return __builtin_bit_cast(double,
                              (uint64_t)lo | ((uint64_t)__float_as_uint(c) << 32));
}
__device__ __forceinline__ float key_cost(double k) {
    return __uint_as_float((uint32_t)(__builtin_bit_cast(uint64_t, k) >> 32));
}
__device__ __forceinline__ uint32_t key_lo(double k) {
    return (uint32_t)__builtin_bit_cast(uint64_t, k);
}
// Keys are never NaN (the high dword is a non-negative fp32 cost <= +inf) and
// IEEE min needs no canonicalisation here, so issue v_min_f64 directly.
__device__ __forceinline__ double kmin(double a, double b) {
    double r;
    asm("v_min_f64 %0, %1, %2" : "=v"(r) : "v"(a), "v"(b));
    return r;
}

__device__ __forceinline__ double kmin_xor(double k, int m) {
    const uint32_t lo = key_lo(k), hi = __float_as_uint(key_cost(k));
    const uint32_t plo = __shfl_xor(lo, m), phi = __shfl_xor(hi, m);
    return kmin(k, key_of(plo, __uint_as_float(phi)));
}

// Min with the neighbour lane (lane ^ 1) through a DPP quad permutation
// [1,0,3,2]: two v_mov_b32_dpp and one v_min_f64, no LDS round trip.
__device__ __forceinline__ double kmin_xor1(double k) {
    const int lo = (int)key_lo(k), hi = (int)__float_as_uint(key_cost(k));
    const uint32_t plo = (uint32_t)__builtin_amdgcn_mov_dpp(lo, 0xB1, 0xF, 0xF, false);
    const uint32_t phi = (uint32_t)__builtin_amdgcn_mov_dpp(hi, 0xB1, 0xF, 0xF, false);
    return kmin(k, key_of(plo, __uint_as_float(phi)));
}

// A global-memory pointer the caller knows to be the same in every lane,
// moved to SGPRs and typed as global (so accesses through it are global_*
// instructions, not flat ones, which would also count against lgkmcnt).
typedef __attribute__((address_space(1))) uint8_t gbyte_t;
__device__ __forceinline__ gbyte_t* uniform_gptr(uint8_t* p) {
    const uint64_t v = (uint64_t)(size_t)p;
    const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)v);
    const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(v >> 32));
    return (gbyte_t*)(size_t)(((uint64_t)hi << 32) | lo);
}

// Byte address of a __shared__ location in the LDS aperture.
__device__ __forceinline__ uint32_t lds_addr(const float* p) {
    return (uint32_t)(size_t)(__attribute__((address_space(3))) const float*)(p);
}

// Stores the cost halves of two keys to dwords D and D+1 after `addr` with
// one ds_write2_b32 straight from the key registers (a vector store of the
// four costs would first gather them into consecutive VGPRs).  The compiler
// does not see this store: the caller waits with lgkmcnt(0) before the
// barrier that publishes it.
template <int D>
__device__ __forceinline__ void lds_store_cost2(uint32_t addr, double k0, double k1) {
    asm volatile("ds_write2_b32 %0, %1, %2 offset0:%3 offset1:%4"
                 :
                 : "v"(addr), "v"(key_cost(k0)), "v"(key_cost(k1)), "i"(D), "i"(D + 1)
                 : "memory");
}

template <int C, int c = 0>
__device__ __forceinline__ void lds_store_costs(uint32_t addr, const double* run) {
    if constexpr (c < C) {
        lds_store_cost2<c>(addr, run[c], run[c + 1]);
        lds_store_costs<C, c + 2>(addr, run);
    }
}

// fp32 minima for the steps and kernels that need no argmin.  Costs are never
// NaN (a NaN target ends the call with status 11) and IEEE min needs no
// canonicalisation here, so the instructions are issued directly.
__device__ __forceinline__ float fmin2(float a, float b) {
    float r;
    asm("v_min_f32 %0, %1, %2" : "=v"(r) : "v"(a), "v"(b));
    return r;
}
__device__ __forceinline__ float fmin3(float a, float b, float c) {
    float r;
    asm("v_min3_f32 %0, %1, %2, %3" : "=v"(r) : "v"(a), "v"(b), "v"(c));
    return r;
}

// Minimum of v[0..N) in triples (a v_min_f32 pair tree measured 3-7 %
// slower); a level's one or two leftover values pass to the next level
// unreduced, so N values take ceil((N-1)/2) instructions.
template <int N>
__device__ __forceinline__ float fmin_tree(const float* v) {
    if constexpr (N == 1) {
        return v[0];
    } else if constexpr (N == 2) {
        return fmin2(v[0], v[1]);
    } else if constexpr (N == 3) {
        return fmin3(v[0], v[1], v[2]);
    } else {
        constexpr int M = N / 3, R = N % 3;
        float r[M + R];
#pragma unroll
        for (int m = 0; m < M; ++m) r[m] = fmin3(v[3 * m], v[3 * m + 1], v[3 * m + 2]);
#pragma unroll
        for (int m = 0; m < R; ++m) r[M + m] = v[3 * M + m];
        return fmin_tree<M + R>(r);
    }
}

// A compile-time switch passed to a generic lambda, and the running minimum's
// type per reduction: a (cost, index) key or the fp32 cost alone.
template <bool B> struct BoolC { static constexpr bool value = B; };
template <bool KEYS> struct RunType { typedef float type; };
template <> struct RunType<true> { typedef double type; };
__device__ __forceinline__ float cost_of(double k) { return key_cost(k); }
__device__ __forceinline__ float cost_of(float c) { return c; }

// Backpointer of group j in one step's row.
template <int K>
__device__ __forceinline__ int bp_lookup(const uint8_t* row, int j) {
    using G = Geom<K>;
    if constexpr (G::HALF) {
        return row[j];
    } else {
        typedef typename UnitT<G::UNIT>::type unit_t;
        const unit_t u = ((const unit_t*)row)[j / G::C];
        return (int)((u >> ((j % G::C) * K)) & (unit_t)(G::NC - 1));
    }
}

// --------------------------------------------------------------- forward DP
// Whether the candidate arithmetic is issued grouped by opcode (see fwd_run):
// measured faster for K >= 6, and for K = 4, 5 with T >= 2 sequences per
// workgroup (K=4 +1.6 % with the wave priorities below); at T = 1 (the
// column chain) K = 4 and 5 are 1-3 % faster ungrouped.
template <int K, int T>
constexpr bool kGroupOps = (K >= 6) || ((K == 4 || K == 5) && T >= 2);

// The same choice for the min-only steps.
template <int K, int T>
constexpr bool kGroupOpsMin = kGroupOps<K, T>;

// Candidates per chunk of the min tree: 8 wherever the smaller chunk's keys
// make room for the fp32 codebook registers -- every K at T = 1 (the column
// chain) and K != 6 at any T (16-wide chunks spilled there: K=5 batched
// 285k -> 367k tiles/s, K=4 batched 346k -> 361k, the 5120x5120 column
// chain at K=4/5/6/7 0.355/0.366/0.350/0.42 s -> 0.336/0.345/0.340/0.358 s,
// K=7 batched +1 % with the wave priorities below); 16 for K = 6 at T >= 2,
// where 8 measured 2 % slower.
template <int K, int T>
constexpr int kChunkW =
    (T == 1 || K != 6) ? (Geom<K>::NCH < 8 ? Geom<K>::NCH : 8) : Geom<K>::NCH;

// Candidates per chunk in the min-only steps (fp32 costs, no keys): the same
// widths.
template <int K, int T>
constexpr int kChunkWMin = kChunkW<K, T>;

// Wave priorities within a step (s_setprio).  All 16 waves meet at the
// step's barrier, and the SIMD's arbiter otherwise serves its oldest wave
// first, so the same waves run ahead every step while the last one's
// dependency tail (min tree, cost stores) stalls everyone at the barrier.
// Each wave is raised to kPrioTop<K> after the barrier and lowered as it
// passes fixed points of its step's work, so that waves ahead yield the
// SIMD to those behind and all arrive together.  Points, in units of
// (sequence, chunk, group) of the step: K >= 5 drop to 1 at 5/8 and to 0 at
// 7/8 (rescanned last: 15/16 for the second drop, 1/2 or 3/4 for the first,
// and 0 for the first in the column chain, all slower), K = 4 to 1 at half and to 0 at seven eighths with four sequences
// per workgroup (three quarters before the early pair stores of kEarlyPair;
// with them 7/8 measured +0.8 %: 435.4k -> 438.9k tiles/s, 13/16, 27/32 and
// 29/32 in between, 15/16 -0.9 %, no second drop -4 %), at three quarters
// with two, and for a single sequence (the column chain) to 1 as soon as the
// step's target and first minima are read (unit 0) and to 0 at 7/8 (c5 K=4
// sweep 946-948 -> 917 ms, c3 271.6-271.8 -> 263 ms, against the 1/4 and
// 5/8 used before; 1 and 7 units, 2 and 6 or 7, 0 and 6 in between; never
// dropping to 0 +3 %; a first drop at 0 is 3-4 % slower for four sequences
// and for the K = 5, 6 chains), K = 3 to 1 at the step's first group and
// to 0 at 5/8 (one level, 1 -> 0 at three quarters, before: batched 389.9k
// -> 394.9k tiles/s and the 5120x5120 column chain 294.1 -> 287.3 ms with
// the drop at 5/8, then 396k -> 405k with the second level; 3/8, 1/2, 3/4
// and 7/8 slower), K = 2 (one chunk
// of 4-candidate groups) to 1 right after the
// step's target is read and to 0 after three quarters of its groups
// (batched 343k -> 360k tiles/s, the 5120x5120 column chain 308 -> 294 ms,
// against the quarter used before; 1/8 .. 15/16 of the groups and no drop
// to 0 scanned, every other point slower; the drop to 1 moved into the
// groups 2-4 % slower).  Measured against no priorities (same box,
// alternating runs): batched K = 2..7 256k/339k/360k/364k/358k/352k ->
// 311k/371k/391k/392k/391k/390k tiles/s with K >= 5 on the K = 4 points,
// which K >= 5's own add 1 % to (and 2.5 % to their column chain, where
// K = 4 loses 2 % with them); the 5120x5120 column chain at K = 2..7
// -10/-3/-3/-11/-9/-9 %.  Slower: a fourth level for K >= 4.
template <int K>
constexpr int kPrioTop = 2;

// Whether a K=4 key step stores the lane's first two group minima as soon as
// they are final, so that the LDS writes overlap the two remaining groups'
// trees (the other two leave at the end of the step): batched K=4 at four
// sequences per workgroup 431.1k / 431.7k -> 433.9k / 434.4k tiles/s (same
// box, alternating runs, states identical); the column chain (one sequence)
// 947-948 -> 949 ms, so not there.
template <int K, int T>
constexpr bool kEarlyPair = (K == 4 && T >= 2);

// Whether a sequence-step recomputes the lane's offsets instead of keeping
// them live (see fwd_run): measured faster for one sequence per workgroup
// at K = 2, 3 (the column chain: 5120x5120 sweep K=2 -3 %, K=3 -6 %; K=2
// batched unchanged) and slower elsewhere (batched K=5..7 -1..-4 %, the
// chain at K=4 +1.5 %).
template <int K, int T>
constexpr bool kRematLane = (T == 1 && K <= 3);

// Shared memory of one forward run over T sequences.
template <int K, int T>
struct FwdSmem {
    __attribute__((aligned(16))) float bbuf[T][2][Geom<K>::SPL];
    float xs[T][kSteps];
    int32_t ovs[T];                  // pin values (-1: free run), set by the caller
    double red[kFwdThreads / 64];
};

// Forward DP of sequences q0 .. q0+ntile-1 (ntile <= T) in lockstep by one
// 1024-thread workgroup (the codebook registers are shared by the T
// sequences; one barrier per step).  The caller fills sm.ovs[0..T) before
// the call; the final state of sequence q0+tt is written to send[tt] (global
// or shared memory).  tid is threadIdx.x (a persistent caller passes it
// opaque per task, so that nothing derived from it is hoisted out of its
// task loop and kept live across it).
template <int K, int T>
__device__ __forceinline__ void fwd_run(
    FwdSmem<K, T>& sm, const float* __restrict__ X, int xstride, int xlen, int q0, int ntile,
    const float* __restrict__ lut, int roll, int nsteps, int store_lo, bool pinned,
    uint8_t* __restrict__ bp, int32_t* send, uint32_t* __restrict__ err, int tid) {
    using G = Geom<K>;
    auto& bbuf = sm.bbuf;
    auto& xs = sm.xs;
    auto& ovs = sm.ovs;
    auto& red = sm.red;

#pragma unroll
    for (int r0 = 0; r0 < T * kSteps; r0 += kFwdThreads) {
        if (r0 + kFwdThreads <= T * kSteps || tid < T * kSteps - r0) {
            const int idx = r0 + tid, tt = idx / kSteps, e = idx % kSteps;
            float v = 0.0f;
            if (tt < ntile && e < xlen) {
                v = X[(size_t)(q0 + tt) * xstride + e];
                if (v != v) atomicOr(err, 1u);
            }
            xs[tt][e] = v;
        }
    }

    // Owned groups and candidates: groups j_c = jbase + c, candidate w of a
    // group is state j_c + (wbase + w) * SP; local index l = c*W + w.
    const int jbase = G::HALF ? (tid >> 1) : tid * G::C;
    const int wbase = G::HALF ? (tid & 1) * G::W : 0;
    constexpr int NCHK = kChunkW<K, T>;         // candidates per chunk (key steps)
    // codebook value of local state l (the fp32 table entry)
    float f32[G::NSTATE];
#pragma unroll
    for (int l = 0; l < G::NSTATE; ++l)
        f32[l] = lut[jbase + l / G::W + (wbase + l % G::W) * G::SP];
    // fl(f_l - x): one rounding of the exact difference, as the reference's
    // fp32 subtraction
    auto fsub = [&](int l, float negx) { return f32[l] + negx; };
    // Per-lane key tags: distinct per lane so they stay in VGPRs next to the
    // cost they are paired with; the low byte is the candidate index.
    uint32_t tag[NCHK];
#pragma unroll
    for (int w = 0; w < NCHK; ++w) tag[w] = ((uint32_t)tid << 8) | (uint32_t)(wbase + w);
    __syncthreads();

    // Start mask b_0: 0 everywhere (free) or 0 only at group ov (pinned).
    for (int tt = 0; tt < T; ++tt) {
        const int ov = ovs[tt];
        if (!G::HALF || (tid & 1) == 0) {
#pragma unroll
            for (int c = 0; c < G::C; ++c) {
                const int j = jbase + c;
                bbuf[tt][0][bslot<K>(j)] = (ov < 0 || j == ov) ? 0.0f : __builtin_inff();
            }
        }
    }
    __syncthreads();

    const int a0 = jbase >> K;  // first NC x NC block this thread reads
    // b slot offset of every predecessor this lane reads (constant per lane)
    const int rpad = bslot<K>(a0 + wbase * G::Q) - (a0 + wbase * G::Q);

    // Step i of every sequence of the group, then the barrier that publishes
    // b_{i+1}.  KEYS selects the reduction: steps whose backpointer row is
    // kept (i >= store_lo) and the last step reduce (cost, index) keys with
    // v_min_f64; the steps before store_lo, whose links no traceback ever
    // reads (a run keeps links only after back_from, quantize.py:273-277,
    // 287-292), reduce the fp32 costs alone with a v_min3_f32 tree -- the
    // same minima b (the min of a set of non-NaN costs is one of them,
    // whatever the order), half an instruction per candidate against the
    // key path's one v_min_f64 (a slow-rate instruction), and no backpointer
    // row.
    auto step = [&](auto keys_c, int i) __attribute__((always_inline)) {
        constexpr bool KEYS = decltype(keys_c)::value;
        typedef typename RunType<KEYS>::type run_t;
        constexpr int NCH = KEYS ? kChunkW<K, T> : kChunkWMin<K, T>;  // candidates per chunk
        constexpr int NCHUNK = G::W / NCH;
        // Target of step i of the sequence rolled right by `roll`.
        const int u = (i - roll < 0) ? i - roll + xlen : i - roll;
#pragma unroll 1
        for (int tt = 0; tt < ntile; ++tt) {
            // Keep the codebook registers opaque per sequence-step so that
            // they stay put in VGPRs rather than being re-derived.
#pragma unroll
            for (int l = 0; l < G::NSTATE; ++l) asm volatile("" : "+v"(f32[l]));
            // The lane's LDS and backpointer offsets: kept live across the
            // steps, or (kRematLane) recomputed here from an opaque copy of
            // the thread index, which frees their registers -- the compiler
            // had spilled them and reloaded them (a scratch load and a wait)
            // at every step.
            int tl = tid, jb = jbase, wb = wbase, ab = a0, rp = rpad;
            if constexpr (kRematLane<K, T>) {
                asm volatile("" : "+v"(tl));
                jb = G::HALF ? (tl >> 1) : tl * G::C;
                wb = G::HALF ? (tl & 1) * G::W : 0;
                ab = jb >> K;
                rp = bslot<K>(ab + wb * G::Q) - (ab + wb * G::Q);
            }
            const int q = q0 + tt;
            const float negx = -__int_as_float(
                __builtin_amdgcn_readfirstlane(__float_as_int(xs[tt][u])));
            if constexpr (K == 2) __builtin_amdgcn_s_setprio(1);
            const float* bcur = bbuf[tt][i & 1];

            run_t run[G::C];
#pragma unroll
            for (int qc = 0; qc < NCHUNK; ++qc) {
                float B[G::NB][NCH];
#pragma unroll
                for (int w = 0; w < NCH; ++w) {
                    const float* src = bcur + ab + rp + (wb + qc * NCH + w) * G::Q;
                    if constexpr (G::NB == 4) {
                        const float4 v = *(const float4*)src;
                        B[0][w] = v.x; B[1][w] = v.y; B[2][w] = v.z; B[3][w] = v.w;
                    } else {
                        B[0][w] = src[0];
                    }
                }
#pragma unroll
                for (int c = 0; c < G::C; ++c) {
                    const int blk = c / G::CB;
                    if constexpr (K == 2) {
                        if (c == G::C * 3 / 4) __builtin_amdgcn_s_setprio(0);
                    }
                    if constexpr (K >= 3) {
                        constexpr int U = T * NCHUNK * G::C;  // units of a step
                        const int pos = (tt * NCHUNK + qc) * G::C + c;
                        // drop points, as fractions of the step's units
                        constexpr int D1 = K >= 5                ? U * 5 / 8
                                           : K == 4 && T == 1 ? 0
                                           : K == 3           ? 0
                                           : T == 1           ? U / 4
                                                              : U / 2;
                        constexpr int D0 = K >= 5                ? U * 7 / 8
                                           : K == 4 && T == 1 ? U * 7 / 8
                                           : K == 4 && T == 4 ? U * 7 / 8
                                           : K == 3           ? U * 5 / 8
                                                              : U * 3 / 4;
                        if (pos == D1) __builtin_amdgcn_s_setprio(1);
                        if (pos == D0) __builtin_amdgcn_s_setprio(0);
                    }
                    // candidate costs fl(fl(fl(f - x)^2) + b)
                    float dv[NCH];
                    if constexpr (KEYS ? kGroupOps<K, T> : kGroupOpsMin<K, T>) {
                        // Issue the chunk's candidates opcode by opcode (all
                        // subs, then all squares, then all adds): gfx950
                        // issues adjacent independent v_mul_f32 / v_add_f32
                        // faster than one per 4 cycles, which a
                        // dependency-ordered schedule forfeits; the empty asm
                        // statements fix the phase order.
#pragma unroll
                        for (int w = 0; w < NCH; ++w) {
                            dv[w] = fsub(c * G::W + qc * NCH + w, negx);
                        }
#pragma unroll
                        for (int w = 0; w < NCH; ++w) asm volatile("" : "+v"(dv[w]));
#pragma unroll
                        for (int w = 0; w < NCH; ++w) dv[w] = dv[w] * dv[w];
#pragma unroll
                        for (int w = 0; w < NCH; ++w) asm volatile("" : "+v"(dv[w]));
#pragma unroll
                        for (int w = 0; w < NCH; ++w) dv[w] = dv[w] + B[blk][w];
                    } else {
                        // K <= 3, and K = 4, 5 at T = 1: the compiler's own
                        // interleaving measures faster.
#pragma unroll
                        for (int w = 0; w < NCH; ++w) {
                            const float d = fsub(c * G::W + qc * NCH + w, negx);
                            const float e = d * d;
                            dv[w] = e + B[blk][w];
                        }
                    }
                    if constexpr (KEYS) {
                        double kk[NCH];
#pragma unroll
                        for (int w = 0; w < NCH; ++w) kk[w] = key_of(tag[w], dv[w]);
#pragma unroll
                        for (int st = 1; st < NCH; st *= 2)
#pragma unroll
                            for (int w = 0; w < NCH; w += 2 * st) kk[w] = kmin(kk[w], kk[w + st]);
                        if (qc == 0) {
                            run[c] = kk[0];
                        } else {
                            const double kq = key_of(key_lo(kk[0]) + (uint32_t)(qc * NCH),
                                                     key_cost(kk[0]));
                            run[c] = kmin(run[c], kq);
                        }
                    } else if (qc == 0) {
                        run[c] = fmin_tree<NCH>(dv);
                    } else {
                        // the running minimum joins the chunk's tree
                        float v[NCH + 1];
#pragma unroll
                        for (int w = 0; w < NCH; ++w) v[w] = dv[w];
                        v[NCH] = run[c];
                        run[c] = fmin_tree<NCH + 1>(v);
                    }
                    if constexpr (KEYS && kEarlyPair<K, T>) {
                        if (qc == NCHUNK - 1 && c == 1 && i + 1 < nsteps)
                            lds_store_cost2<0>(lds_addr(bbuf[tt][(i + 1) & 1] + bslot<K>(jb)),
                                               run[0], run[1]);
                    }
                    if constexpr (K == 2) {
                        // K=2's 16 costs per lane leave in 16-byte quads as
                        // soon as each quad of groups is done, overlapping
                        // the LDS writes with the remaining groups (+4 %;
                        // K=3's 8 measured 2 % slower this way)
                        static_assert(NCHUNK == 1 && G::C % 4 == 0, "run[c] final per group");
                        if (c % 4 == 3 && i + 1 < nsteps) {
                            float* bq = bbuf[tt][(i + 1) & 1] + bslot<K>(jb) + (c - 3);
                            *(float4*)bq = make_float4(cost_of(run[c - 3]), cost_of(run[c - 2]),
                                                       cost_of(run[c - 1]), cost_of(run[c]));
                        }
                    }
                }
            }
            if constexpr (G::HALF) {
                // merge the two halves of the group (lanes 2t, 2t+1)
                if constexpr (KEYS) {
                    run[0] = kmin_xor1(run[0]);
                } else {
                    const float o = __int_as_float(__builtin_amdgcn_mov_dpp(
                        __float_as_int(run[0]), 0xB1, 0xF, 0xF, false));
                    run[0] = fmin2(run[0], o);
                }
            }

            if (i + 1 < nsteps) {
                float* bnext = bbuf[tt][(i + 1) & 1] + bslot<K>(jb);
                if constexpr (K == 2) {
                    // stored per quad of groups above
                } else if constexpr (KEYS && kEarlyPair<K, T>) {
                    lds_store_cost2<2>(lds_addr(bnext), run[2], run[3]);  // 0, 1 above
                } else if constexpr (KEYS && (G::C == 2 || G::C == 4)) {
                    lds_store_costs<G::C>(lds_addr(bnext), run);
                } else if constexpr (G::C == 2) {
                    *(float2*)bnext = make_float2(cost_of(run[0]), cost_of(run[1]));
                } else if constexpr (G::C % 4 == 0) {
                    // 4, 8 or 16 costs per lane: 16-byte stores keep each
                    // lane's bytes contiguous (dword pairs at a 32/64-byte
                    // lane stride would pile onto a few LDS banks).
#pragma unroll
                    for (int c = 0; c < G::C; c += 4)
                        *(float4*)(bnext + c) =
                            make_float4(cost_of(run[c]), cost_of(run[c + 1]),
                                        cost_of(run[c + 2]), cost_of(run[c + 3]));
                } else {
                    if (!G::HALF || (tl & 1) == 0) bnext[0] = cost_of(run[0]);
                }
                if constexpr (KEYS) {
                    if (i >= store_lo) {
                        // this step's backpointer row: a wave-uniform base
                        // (SGPRs) plus a 32-bit lane offset, so the store
                        // takes the SGPR-base form and no 64-bit per-lane
                        // address is carried across steps (the offset is
                        // opaque here: hoisted out of the step loop, its
                        // 64-bit extension was kept live there instead, and
                        // spilled in the column-chain kernel)
                        gbyte_t* const bprow =
                            uniform_gptr(bp + ((size_t)q * kSlots + (size_t)i) * G::BPSTEP);
                        uint32_t loff = G::HALF ? (uint32_t)jb : (uint32_t)(tl * G::UNIT);
                        asm volatile("" : "+v"(loff));
                        if constexpr (G::HALF) {
                            if ((tl & 1) == 0)
                                bprow[loff] = (uint8_t)(key_lo(run[0]) & 0x7F);
                        } else {
                            // Funnel-shift each group's K index bits (the low
                            // bits of its key tag) in from the top, one
                            // v_alignbit_b32 per group; group c ends at bits
                            // [cK, (c+1)K).
                            typedef typename UnitT<G::UNIT>::type unit_t;
                            uint32_t bits = 0;
#pragma unroll
                            for (int c = 0; c < G::C; ++c)
                                bits = __builtin_amdgcn_alignbit(key_lo(run[c]), bits, (uint32_t)K);
                            if constexpr (G::BITS < 32) bits >>= (32 - G::BITS);
                            *(__attribute__((address_space(1))) unit_t*)(bprow + loff) =
                                (unit_t)bits;
                        }
                    }
                }
            } else if constexpr (KEYS) {
                if (pinned) {
                    // Pinned end: the allowed final states are exactly group
                    // ov's candidates, so s_end = ov + argmin_w * SP.  When
                    // even the best allowed cost is +inf, cost + mask is +inf
                    // everywhere and the reference's argmin returns state 0
                    // (quantize.py:298-306).
                    const int ov = ovs[tt];
#pragma unroll
                    for (int c = 0; c < G::C; ++c)
                        if (jb + c == ov && (!G::HALF || (tl & 1) == 0)) {
                            const float m = key_cost(run[c]);
                            send[tt] = (m == __builtin_inff())
                                          ? 0
                                          : ov + (int)(key_lo(run[c]) & (uint32_t)(G::NC - 1)) *
                                                     G::SP;
                        }
                } else {
                    // Free end: lowest state index among the minimum costs.
                    // The first argmin of a group is its lowest state; across
                    // groups compare (cost, state) as one key.
                    double best = 0.0;
#pragma unroll
                    for (int c = 0; c < G::C; ++c) {
                        const uint32_t s = (uint32_t)(jb + c) +
                                           (key_lo(run[c]) & (uint32_t)(G::NC - 1)) *
                                               (uint32_t)G::SP;
                        const double kc = key_of(s, key_cost(run[c]));
                        best = (c == 0) ? kc : kmin(best, kc);
                    }
#pragma unroll
                    for (int m = 32; m >= 1; m >>= 1) best = kmin_xor(best, m);
                    if ((tid & 63) == 0) red[tid >> 6] = best;
                    __syncthreads();
                    if (tid == 0) {
                        double b = red[0];
#pragma unroll
                        for (int wv = 1; wv < kFwdThreads / 64; ++wv) b = kmin(b, red[wv]);
                        send[tt] = (int)key_lo(b);
                    }
                    __syncthreads();
                }
            }
        }
        // The cost stores above are inline ds_write2_b32 the compiler does
        // not track: complete them before the barrier publishes b_{i+1}.
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        __syncthreads();
        __builtin_amdgcn_s_setprio(kPrioTop<K>);
    };

    // Min-only steps 0 .. npre-1 (never the last step, which takes the
    // final argmin), then the key steps.
    const int npre = store_lo <= 0 ? 0 : (store_lo < nsteps - 1 ? store_lo : nsteps - 1);
    int i = 0;
    for (; i < npre; ++i) step(BoolC<false>{}, i);
    for (; i < nsteps; ++i) step(BoolC<true>{}, i);
    __builtin_amdgcn_s_setprio(0);
}

// One workgroup advances sequences blockIdx.x*T .. +T-1; ov_in NULL = free
// runs, else each run is pinned to its ov at both ends.
template <int K, int T>
__global__ __launch_bounds__(kFwdThreads) void fwd_kernel(
    const float* __restrict__ X, int xstride, int xlen, int nseq,
    const float* __restrict__ lut, int roll, int nsteps, int store_lo,
    const int32_t* __restrict__ ov_in,
    uint8_t* __restrict__ bp, int32_t* __restrict__ send, uint32_t* __restrict__ err) {
    __shared__ FwdSmem<K, T> sm;
    const int q0 = blockIdx.x * T;
    const int ntile = (nseq - q0) < T ? (nseq - q0) : T;   // sequences in this group
    const bool pinned = (ov_in != nullptr);
    if (threadIdx.x < T)
        sm.ovs[threadIdx.x] = (pinned && (int)threadIdx.x < ntile) ? ov_in[q0 + threadIdx.x] : -1;
    fwd_run<K, T>(sm, X, xstride, xlen, q0, ntile, lut, roll, nsteps, store_lo, pinned, bp,
                  send + q0, err, (int)threadIdx.x);
}

// ---------------------------------------------------------------- traceback
// The links of slots hi down to lo of one staged chunk (slot sl's row at
// stage + (sl - lo) * BPSTEP), chased by one thread from s = s_{hi+1}:
// s_sl = x + bp_sl[x] * SP with x = s_{sl+1} >> K.  Returns s_lo; stores
// st[sl] = s_sl when STORE.
//
// Written for the latency of the serial chain.  Each link reads the aligned
// 32-bit word holding group x's bits (GW groups per word) and extracts them;
// x_{sl-1} = x >> K | bp << (16 - 2K), so the next word's address is one
// shift-add of bp onto a part that depends on x alone (the bit ranges are
// disjoint), and wait -> extract -> shift-add -> load is the only dependent
// path.  The state, its store, the next x and the next word's x part are
// computed while the next load is in flight (the load after the last link
// re-reads row 0).  The values live in VGPRs: a scalar chain pays a
// readfirstlane per link.
template <int K, bool STORE>
__device__ __forceinline__ int chase_links(const uint8_t* stage, int hi, int lo, int32_t* st,
                                           int s) {
    using G = Geom<K>;
    constexpr int LC = G::HALF ? 0 : 6 - K;                 // log2 groups per unit
    constexpr int LUW = G::UNIT == 4 ? 0 : G::UNIT == 2 ? 1 : 2;  // log2 units per word
    constexpr int LGW = LC + LUW;                           // log2 groups per word
    constexpr int SB = 16 - 2 * K - LGW + 2;                // bp's shift in the next address
    static_assert(16 - 2 * K >= LGW, "bp bits above the word index's x part");
    // bit offset of group x in its word
    auto offset = [](uint32_t x) {
        return (x & ((1u << LC) - 1)) * K + ((x >> LC) & ((1u << LUW) - 1)) * (8 * G::UNIT);
    };
    int zero;
    asm volatile("v_mov_b32 %0, 0" : "=v"(zero));
    uint32_t x = (uint32_t)((s + zero) >> K) & (uint32_t)(G::SP - 1);
    uint32_t row = (uint32_t)(hi - lo) * G::BPSTEP;
    uint32_t v = *(const uint32_t*)(stage + row + ((x >> LGW) << 2));
    uint32_t sv = (uint32_t)s;
    row = row >= (uint32_t)G::BPSTEP ? row - G::BPSTEP : 0u;
    uint32_t rest = row + ((x >> (K + LGW)) << 2);
    uint32_t sh = offset(x);
    for (int sl = hi; sl >= lo; --sl) {
        const uint32_t b = __builtin_amdgcn_ubfe(v, sh, (uint32_t)K);
        uint32_t addr;
        asm("v_lshl_add_u32 %0, %1, %2, %3" : "=v"(addr) : "v"(b), "i"(SB), "v"(rest));
        v = *(const uint32_t*)(stage + addr);
        __builtin_amdgcn_sched_barrier(0);   // the link's ops stay ahead of the rest
        sv = x | (b << (16 - K));
        if constexpr (STORE) st[sl] = (int32_t)sv;
        x = (x >> K) | (b << (16 - 2 * K));
        row = row >= (uint32_t)G::BPSTEP ? row - G::BPSTEP : 0u;
        rest = row + ((x >> (K + LGW)) << 2);
        sh = offset(x);
    }
    return (int)sv;
}

// The links of slots hi .. lo, storing the states when st is non-null.
template <int K>
__device__ __forceinline__ int chase_links(const uint8_t* stage, int hi, int lo, int32_t* st,
                                           int s) {
    return st ? chase_links<K, true>(stage, hi, lo, st, s)
              : chase_links<K, false>(stage, hi, lo, st, s);
}

// Traceback of one sequence by the calling workgroup: from cur = s_{nsteps-1}
// (shared; set by the caller before a barrier) down to step `stop`.  The
// backpointer slots stop .. nsteps-2 (slot i-1 links s_i to s_{i-1}) are
// staged through `stage` in coalesced 16-byte loads by all threads, and one
// thread chases the links in LDS.  On return (after a barrier) cur = s_stop
// and st[i] = s_i for stop <= i <= nsteps-2 when st is non-null.
template <int K>
__device__ __forceinline__ void tb_chase(const uint8_t* __restrict__ bpq, int nsteps, int stop,
                                         uint4* stage, int stage_bytes, int32_t* st,
                                         int32_t& cur) {
    using G = Geom<K>;
    const int tid = threadIdx.x, nthr = blockDim.x;
    const int ch = stage_bytes / G::BPSTEP;  // slots per staged chunk
    for (int hi = nsteps - 2; hi >= stop; ) {
        const int lo = (hi - ch + 1 > stop) ? hi - ch + 1 : stop;
        const int n16 = (hi - lo + 1) * (G::BPSTEP / 16);
        const uint4* src = (const uint4*)(bpq + (size_t)lo * G::BPSTEP);
        __syncthreads();
        for (int k = tid; k < n16; k += nthr) stage[k] = src[k];
        __syncthreads();
        if (tid == 0) cur = chase_links<K>((const uint8_t*)stage, hi, lo, st, cur);
        hi = lo - 1;
    }
    __syncthreads();
}

// tb_chase for a 1024-thread workgroup with a fixed 64 KiB staging area and
// the next two chunks' loads in flight in registers while thread 0 chases
// the current chunk (per chunk: store, barrier, issue the load two chunks
// ahead, chase), so the chase rather than the load latency sets the pace.
// Same contract as tb_chase.
constexpr int kTbStage = 65536;

// Loads chunk c (slots lo .. hi, 64 KiB at most) of a tb_chase_pf run into
// this thread's four registers.
template <int K>
__device__ __forceinline__ void tb_chunk_load(const uint8_t* __restrict__ bpq, int nsteps,
                                              int stop, int nc, int c, int tid, uint4& r0,
                                              uint4& r1, uint4& r2, uint4& r3) {
    using G = Geom<K>;
    constexpr int CH = kTbStage / G::BPSTEP;
    if (c >= nc) return;
    const int hi = nsteps - 2 - c * CH, lo = (hi - CH + 1 > stop) ? hi - CH + 1 : stop;
    const int n16 = (hi - lo + 1) * (G::BPSTEP / 16);
    const uint4* src = (const uint4*)(bpq + (size_t)lo * G::BPSTEP);
    if (tid < n16) r0 = src[tid];
    if (tid + kFwdThreads < n16) r1 = src[tid + kFwdThreads];
    if (tid + 2 * kFwdThreads < n16) r2 = src[tid + 2 * kFwdThreads];
    if (tid + 3 * kFwdThreads < n16) r3 = src[tid + 3 * kFwdThreads];
}

template <int K>
__device__ __forceinline__ void tb_chase_pf(const uint8_t* __restrict__ bpq, int nsteps,
                                            int stop, uint4* stage, int32_t* st,
                                            int32_t& cur) {
    using G = Geom<K>;
    constexpr int CH = kTbStage / G::BPSTEP;           // slots per chunk
    static_assert(kTbStage / 16 == 4 * kFwdThreads, "four uint4 per thread per chunk");
    const int tid = threadIdx.x;
    const int nc = (nsteps - 1 - stop + CH - 1) / CH;  // slots stop .. nsteps-2
    uint4 a0, a1, a2, a3, b0, b1, b2, b3;
    tb_chunk_load<K>(bpq, nsteps, stop, nc, 0, tid, a0, a1, a2, a3);
    tb_chunk_load<K>(bpq, nsteps, stop, nc, 1, tid, b0, b1, b2, b3);
    for (int c = 0; c < nc; ++c) {
        const int hi = nsteps - 2 - c * CH, lo = (hi - CH + 1 > stop) ? hi - CH + 1 : stop;
        const int n16 = (hi - lo + 1) * (G::BPSTEP / 16);
        __syncthreads();                                // previous chase done with stage
        if (tid < n16) stage[tid] = a0;
        if (tid + kFwdThreads < n16) stage[tid + kFwdThreads] = a1;
        if (tid + 2 * kFwdThreads < n16) stage[tid + 2 * kFwdThreads] = a2;
        if (tid + 3 * kFwdThreads < n16) stage[tid + 3 * kFwdThreads] = a3;
        __syncthreads();
        a0 = b0; a1 = b1; a2 = b2; a3 = b3;
        tb_chunk_load<K>(bpq, nsteps, stop, nc, c + 2, tid, b0, b1, b2, b3);
        if (tid == 0) cur = chase_links<K>((const uint8_t*)stage, hi, lo, st, cur);
    }
    __syncthreads();
}

// Word wd of one sequence's packed EXL3 trellis, from its states st[0..255]:
// symbol t = s_t mod 2^K at stream bits [tK, (t+1)K), MSB first; 32-bit
// words MSB first (quantize.py:360-378).
template <int K, typename S>
__device__ __forceinline__ uint32_t pack_word(const S* st, int wd) {
    uint32_t word = 0;
    for (int bb = 0; bb < 32; ++bb) {
        const int b = wd * 32 + bb, t = b / K, k = b - t * K;
        word |= (((uint32_t)st[t] >> (K - 1 - k)) & 1u) << (31 - bb);
    }
    return word;
}

// Stores a packed word as the int16 pair [low half, high half].
__device__ __forceinline__ void store_word(int16_t* o, uint32_t word) {
    o[0] = (int16_t)(uint16_t)(word & 0xFFFFu);
    o[1] = (int16_t)(uint16_t)(word >> 16);
}

template <int K>
__global__ __launch_bounds__(kTbThreads) void tb_kernel(
    const uint8_t* __restrict__ bp, const int32_t* __restrict__ send, int nsteps, int stop,
    int shift, int32_t* __restrict__ sout, int32_t* __restrict__ states,
    int16_t* __restrict__ trellis) {
    using G = Geom<K>;
    constexpr int STAGE = 32768;
    __shared__ uint4 stage[STAGE / 16];
    __shared__ int32_t st[kSteps];
    __shared__ int32_t cur;

    const int q = blockIdx.x, tid = threadIdx.x;
    const uint8_t* bpq = bp + (size_t)q * ((size_t)kSlots * G::BPSTEP);
    const bool keep = (states != nullptr) || (trellis != nullptr);
    if (tid == 0) {
        cur = send[q] & 0xFFFF;
        if (keep) st[nsteps - 1] = cur;
    }
    tb_chase<K>(bpq, nsteps, stop, stage, STAGE, keep ? st : nullptr, cur);
    if (sout && tid == 0) sout[q] = cur >> shift;
    if (states) {
        for (int t = tid; t < nsteps; t += kTbThreads) states[(size_t)q * nsteps + t] = st[t];
    }
    if (trellis && nsteps == kSteps) {
        for (int wd = tid; wd < 8 * K; wd += kTbThreads)
            store_word(trellis + (size_t)q * 16 * K + 2 * wd, pack_word<K>(st, wd));
    }
}

// Traceback with one lane per sequence, for large batches: each lane chases
// its sequence's links with dependent loads of just the backpointer unit
// each step needs (1-4 bytes) instead of staging whole rows, so HBM reads
// drop from 255 x BPSTEP bytes per sequence to one cache line per step; the
// chase is latency-bound per sequence but all sequences chase at once.
// States collect in LDS (odd dword row stride: conflict-free) and leave
// coalesced, as states and/or the packed trellis.
constexpr int kTbLaneSeqs = 64;

template <int K>
__global__ __launch_bounds__(kTbLaneSeqs) void tb_lane_kernel(
    const uint8_t* __restrict__ bp, int nseq, const int32_t* __restrict__ send, int nsteps,
    int stop, int shift, int32_t* __restrict__ sout, int32_t* __restrict__ states,
    int16_t* __restrict__ trellis) {
    using G = Geom<K>;
    constexpr int ROW = kSteps + 2;
    __shared__ uint16_t st[kTbLaneSeqs][ROW];
    const int l = threadIdx.x;
    const int q0 = blockIdx.x * kTbLaneSeqs;
    const int q = q0 + l;
    const bool keep = (states != nullptr) || (trellis != nullptr);
    if (q < nseq) {
        int s = send[q] & 0xFFFF;
        if (keep) st[l][nsteps - 1] = (uint16_t)s;
        const uint8_t* bpq = bp + (size_t)q * ((size_t)kSlots * G::BPSTEP);
        for (int sl = nsteps - 2; sl >= stop; --sl) {
            const int j = (s >> K) & (G::SP - 1);
            s = j + bp_lookup<K>(bpq + (size_t)sl * G::BPSTEP, j) * G::SP;
            if (keep) st[l][sl] = (uint16_t)s;
        }
        if (sout) sout[q] = s >> shift;
    }
    __syncthreads();
    const int nt = (nseq - q0) < kTbLaneSeqs ? (nseq - q0) : kTbLaneSeqs;
    if (states) {
        for (int t = 0; t < nt; ++t)
            for (int e = l; e < nsteps; e += kTbLaneSeqs)
                states[(size_t)(q0 + t) * nsteps + e] = st[t][e];
    }
    if (trellis && nsteps == kSteps) {
        for (int idx = l; idx < nt * 8 * K; idx += kTbLaneSeqs) {
            const int t = idx / (8 * K), wd = idx - t * (8 * K);
            store_word(trellis + (size_t)(q0 + t) * 16 * K + 2 * wd, pack_word<K>(st[t], wd));
        }
    }
}

// ------------------------------------------------- deferred-argmin encode
// The batched forward of fwd_run without the argmin: its min tree takes the
// group minima of the fp32 costs alone (v_min3_f32 / v_min_f32, half an
// instruction per candidate against fwd_run's v_min_f64 on a 64-bit
// (cost, index) key), and each step's minima b_{i+1} go to LDS for the next
// step and, for steps store_lo .. nsteps-2, to HBM: one row of SP floats per
// step in `bm` (Geom<K>::SP * 4 bytes, kSlots rows per sequence, row r
// holding b_r).  The traceback (tb_defer_kernel) then recomputes, for the one
// group on the path at each link, the costs of its NC candidates from b_{i-1},
// the codebook and x_{i-1} with the forward's own fp32 operations, and takes
// the first index of their minimum -- the reference's tie rule
// (quantize.py:288-292,316-319).  The final state (the argmin of the last
// step) is found after the step loop from b_{nsteps-1}, which stays in LDS.
//
// Worth it where the minima rows are small enough to write: SP * 4 bytes per
// tile-step is 16 KiB at K=4 (8 times the packed backpointers) and 2 KiB at
// K=7; K = 2, 3 would write 64 / 32 KiB per tile-step, more than HBM takes at
// the forward's rate, so they keep fwd_run.
// Minima rows kept per sequence (row r holds b_r, r = 1 .. 254) and their
// bytes per sequence.
template <int K>
constexpr size_t defer_tile_bytes() {
    return (size_t)kSlots * Geom<K>::SP * sizeof(float);
}

// Forward DP of sequences q0 .. q0+ntile-1 by one 1024-thread workgroup with
// the argmin deferred to the traceback (see above).  Arguments as fwd_run,
// with bm the minima rows (defer_tile_bytes<K>() per sequence).
template <int K, int T>
__device__ __forceinline__ void fwd_run_defer(
    FwdSmem<K, T>& sm, const float* __restrict__ X, int xstride, int xlen, int q0, int ntile,
    const float* __restrict__ lut, int roll, int nsteps, int store_lo, bool pinned,
    float* __restrict__ bm, int32_t* send, uint32_t* __restrict__ err, int tid) {
    using G = Geom<K>;
    static_assert(K >= 4, "K = 2, 3 keep the key-argmin forward");
    static_assert(G::NB == 1, "one predecessor block per thread");
    auto& bbuf = sm.bbuf;
    auto& xs = sm.xs;
    auto& ovs = sm.ovs;
    auto& red = sm.red;

#pragma unroll
    for (int r0 = 0; r0 < T * kSteps; r0 += kFwdThreads) {
        if (r0 + kFwdThreads <= T * kSteps || tid < T * kSteps - r0) {
            const int idx = r0 + tid, tt = idx / kSteps, e = idx % kSteps;
            float v = 0.0f;
            if (tt < ntile && e < xlen) {
                v = X[(size_t)(q0 + tt) * xstride + e];
                if (v != v) atomicOr(err, 1u);
            }
            xs[tt][e] = v;
        }
    }

    const int jbase = G::HALF ? (tid >> 1) : tid * G::C;
    const int wbase = G::HALF ? (tid & 1) * G::W : 0;
    constexpr int NCH = kChunkW<K, T>;
    constexpr int NCHUNK = G::W / NCH;
    float f32[G::NSTATE];
#pragma unroll
    for (int l = 0; l < G::NSTATE; ++l)
        f32[l] = lut[jbase + l / G::W + (wbase + l % G::W) * G::SP];
    auto fsub = [&](int l, float negx) { return f32[l] + negx; };
    __syncthreads();

    for (int tt = 0; tt < T; ++tt) {
        const int ov = ovs[tt];
        if (!G::HALF || (tid & 1) == 0) {
#pragma unroll
            for (int c = 0; c < G::C; ++c) {
                const int j = jbase + c;
                bbuf[tt][0][bslot<K>(j)] = (ov < 0 || j == ov) ? 0.0f : __builtin_inff();
            }
        }
    }
    __syncthreads();

    const int a0 = jbase >> K;
    const int rpad = bslot<K>(a0 + wbase * G::Q) - (a0 + wbase * G::Q);
    // b_{i+1} of the last step is never stored (the final state is found
    // from LDS below); rows store_lo .. nsteps-2 are
    const int last_row = nsteps - 2;
    for (int i = 0; i + 1 < nsteps; ++i) {
        const int u = (i - roll < 0) ? i - roll + xlen : i - roll;
#pragma unroll 1
        for (int tt = 0; tt < ntile; ++tt) {
#pragma unroll
            for (int l = 0; l < G::NSTATE; ++l) asm volatile("" : "+v"(f32[l]));
            const int q = q0 + tt;
            const float negx = -__int_as_float(
                __builtin_amdgcn_readfirstlane(__float_as_int(xs[tt][u])));
            const float* bcur = bbuf[tt][i & 1];
            float run[G::C];
#pragma unroll
            for (int qc = 0; qc < NCHUNK; ++qc) {
                float B[G::NB][NCH];
#pragma unroll
                for (int w = 0; w < NCH; ++w) {
                    const float* src = bcur + a0 + rpad + (wbase + qc * NCH + w) * G::Q;
                    B[0][w] = src[0];
                }
#pragma unroll
                for (int c = 0; c < G::C; ++c) {
                    constexpr int U = T * NCHUNK * G::C;
                    const int pos = (tt * NCHUNK + qc) * G::C + c;
                    constexpr int D1 = K >= 5 ? U * 5 / 8 : T == 1 ? U / 4 : U / 2;
                    constexpr int D0 = K >= 5 ? U * 7 / 8 : K == 4 && T == 1 ? U * 5 / 8
                                                                              : U * 3 / 4;
                    if (pos == D1) __builtin_amdgcn_s_setprio(1);
                    if (pos == D0) __builtin_amdgcn_s_setprio(0);
                    float dv[NCH];
                    if constexpr (kGroupOps<K, T>) {
#pragma unroll
                        for (int w = 0; w < NCH; ++w) dv[w] = fsub(c * G::W + qc * NCH + w, negx);
#pragma unroll
                        for (int w = 0; w < NCH; ++w) asm volatile("" : "+v"(dv[w]));
#pragma unroll
                        for (int w = 0; w < NCH; ++w) dv[w] = dv[w] * dv[w];
#pragma unroll
                        for (int w = 0; w < NCH; ++w) asm volatile("" : "+v"(dv[w]));
#pragma unroll
                        for (int w = 0; w < NCH; ++w) dv[w] = dv[w] + B[0][w];
                    } else {
#pragma unroll
                        for (int w = 0; w < NCH; ++w) {
                            const float d = fsub(c * G::W + qc * NCH + w, negx);
                            dv[w] = d * d + B[0][w];
                        }
                    }
                    const float m = fmin_tree<NCH>(dv);
                    run[c] = (qc == 0) ? m : fmin2(run[c], m);
                }
            }
            if constexpr (G::HALF) {
                // merge the two halves of the group (lanes 2t, 2t+1) with a
                // DPP quad permutation [1,0,3,2]
                const float o = __int_as_float(__builtin_amdgcn_mov_dpp(
                    __float_as_int(run[0]), 0xB1, 0xF, 0xF, false));
                run[0] = fmin2(run[0], o);
            }
            float* bnext = bbuf[tt][(i + 1) & 1] + bslot<K>(jbase);
            if constexpr (G::C == 4) {
                *(float4*)bnext = make_float4(run[0], run[1], run[2], run[3]);
            } else if constexpr (G::C == 2) {
                *(float2*)bnext = make_float2(run[0], run[1]);
            } else {
                if (!G::HALF || (tid & 1) == 0) bnext[0] = run[0];
            }
            if (i + 1 >= store_lo && i + 1 <= last_row) {
                // row i+1 of this sequence: a wave-uniform base plus the
                // lane's offset; streamed past the caches (read back only by
                // the traceback, after the launch)
                gbyte_t* const row = uniform_gptr(
                    (uint8_t*)(bm + ((size_t)q * kSlots + (size_t)(i + 1)) * G::SP));
                gbyte_t* const dst = row + (uint32_t)jbase * 4u;
                typedef float v4f __attribute__((ext_vector_type(4)));
                typedef float v2f __attribute__((ext_vector_type(2)));
                if constexpr (G::C == 4) {
                    const v4f v = {run[0], run[1], run[2], run[3]};
                    __builtin_nontemporal_store(v, (__attribute__((address_space(1))) v4f*)dst);
                } else if constexpr (G::C == 2) {
                    const v2f v = {run[0], run[1]};
                    __builtin_nontemporal_store(v, (__attribute__((address_space(1))) v2f*)dst);
                } else {
                    if (!G::HALF || (tid & 1) == 0)
                        __builtin_nontemporal_store(
                            run[0], (__attribute__((address_space(1))) float*)dst);
                }
            }
        }
        __syncthreads();
        __builtin_amdgcn_s_setprio(kPrioTop<K>);
    }
    __builtin_amdgcn_s_setprio(0);

    // The last step: c[s] = fl(fl(fl(f[s] - x)^2) + b_{nsteps-1}[s >> K]), then
    // the final state -- pinned: the first minimum among the states with
    // s mod SP == ov (state 0 when every allowed cost is +inf,
    // quantize.py:298-306); free: the lowest state index among the minimum
    // costs (quantize.py:306,315).  Thread t takes states t + 1024 k with the
    // codebook read from the table (its registers are free by now) and
    // (cost, state) 64-bit keys, whose fp64 order is the lexicographic one.
    const int ul = (nsteps - 1 - roll < 0) ? nsteps - 1 - roll + xlen : nsteps - 1 - roll;
    for (int tt = 0; tt < ntile; ++tt) {
        const float negx = -xs[tt][ul];
        const float* bcur = bbuf[tt][(nsteps - 1) & 1];
        const int ov = ovs[tt];
        double best = key_of(0xFFFFFFFFu, __builtin_inff());
#pragma unroll 8
        for (int k = 0; k < 65536 / kFwdThreads; ++k) {
            const int st_ = tid + k * kFwdThreads;
            const float f = lut[st_];
            const float d = f + negx;
            const float cost = d * d + bcur[bslot<K>(st_ >> K)];
            const bool allowed = !pinned || ((st_ & (G::SP - 1)) == ov);
            best = kmin(best, key_of((uint32_t)st_, allowed ? cost : __builtin_inff()));
        }
#pragma unroll
        for (int m = 32; m >= 1; m >>= 1) best = kmin_xor(best, m);
        if ((tid & 63) == 0) red[tid >> 6] = best;
        __syncthreads();
        if (tid == 0) {
            double b = red[0];
#pragma unroll
            for (int wv = 1; wv < kFwdThreads / 64; ++wv) b = kmin(b, red[wv]);
            // pinned: an all-+inf allowed group leaves the minimum at +inf and
            // the reference's argmin returns state 0
            send[tt] = (pinned && key_cost(b) == __builtin_inff()) ? 0 : (int)key_lo(b);
        }
        __syncthreads();
    }
}

template <int K, int T>
__global__ __launch_bounds__(kFwdThreads) void fwd_defer_kernel(
    const float* __restrict__ X, int xstride, int xlen, int nseq,
    const float* __restrict__ lut, int roll, int nsteps, int store_lo,
    const int32_t* __restrict__ ov_in, float* __restrict__ bm, int32_t* __restrict__ send,
    uint32_t* __restrict__ err) {
    __shared__ FwdSmem<K, T> sm;
    const int q0 = blockIdx.x * T;
    const int ntile = (nseq - q0) < T ? (nseq - q0) : T;
    const bool pinned = (ov_in != nullptr);
    if (threadIdx.x < T)
        sm.ovs[threadIdx.x] = (pinned && (int)threadIdx.x < ntile) ? ov_in[q0 + threadIdx.x] : -1;
    fwd_run_defer<K, T>(sm, X, xstride, xlen, q0, ntile, lut, roll, nsteps, store_lo, pinned,
                        bm, send + q0, err, (int)threadIdx.x);
}

// Traceback of the deferred-argmin forward, one lane per sequence: from
// s = send[q] (the state at step nsteps-1) down to step `stop`; at link i
// the group j = s_i >> K's NC candidates s' = j + w SP cost
// fl(fl(fl(f[s'] - x_{i-1})^2) + b_{i-1}[(j >> K) + w Q]) with b_{i-1} from
// row i-1 of bm (or the start mask when i-1 = 0: 0, or 0 / +inf around the
// pin ov_in[q]); s_{i-1} = j + w* SP for the first w of the minimum.
// Targets x_t of step t are X[q][(t - roll) mod xlen].  Outputs as
// tb_lane_kernel.
constexpr int kTbDeferChunk = 16;     // candidates recomputed per batch of loads

template <int K>
__global__ __launch_bounds__(kTbLaneSeqs) void tb_defer_kernel(
    const float* __restrict__ bm, const float* __restrict__ X, int xstride, int xlen, int roll,
    const float* __restrict__ lut, int nseq, const int32_t* __restrict__ send,
    const int32_t* __restrict__ ov_in, int nsteps, int stop, int shift,
    int32_t* __restrict__ sout, int32_t* __restrict__ states, int16_t* __restrict__ trellis) {
    using G = Geom<K>;
    constexpr int ROW = kSteps + 2;
    constexpr int CH = G::NC < kTbDeferChunk ? G::NC : kTbDeferChunk;
    __shared__ uint16_t st[kTbLaneSeqs][ROW];
    const int l = threadIdx.x;
    const int q0 = blockIdx.x * kTbLaneSeqs;
    const int q = q0 + l;
    const bool keep = (states != nullptr) || (trellis != nullptr);
    if (q < nseq) {
        int s = send[q] & 0xFFFF;
        if (keep) st[l][nsteps - 1] = (uint16_t)s;
        const float* xq = X + (size_t)q * xstride;
        const float* bq = bm + (size_t)q * kSlots * G::SP;
        const int ov = ov_in ? ov_in[q] : -1;
        for (int i = nsteps - 1; i > stop; --i) {
            const int j = (s >> K) & (G::SP - 1);
            const int a = j >> K;
            const int u = (i - 1 - roll < 0) ? i - 1 - roll + xlen : i - 1 - roll;
            const float negx = -xq[u];
            const float* brow = bq + (size_t)(i - 1) * G::SP + a;
            float best = 0.0f;
            int bw = 0;
#pragma unroll 1
            for (int w0 = 0; w0 < G::NC; w0 += CH) {
                float bv[CH], f[CH];
#pragma unroll
                for (int w = 0; w < CH; ++w) {
                    const int g = a + (w0 + w) * G::Q;
                    bv[w] = (i - 1 == 0) ? ((ov < 0 || g == ov) ? 0.0f : __builtin_inff())
                                         : brow[(w0 + w) * G::Q];
                    f[w] = lut[j + (w0 + w) * G::SP];
                }
#pragma unroll
                for (int w = 0; w < CH; ++w) {
                    const float d = f[w] + negx;
                    const float c = d * d + bv[w];
                    if ((w0 == 0 && w == 0) || c < best) {
                        best = c;
                        bw = w0 + w;
                    }
                }
            }
            s = j + bw * G::SP;
            if (keep) st[l][i - 1] = (uint16_t)s;
        }
        if (sout) sout[q] = s >> shift;
    }
    __syncthreads();
    const int nt = (nseq - q0) < kTbLaneSeqs ? (nseq - q0) : kTbLaneSeqs;
    if (states) {
        for (int t = 0; t < nt; ++t)
            for (int e = l; e < nsteps; e += kTbLaneSeqs)
                states[(size_t)(q0 + t) * nsteps + e] = st[t][e];
    }
    if (trellis && nsteps == kSteps) {
        for (int idx = l; idx < nt * 8 * K; idx += kTbLaneSeqs) {
            const int t = idx / (8 * K), wd = idx - t * (8 * K);
            store_word(trellis + (size_t)(q0 + t) * 16 * K + 2 * wd, pack_word<K>(st[t], wd));
        }
    }
}

// ------------------------------------------------------ fused tail-bite
// Both QTIP passes of n sequences in one launch of 2n single-sequence
// workgroups, for batches too small to fill the GPU twice over (the 16-row
// blocks of the BlockLDLQ sweep: 64..384 tiles on 256 CUs).  Each workgroup
// takes the next task from an atomic counter: tasks 0..n-1 run pass 1 (free
// run of the rolled sequence, n1 steps) and trace it back inside the
// workgroup to ov = s_pivot >> K, published with a release store of the
// launch's epoch into flags[q]; tasks n..2n-1 wait for that flag (acquire)
// and run pass 2 pinned to ov.  Tasks are taken in start order, so a pass-2
// task only ever waits for a pass-1 task that is already running: the wait
// always ends.  It is also bounded (spin_limit polls, err |= 2 on expiry)
// so that an unexpected stall ends the launch with an error instead of a
// hang.  With n = 320 on 256 CUs the 640 passes fill 3 rounds instead of the
// 4 of two separate launches.  Pass-2 backpointers reuse the sequence's
// pass-1 slots (pass 1 has finished reading them before it publishes); the
// pass-2 traceback runs as tb_kernel afterwards.
template <int K>
__global__ __launch_bounds__(kFwdThreads) void tailbite_fused_kernel(
    const float* __restrict__ X, int nseq, const float* __restrict__ lut, int pivot,
    int n1, uint8_t* __restrict__ bp, int32_t* __restrict__ send, int32_t* __restrict__ ovbuf,
    uint32_t* __restrict__ flags, int32_t* __restrict__ counter, uint32_t epoch,
    int spin_limit, uint32_t* __restrict__ err) {
    using G = Geom<K>;
    __shared__ FwdSmem<K, 1> sm;
    __shared__ int32_t task, cur;
    const int tid = threadIdx.x;
    if (tid == 0) task = atomicAdd(counter, 1);
    __syncthreads();
    const int t = task;
    if (t >= 2 * nseq) {                       // cannot happen with a reset counter
        if (tid == 0) atomicOr(err, 4u);
        return;
    }
    if (t < nseq) {
        if (tid == 0) sm.ovs[0] = -1;
        fwd_run<K, 1>(sm, X, kSteps, kSteps, t, 1, lut, pivot, n1, pivot, false, bp, &cur,
                      err, tid);
        // This workgroup's backpointer stores reach L2 (and are written back
        // past it, since pass 2 of this sequence may run on another XCD and
        // overwrite them) before any thread reads them back.
        __threadfence();
        __syncthreads();
        const uint8_t* bpq = bp + (size_t)t * ((size_t)kSlots * G::BPSTEP);
        tb_chase<K>(bpq, n1, pivot, (uint4*)&sm.bbuf[0][0][0], (int)sizeof(sm.bbuf), nullptr,
                    cur);
        if (tid == 0) {
            __hip_atomic_store(&ovbuf[t], cur >> K, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __hip_atomic_store(&flags[t], epoch, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_AGENT);
        }
    } else {
        const int q = t - nseq;
        if (tid == 0) {
            int ov = -1;
            for (int it = 0;; ++it) {
                if (__hip_atomic_load(&flags[q], __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_AGENT) ==
                    epoch) {
                    ov = __hip_atomic_load(&ovbuf[q], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                    break;
                }
                if (it >= spin_limit) {
                    atomicOr(err, 2u);
                    break;
                }
                __builtin_amdgcn_s_sleep(8);
            }
            sm.ovs[0] = ov;
        }
        __syncthreads();
        if (sm.ovs[0] < 0) return;             // wait expired: reported through err
        fwd_run<K, 1>(sm, X, kSteps, kSteps, q, 1, lut, 0, kSteps, 0, true, bp, send + q,
                      err, tid);
    }
}

// Resets the fused kernel's task counter (a kernel rather than a memset so
// the sequence stays capturable in a HIP graph).
__global__ void reset_counter_kernel(int32_t* counter) { *counter = 0; }

// p[0..n) = v, one word per thread (flags and status words of reused
// scratch; a kernel rather than a memset, as above).
__global__ void fill_u32_kernel(uint32_t* __restrict__ p, uint32_t n, uint32_t v) {
    const uint32_t i = blockIdx.x * 256u + threadIdx.x;
    if (i < n) p[i] = v;
}

// ------------------------------------------------- decode / pack / unpack
// tensor_core_perm (quantize.py:101-118): element t -> row-major 16x16 index.
__device__ __forceinline__ int tc_perm(int t) {
    const int g = t >> 3, e = t & 7;
    const int r0 = (g & 3) * 2, c0 = g >> 2;
    const int rr = (e & 1) + ((e & 2) ? 8 : 0);
    const int cc = (e & 4) ? 8 : 0;
    return (r0 + rr) * 16 + c0 + cc;
}

// 16-bit circular window of the 256K-bit stream ending at bit (t+1)K - 1.
template <int K>
__device__ __forceinline__ uint32_t window_state(const uint32_t* words, int t) {
    constexpr int NB = 256 * K;
    int b = t * K + K - 16;
    if (b < 0) b += NB;
    uint32_t v = 0;
#pragma unroll
    for (int k = 0; k < 16; ++k) {
        int bb = b + k;
        if (bb >= NB) bb -= NB;
        v = (v << 1) | ((words[bb >> 5] >> (31 - (bb & 31))) & 1u);
    }
    return v;
}

template <int K>
__global__ __launch_bounds__(256) void decode_kernel(
    const int16_t* __restrict__ trellis, int tn, const float* __restrict__ lut,
    float* __restrict__ out_f32, uint16_t* __restrict__ out_f16) {
    __shared__ uint32_t words[8 * K];
    const int tile = blockIdx.x, t = threadIdx.x;
    const uint32_t* src = (const uint32_t*)(trellis + (size_t)tile * 16 * K);
    if (t < 8 * K) words[t] = src[t];  // int16 pair [lo, hi] == little-endian u32
    __syncthreads();
    const uint32_t s = window_state<K>(words, t);
    const int p = tc_perm(t);
    const int a = tile / tn, b = tile - a * tn;
    const size_t n = (size_t)tn * 16;
    const size_t idx = (size_t)(16 * a + (p >> 4)) * n + 16 * b + (p & 15);
    const float v = lut[s];
    if (out_f32) out_f32[idx] = v;
    if (out_f16) out_f16[idx] = __builtin_bit_cast(uint16_t, (_Float16)v);
}

template <int K>
__global__ __launch_bounds__(256) void unpack_kernel(const int16_t* __restrict__ trellis,
                                                     int32_t* __restrict__ states) {
    __shared__ uint32_t words[8 * K];
    const int tile = blockIdx.x, t = threadIdx.x;
    const uint32_t* src = (const uint32_t*)(trellis + (size_t)tile * 16 * K);
    if (t < 8 * K) words[t] = src[t];
    __syncthreads();
    states[(size_t)tile * kSteps + t] = (int32_t)window_state<K>(words, t);
}

template <int K>
__global__ __launch_bounds__(64) void pack_kernel(const int32_t* __restrict__ states,
                                                  int16_t* __restrict__ trellis) {
    const int tile = blockIdx.x, wd = threadIdx.x;
    if (wd >= 8 * K) return;
    store_word(trellis + (size_t)tile * 16 * K + 2 * wd,
               pack_word<K>(states + (size_t)tile * kSteps, wd));
}

// ------------------------------------------------- BlockLDLQ column chains
// The whole BlockLDLQ sweep (quantize.py:631-746) as one persistent launch.
// The feedback of 16-row block i only mixes rows within an output column:
// tile (i, j)'s targets are
//     X[r][c] = W[16i+r][16j+c] + sum_{m >= 16(i+1)} L[m][16i+r] * E[m][16j+c],
//     E = W - What  (the error of the tiles already quantized),
// so tile (i, j) depends only on tile (i+1, j): the columns are independent
// chains.  Each of the persistent workgroups takes tile tasks from an atomic
// counter in sweep order (block tk-1 first), waits (acquire, bounded) for
// the previous tile of its chain, (i+1, j), computes the targets (the L and E column
// blocks read in the matrix-core operand layout described below), runs
// both tail-biting passes with in-workgroup tracebacks,
// writes the states, the packed trellis, What and E for the tile, and
// publishes the tile by storing the launch's epoch into its flag once E's
// write-through stores have completed.  A task
// only waits for a task taken before it, whose workgroup is running, so the
// waits always end; columns advance independently, so the GPU is not left
// half idle at the end of every block the way block-synchronous launches of
// tn tiles are.
//
// The feedback is summed in the reference's own order, so that a tile's
// targets are bit-identical to the reference's for the same W and L
// (quantize.py:662-686,743-744).  The reference sweeps the blocks in
// buffers of pb = buf_cols/16 blocks aligned to the bottom block row
// (buffer q holds blocks tk-pb(q+1) .. tk-pb*q-1) and computes block i of
// buffer q(i) as
//     X = (W + L[rows of buffer q(i) below i]^T E) + prod,
//     prod = (..((0 + P_0) + P_1) + ..) + P_{q(i)-1},  P_q = L[rows of q]^T E,
// dropping the first term for the buffer's first block; torch's CPU GEMM
// (MKL sgemm) accumulates every such product of inner dimension <= 128 as
// one fp32 fused multiply-add chain over the rows in ascending order, from
// zero.  Here each buffer's 16x16 chain runs on the matrix cores:
// v_mfma_f32_16x16x1f32 multiplies four independent 16x1 by 1x16 blocks
// and adds each product to its accumulator with one rounding -- a fused
// multiply-add per output per step -- so block b of a wave accumulates
// buffer b's chain in m order exactly.  A round covers 64 buffers (4 per
// wave); the 256 partials of each buffer go to LDS and 256 threads fold
// them into prod in buffer order.
//
// Feedback loads in flight per lane: one block of 16 rows (4 m-quads of L
// and E).  A full round is bound by the matrix cores: 4 waves x 128
// dependent 16x16x1 MFMAs per SIMD.
constexpr int kFbBlk = 4;          // m-quads per block

typedef float v4f __attribute__((ext_vector_type(4)));
typedef float v16f __attribute__((ext_vector_type(16)));

// One wave's feedback chains of a round: block blk of the accumulator is
// buffer bw + blk, and lane (blk, rc) feeds row rc of L and column rc of E
// of that buffer, m-quad mq (4 consecutive m, one 16-byte load of each) at
// byte offset off0 + 256 mq from the wave-uniform bases lb and eb; nqw
// (wave-uniform) m-quads, kFbDepth of them in flight.  The four MFMAs of an
// m-quad add rows m, m+1, m+2, m+3 in that order, so every accumulator is
// one fused multiply-add chain over its buffer's rows in ascending order.
// RAGGED: the lane's own buffer ends after nq <= nqw m-quads (block i's
// partial buffer, or none); its loads past nq re-read its last valid m-quad
// (every address stays inside the matrices) and the values are zeroed where
// they are used, so the extra products leave the chain unchanged.  Zeroing
// them at the load instead would make every load wait for itself.
template <bool RAGGED>
__device__ __forceinline__ v16f fb_chain(const gbyte_t* lb, const gbyte_t* eb, uint32_t off0,
                                         int nq, int nqw) {
    typedef __attribute__((address_space(1))) const v4f gv4_t;
    const v4f z = {0.0f, 0.0f, 0.0f, 0.0f};
    v16f acc;
#pragma unroll
    for (int v = 0; v < 16; ++v) acc[v] = 0.0f;
    // nqw is a whole number nb of blocks (m-quads of whole 16-row blocks)
    const int nb = nqw / kFbBlk;
    auto off = [&](int mq) -> uint32_t {
        if constexpr (RAGGED) {
            const int mc = mq < nq ? mq : (nq > 0 ? nq - 1 : 0);
            return off0 + 256u * (uint32_t)mc;
        } else {
            return off0 + 256u * (uint32_t)mq;
        }
    };
    v4f ra[kFbBlk], re[kFbBlk];
    // m-quad mq into slot u; past the last block it re-reads the last one
    // (never used), so that no load is conditional
    auto load = [&](int u, int bb) __attribute__((always_inline)) {
        const int bc = bb < nb ? bb : nb - 1;
        ra[u] = *(gv4_t*)(lb + off(bc * kFbBlk + u));
        re[u] = *(gv4_t*)(eb + off(bc * kFbBlk + u));
    };
    // A slot is refilled (with the same m-quad of the next block) right
    // after its MFMAs have read it, into the same registers; the scheduling
    // barriers keep each refill there (the compiler would otherwise sink
    // the loads to the end of the block, next to their use).  Every path
    // into the loop has the same loads outstanding, so each wait is for one
    // slot only.
#pragma unroll
    for (int u = 0; u < kFbBlk; ++u) load(u, 0);
    for (int bb = 0; bb < nb; ++bb) {
#pragma unroll
        for (int u = 0; u < kFbBlk; ++u) {
            const int mq = bb * kFbBlk + u;
            v4f a = ra[u], e = re[u];
            if constexpr (RAGGED) {
                a = mq < nq ? a : z;
                e = mq < nq ? e : z;
            }
            acc = __builtin_amdgcn_mfma_f32_16x16x1f32(a.x, e.x, acc, 0, 0, 0);
            acc = __builtin_amdgcn_mfma_f32_16x16x1f32(a.y, e.y, acc, 0, 0, 0);
            acc = __builtin_amdgcn_mfma_f32_16x16x1f32(a.z, e.z, acc, 0, 0, 0);
            acc = __builtin_amdgcn_mfma_f32_16x16x1f32(a.w, e.w, acc, 0, 0, 0);
            __builtin_amdgcn_sched_barrier(0);
            load(u, bb + 1);
            __builtin_amdgcn_sched_barrier(0);
        }
    }
    return acc;
}

// Operand layout of the feedback ("quad layout"): a [k][n] matrix M is
// stored per 16-column block b as a [k/4][16][4] array,
//     Mq[b*16k + (m/4)*64 + 4c + m%4] = M[m][16b + c],
// so the 4 consecutive m of one column are one float4 and the 16 columns x
// 16 m of a feedback group are 1 KiB contiguous.  This kernel writes the
// block-LDL factor L [k][k] in that layout (only the 64x64 tiles holding
// some element with row > column, the part the feedback reads).
__global__ __launch_bounds__(256) void lfac_quads_kernel(const float* __restrict__ L, int k,
                                                         float* __restrict__ Lq) {
    __shared__ float tile[64][65];
    const int c0 = blockIdx.x * 64, r0 = blockIdx.y * 64;   // column / row block of L
    if (r0 + 64 <= c0) return;                               // strictly above the diagonal
    const int tx = threadIdx.x & 63, ty = threadIdx.x >> 6;
    for (int yy = ty; yy < 64; yy += 4) {
        const int r = r0 + yy, c = c0 + tx;
        if (r < k && c < k) tile[yy][tx] = L[(size_t)r * k + c];
    }
    __syncthreads();
    // the tile's 4 column blocks, 64 m each: 1024 contiguous floats per block
    for (int idx = threadIdx.x; idx < 4 * 1024; idx += 256) {
        const int ib = idx >> 10, w = idx & 1023;
        const int mq = w >> 6, c = (w >> 2) & 15, mm = w & 3;
        const int m = r0 + 4 * mq + mm, col = c0 + 16 * ib + c;
        if (m < k && col < k)
            Lq[(size_t)(col >> 4) * 16 * k + (size_t)(m >> 2) * 64 + 4 * c + (m & 3)] =
                tile[4 * mq + mm][16 * ib + c];
    }
}

// ------------------------------------------------- block-128 Hadamard
// out[128b + r][c] = sum_{t=0..127} ht[t][r] * in[128b + t][c] (had_left,
// quantize.py:134-138, with ht = h^T: the multipliers by input row),
// evaluated as torch's CPU sgemm evaluates it: one fp32 fused multiply-add
// chain per output over t ascending, from zero (measured bit for bit against
// an fmaf chain).  Taking h^T makes the 16 multipliers a wave needs at step t
// one contiguous, wave-uniform row segment (scalar loads).  Wave: 16 rows x
// 64 columns; workgroup: 4 waves.
__global__ __launch_bounds__(256) void had_left_kernel(const float* __restrict__ ht,
                                                       const float* __restrict__ in,
                                                       float* __restrict__ out, int cols) {
    const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), ln = threadIdx.x & 63;
    const int c = blockIdx.x * 64 + ln;
    const int r0 = (blockIdx.z * 4 + wv) * 16;
    const bool live = c < cols;
    const float* src = in + (size_t)blockIdx.y * 128 * cols + (live ? c : 0);
    float acc[16];
#pragma unroll
    for (int q = 0; q < 16; ++q) acc[q] = 0.0f;
    for (int t = 0; t < 128; ++t) {
        const float w = src[(size_t)t * cols];
        const float* hr = ht + t * 128 + r0;
#pragma unroll
        for (int q = 0; q < 16; ++q) acc[q] = __builtin_fmaf(hr[q], w, acc[q]);
    }
    if (live) {
        float* dst = out + ((size_t)blockIdx.y * 128 + r0) * cols + c;
#pragma unroll
        for (int q = 0; q < 16; ++q) dst[(size_t)q * cols] = acc[q];
    }
}

// out[r][128b + c] = sum_{t=0..127} h[t][c] * in[r][128b + t] (had_right,
// quantize.py:141-145) without a transpose: each output one fp32 fused
// multiply-add chain over t ascending, from zero -- the products and the
// order of had_left_kernel on the transpose, hence torch's CPU sgemm bits.
// Wave: 8 rows x 64 columns (half of a 128-column block); the 8 inputs of a
// step t are wave-uniform (scalar loads, 8 consecutive t per row at a time)
// and the multipliers h[t][c] one coalesced row segment.  Workgroup: 4
// waves, 32 rows.  (16 rows per wave with 4 steps per scalar load measured
// 1.7x slower: twice the scalar loads per multiply-add.)
constexpr int kHrRows = 8;                 // rows per wave
constexpr int kHrT = 8;                    // steps per scalar load
__global__ __launch_bounds__(256) void had_right_kernel(const float* __restrict__ h,
                                                        const float* __restrict__ in,
                                                        float* __restrict__ out, int rows,
                                                        int cols) {
    const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), ln = threadIdx.x & 63;
    const int b = blockIdx.x >> 1;                          // 128-column block
    const int c = ((blockIdx.x & 1) << 6) + ln;             // column within the block
    const int r0 = (blockIdx.y * 4 + wv) * kHrRows;
    if (r0 >= rows) return;
    const int nr = rows - r0 < kHrRows ? rows - r0 : kHrRows;   // wave-uniform
    const float* src = in + (size_t)r0 * cols + 128 * b;
    float acc[kHrRows];
#pragma unroll
    for (int q = 0; q < kHrRows; ++q) acc[q] = 0.0f;
    if (nr == kHrRows) {
        for (int t0 = 0; t0 < 128; t0 += kHrT) {
#pragma unroll
            for (int t = t0; t < t0 + kHrT; ++t) {
                const float hv = h[t * 128 + c];
#pragma unroll
                for (int q = 0; q < kHrRows; ++q)
                    acc[q] = __builtin_fmaf(hv, src[(size_t)q * cols + t], acc[q]);
            }
        }
    } else {
        for (int t = 0; t < 128; ++t) {
            const float hv = h[t * 128 + c];
            for (int q = 0; q < nr; ++q)
                acc[q] = __builtin_fmaf(hv, src[(size_t)q * cols + t], acc[q]);
        }
    }
    float* dst = out + (size_t)r0 * cols + 128 * b + c;
#pragma unroll
    for (int q = 0; q < kHrRows; ++q)
        if (q < nr) dst[(size_t)q * cols] = acc[q];
}

template <int K>
__global__ __launch_bounds__(kFwdThreads) void ldlq_chain_kernel(
    const float* __restrict__ W, const float* __restrict__ Lq, int k, int n, int jc0, int tnl,
    const float* __restrict__ lut, int pivot, int n1, uint8_t* __restrict__ bp,
    float* __restrict__ xbuf, float* __restrict__ hatW, float* __restrict__ Eq,
    int32_t* __restrict__ states, int16_t* __restrict__ trellis, uint32_t* __restrict__ flags,
    int32_t* __restrict__ counter, uint32_t epoch, int spin_limit, uint32_t* __restrict__ err,
    int xdump, int pbuf) {
    using G = Geom<K>;
    __shared__ FwdSmem<K, 1> sm;
    // traceback staging: the forward's b buffers where they hold 64 KiB; the
    // feedback's per-buffer partials use the same 64 KiB before the passes
    constexpr bool kOwnStage = 2 * sizeof(float) * G::SPL < (size_t)kTbStage;
    __shared__ __attribute__((aligned(16))) uint4 tbstage[kOwnStage ? kTbStage / 16 : 1];
    uint4* const stage = kOwnStage ? tbstage : (uint4*)&sm.bbuf[0][0][0];
    __shared__ int32_t st[kSteps];
    __shared__ int32_t task, cur, ok;
    const int tid = threadIdx.x;
    // this launch sweeps the column tiles jc0 .. jc0+tnl-1 of the [k][n]
    // matrices (its trellis holds just those: [tk][tnl][16K])
    const int tk = k / 16, tn = n / 16, ntask = tk * tnl;
    // this workgroup's backpointer slot and target row (or the dump row)
    uint8_t* const bpw = bp + (size_t)blockIdx.x * ((size_t)kSlots * G::BPSTEP);
    // Thread 0 publishes a finished tile and fetches the next task in ONE
    // block right before the barrier that opens the loop body.  Two separate
    // thread-0 blocks on either side of the back edge get merged by the
    // compiler into a per-lane exit of the barrier loop: the other lanes of
    // wave 0 then re-enter the body without thread 0 (stale task, no flag)
    // and the launch never ends.  The loop-control values are read through
    // readfirstlane so that the loop's exits are wave-uniform branches.
    if (tid == 0) task = atomicAdd(counter, 1);
    // A workgroup runs at most ntask tasks; the bound also ends the loop
    // (err |= 4) should the task sequence ever fail to advance.
    for (int done = 0;; ++done) {
        __syncthreads();
        const int t = __builtin_amdgcn_readfirstlane(task);
        if (t >= ntask) break;
        if (done >= ntask) {
            if (tid == 0) atomicOr(err, 4u);
            break;
        }
        const int i = tk - 1 - t / tnl, jl = t - (t / tnl) * tnl, j = jc0 + jl;
        // targets row: the workgroup's own, or the tile's (row-block order)
        float* const xs = xbuf + (xdump ? (size_t)i * tn + j : (size_t)blockIdx.x) * kSteps;
        // wait for tile (i+1, j), this launch's task t - tnl
        if (tid == 0) {
            int good = 1;
            if (Lq != nullptr && i + 1 < tk) {
                const uint32_t* f = flags + (size_t)(i + 1) * tn + j;
                // relaxed polls (no cache invalidation per poll), one acquire
                // fence once the flag is seen
                for (int it = 0;; ++it) {
                    if (__hip_atomic_load(f, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == epoch) {
                        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
                        break;
                    }
                    if (it >= spin_limit) {
                        atomicOr(err, 2u);
                        good = 0;
                        break;
                    }
                    // another wait already expired: the chain will not
                    // complete, so end this one too instead of timing out
                    if ((it & 63) == 63 &&
                        (__hip_atomic_load(err, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) & 2u)) {
                        good = 0;
                        break;
                    }
                    __builtin_amdgcn_s_sleep(8);
                }
            }
            ok = good;
        }
        __syncthreads();
        if (!__builtin_amdgcn_readfirstlane(ok)) break;
        // targets in the reference's order (see above): rounds of 64 buffers,
        // buffer b = b0 + 4 wv + (lane >> 4) in block (lane >> 4) of the
        // wave's accumulator; lane (blk, rc) feeds row rc of L and column rc
        // of E of that buffer, 4 consecutive m per 16-byte load (quad
        // layout), kFbPrefetch m-quads ahead; b == qi is the part of block
        // i's own buffer below it.
        {
            float* const P = (float*)stage;               // [64][256] partials
            const int wv = tid >> 6, ln = tid & 63, blk = ln >> 4, rc = ln & 15;
            const int qi = (tk - 1 - i) / pbuf, cur = tk - pbuf * qi, nbuf = qi + 1;
            const bool has_gin = (i + 1 < cur);
            const bool fb = (Lq != nullptr);
            float prod = 0.0f, gin = 0.0f;
            for (int b0 = 0; fb && b0 < nbuf; b0 += 64) {
                const int bw = b0 + 4 * wv, b = bw + blk;
                int mlo = 0, nq = 0;
                if (b < qi) {
                    mlo = 16 * (tk - pbuf * (b + 1));
                    nq = 4 * pbuf;
                } else if (b == qi) {
                    mlo = 16 * (i + 1);
                    nq = 4 * (cur - i - 1);
                }
                // wave-uniform step count: full buffers if the wave holds
                // one, else block i's own buffer; shorter lanes feed zeros,
                // whose products leave the accumulator unchanged
                const int nqw = __builtin_amdgcn_readfirstlane(
                    bw < qi ? 4 * pbuf : (bw == qi ? 4 * (cur - i - 1) : 0));
                v16f acc;
#pragma unroll
                for (int v = 0; v < 16; ++v) acc[v] = 0.0f;
                if (nqw > 0) {
                    // L's column block i and E's column block j (wave-uniform
                    // bases) at the lane's offset: the first m-quad of its
                    // buffer, column rc
                    const gbyte_t* const lb = uniform_gptr((uint8_t*)(Lq + (size_t)i * 16 * k));
                    const gbyte_t* const eb = uniform_gptr((uint8_t*)(Eq + (size_t)j * 16 * k));
                    const uint32_t off0 = 4u * ((uint32_t)(mlo >> 2) * 64u + 4u * (uint32_t)rc);
                    // every lane of the wave runs nqw m-quads unless the wave
                    // holds block i's own buffer or a buffer past it
                    if (bw + 3 < qi)
                        acc = fb_chain<false>(lb, eb, off0, nq, nqw);
                    else
                        acc = fb_chain<true>(lb, eb, off0, nq, nqw);
                }
                // accumulator register v = 4 blk' + t of lane (q, c): block
                // blk', row 4q + t, column c
#pragma unroll
                for (int v = 0; v < 16; ++v)
                    P[(4 * wv + (v >> 2)) * 256 + (4 * blk + (v & 3)) * 16 + rc] = acc[v];
                __syncthreads();
                if (tid < 256) {
                    // the round's partials in buffer order, read eight at a
                    // time so that one LDS latency covers eight adds
                    const int nr = (nbuf - b0) < 64 ? (nbuf - b0) : 64;
                    int sl = 0;
                    for (; sl + 8 <= nr; sl += 8) {
                        float v[8];
#pragma unroll
                        for (int u = 0; u < 8; ++u) v[u] = P[(sl + u) * 256 + tid];
#pragma unroll
                        for (int u = 0; u < 8; ++u) {
                            if (b0 + sl + u < qi) prod = prod + v[u];
                            else gin = v[u];
                        }
                    }
                    for (; sl < nr; ++sl) {
                        const float v = P[sl * 256 + tid];
                        if (b0 + sl < qi) prod = prod + v;
                        else gin = v;
                    }
                }
                __syncthreads();
            }
            if (tid < 256) {
                const int pe = tid;                       // tile element handled here
                const float w = W[(size_t)(16 * i + (pe >> 4)) * n + 16 * j + (pe & 15)];
                // no factor: the targets are W itself (quantize.py:680)
                P[pe] = !fb ? w : (has_gin ? (w + gin) + prod : w + prod);
            }
            __syncthreads();
            // sequence order x_t = tile[perm[t]] (quantize.py:684-686); thread
            // q writes target q, fwd_run reads it back in thread q
            if (tid < 256) xs[tid] = P[tc_perm(tid)];
        }
        __syncthreads();
        // pass 1: free run of the sequence rolled by pivot, traced back to
        // pivot; pass 2: pinned to ov = s_pivot >> K, full traceback into st
        // (one call site of the forward body for both passes)
#pragma unroll 1
        for (int pass = 0; pass < 2; ++pass) {
            const int nst = pass ? kSteps : n1, lo = pass ? 0 : pivot;
            if (tid == 0) sm.ovs[0] = pass ? (cur >> K) : -1;
            int tidv = tid;
            const float* lutv = lut;
            asm volatile("" : "+v"(tidv));
            asm volatile("" : "+s"(lutv));
            fwd_run<K, 1>(sm, xs, kSteps, kSteps, 0, 1, lutv, pass ? 0 : pivot, nst, lo,
                          pass != 0, bpw, &cur, err, tidv);
            // the backpointers are read back by this workgroup only: the
            // barrier's workgroup-scope ordering suffices
            __syncthreads();
            if (pass && tid == 0) st[kSteps - 1] = cur & 0xFFFF;
            __syncthreads();
            tb_chase_pf<K>(bpw, nst, lo, stage, pass ? st : nullptr, cur);
        }
        // outputs of the tile
        const size_t tile = (size_t)i * tn + j;
        if (tid < kSteps) {
            const int s = st[tid];
            const int pe = tc_perm(tid);
            const size_t g = (size_t)(16 * i + (pe >> 4)) * n + 16 * j + (pe & 15);
            const float w = lut[s];
            hatW[g] = w;
            const int m = 16 * i + (pe >> 4);                 // E in the quad layout
            // E is all that other workgroups read of the tile (their
            // feedback, on any XCD): an agent-scope store (sc1) writes it
            // through this XCD's L2, visible agent-wide once it completes
            __hip_atomic_store(&Eq[(size_t)j * 16 * k + (size_t)(m >> 2) * 64 + 4 * (pe & 15) +
                                   (m & 3)],
                               W[g] - w, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            if (states) states[tile * kSteps + tid] = s;
        } else if (tid < kSteps + 8 * K) {
            const int wd = tid - kSteps;
            store_word(trellis + ((size_t)i * tnl + jl) * 16 * K + 2 * wd, pack_word<K>(st, wd));
        }
        // Every wave's stores complete before the barrier (explicitly: the
        // barrier's workgroup-scope release does not wait for them), so E's
        // write-through stores are visible agent-wide before thread 0 stores
        // the flag, which therefore cannot overtake them; the waiter's
        // acquire fence then invalidates its L2 before it reads E.  A release
        // store here would add an L2 write-back of every dirty line of the
        // XCD (buffer_wbl2: the other workgroups' backpointer rows among
        // them), which no waiter needs -- the rest of the tile (W_hat,
        // states, trellis) is read only after the launch.  c5 K=4: 950
        // against 958 ms per sweep, results identical.
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        __syncthreads();
        if (tid == 0) {
            __hip_atomic_store(flags + tile, epoch, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            task = atomicAdd(counter, 1);
        }
    }
}

template <template <int> class F, typename... A>
hipError_t dispatch_k(int K, A... a) {
    switch (K) {
        case 2: return F<2>::run(a...);
        case 3: return F<3>::run(a...);
        case 4: return F<4>::run(a...);
        case 5: return F<5>::run(a...);
        case 6: return F<6>::run(a...);
        case 7: return F<7>::run(a...);
        default: return hipErrorInvalidValue;
    }
}

// Largest group size whose LDS footprint (2 x SP floats + 1 KiB per
// sequence) fits one CU's 160 KiB.
template <int K>
constexpr int max_group() {
    constexpr size_t per = 2 * sizeof(float) * Geom<K>::SPL + 1024 + 16;
    return (8 * per + 512 <= 160 * 1024) ? 8 : (4 * per + 512 <= 160 * 1024) ? 4
         : (2 * per + 512 <= 160 * 1024) ? 2 : 1;
}

template <int K>
struct FwdL {
    static hipError_t run(const float* X, int xstride, int xlen, int nseq,
                          const float* lut, int roll, int nsteps, int store_lo,
                          const int32_t* ov_in, void* bp, int32_t* send, uint32_t* err,
                          int group, hipStream_t s) {
        const int T = group <= 1 ? 1 : group <= 2 ? 2 : group <= 4 ? 4 : 8;
        if (T > max_group<K>()) return hipErrorInvalidValue;
        const int nwg = (nseq + T - 1) / T;
        if (T == 1)
            hipLaunchKernelGGL((fwd_kernel<K, 1>), dim3(nwg), dim3(kFwdThreads), 0, s, X,
                               xstride, xlen, nseq, lut, roll, nsteps, store_lo, ov_in,
                               (uint8_t*)bp, send, err);
        else if constexpr (max_group<K>() >= 2) {
            if (T == 2)
                hipLaunchKernelGGL((fwd_kernel<K, 2>), dim3(nwg), dim3(kFwdThreads), 0, s,
                                   X, xstride, xlen, nseq, lut, roll, nsteps, store_lo,
                                   ov_in,
                                   (uint8_t*)bp, send, err);
            else if constexpr (max_group<K>() >= 4) {
                if (T == 4)
                    hipLaunchKernelGGL((fwd_kernel<K, 4>), dim3(nwg), dim3(kFwdThreads), 0, s,
                                       X, xstride, xlen, nseq, lut, roll, nsteps, store_lo,
                                       ov_in, (uint8_t*)bp, send, err);
                else if constexpr (max_group<K>() >= 8)
                    hipLaunchKernelGGL((fwd_kernel<K, 8>), dim3(nwg), dim3(kFwdThreads), 0, s,
                                       X, xstride, xlen, nseq, lut, roll, nsteps, store_lo,
                                       ov_in, (uint8_t*)bp, send, err);
            }
        }
        return hipGetLastError();
    }
};

#ifndef XTQ_FWD_K3_TU
template <>
struct FwdL<3> {
    static hipError_t run(const float* X, int xstride, int xlen, int nseq,
                          const float* lut, int roll, int nsteps, int store_lo,
                          const int32_t* ov_in, void* bp, int32_t* send, uint32_t* err,
                          int group, hipStream_t s) {
        return launch_forward_k3(X, xstride, xlen, nseq, lut, roll, nsteps, store_lo, ov_in,
                                 bp, send, err, group, s);
    }
};
#endif

template <int K>
struct GroupSel {
    static hipError_t run(int nseq, int ncu, int* out) {
        // One workgroup per CU is resident; prefer the largest group that
        // still gives every CU at least two workgroups.
        int T = max_group<K>();
        while (T > 1 && (nseq + T - 1) / T < 2 * ncu) T >>= 1;
        *out = T;
        return hipSuccess;
    }
};

template <int K>
struct FwdDeferL {
    static hipError_t run(const float* X, int xstride, int xlen, int nseq,
                          const float* lut, int roll, int nsteps, int store_lo,
                          const int32_t* ov_in, void* bm, int32_t* send, uint32_t* err,
                          int group, hipStream_t s) {
        if constexpr (K < 4) {
            return hipErrorInvalidValue;
        } else {
            const int T = group <= 1 ? 1 : group <= 2 ? 2 : group <= 4 ? 4 : 8;
            if (T > max_group<K>()) return hipErrorInvalidValue;
            const int nwg = (nseq + T - 1) / T;
            float* b = (float*)bm;
            if (T == 1)
                hipLaunchKernelGGL((fwd_defer_kernel<K, 1>), dim3(nwg), dim3(kFwdThreads), 0, s,
                                   X, xstride, xlen, nseq, lut, roll, nsteps, store_lo, ov_in,
                                   b, send, err);
            else if (T == 2)
                hipLaunchKernelGGL((fwd_defer_kernel<K, 2>), dim3(nwg), dim3(kFwdThreads), 0, s,
                                   X, xstride, xlen, nseq, lut, roll, nsteps, store_lo, ov_in,
                                   b, send, err);
            else if constexpr (max_group<K>() >= 4) {
                if (T == 4)
                    hipLaunchKernelGGL((fwd_defer_kernel<K, 4>), dim3(nwg), dim3(kFwdThreads),
                                       0, s, X, xstride, xlen, nseq, lut, roll, nsteps,
                                       store_lo, ov_in, b, send, err);
                else if constexpr (max_group<K>() >= 8)
                    hipLaunchKernelGGL((fwd_defer_kernel<K, 8>), dim3(nwg), dim3(kFwdThreads),
                                       0, s, X, xstride, xlen, nseq, lut, roll, nsteps,
                                       store_lo, ov_in, b, send, err);
            }
            return hipGetLastError();
        }
    }
};

template <int K>
struct TbDeferL {
    static hipError_t run(const void* bm, const float* X, int xstride, int xlen, int roll,
                          const float* lut, int nseq, const int32_t* send,
                          const int32_t* ov_in, int nsteps, int stop, int shift, int32_t* sout,
                          int32_t* states, int16_t* trellis, hipStream_t s) {
        if constexpr (K < 4) {
            return hipErrorInvalidValue;
        } else {
            hipLaunchKernelGGL(tb_defer_kernel<K>, dim3((nseq + kTbLaneSeqs - 1) / kTbLaneSeqs),
                               dim3(kTbLaneSeqs), 0, s, (const float*)bm, X, xstride, xlen, roll,
                               lut, nseq, send, ov_in, nsteps, stop, shift, sout, states,
                               trellis);
            return hipGetLastError();
        }
    }
};

template <int K>
struct DeferBytes {
    static hipError_t run(size_t* out) {
        if constexpr (K < 4) {
            *out = 0;
            return hipErrorInvalidValue;
        } else {
            *out = defer_tile_bytes<K>();
            return hipSuccess;
        }
    }
};

template <int K>
struct FusedL {
    static hipError_t run(const float* X, int nseq, const float* lut, int pivot, int n1,
                          void* bp, int32_t* send, int32_t* ovbuf, uint32_t* flags,
                          int32_t* counter, uint32_t epoch, int spin_limit, uint32_t* err,
                          hipStream_t s) {
        hipLaunchKernelGGL(reset_counter_kernel, dim3(1), dim3(1), 0, s, counter);
        hipLaunchKernelGGL(tailbite_fused_kernel<K>, dim3(2 * nseq), dim3(kFwdThreads), 0, s,
                           X, nseq, lut, pivot, n1, (uint8_t*)bp, send, ovbuf, flags,
                           counter, epoch, spin_limit, err);
        return hipGetLastError();
    }
};

template <int K>
struct ChainL {
    static hipError_t run(const float* W, const float* Lq, int k, int n, int jc0, int tnl,
                          const float* lut, int pivot, int n1, void* bp, int nwg,
                          float* xbuf, int xdump, float* hatW, float* Eq, int32_t* states,
                          int16_t* trellis, uint32_t* flags, int32_t* counter, uint32_t epoch,
                          int spin_limit, uint32_t* err, int pbuf, hipStream_t s) {
        hipLaunchKernelGGL(reset_counter_kernel, dim3(1), dim3(1), 0, s, counter);
        hipLaunchKernelGGL(ldlq_chain_kernel<K>, dim3(nwg), dim3(kFwdThreads), 0, s, W, Lq, k,
                           n, jc0, tnl, lut, pivot, n1, (uint8_t*)bp, xbuf, hatW, Eq, states,
                           trellis, flags, counter, epoch, spin_limit, err, xdump, pbuf);
        return hipGetLastError();
    }
};

template <int K>
struct TbL {
    static hipError_t run(const void* bp, int nseq, const int32_t* send, int nsteps,
                          int stop, int shift, int32_t* sout, int32_t* states,
                          int16_t* trellis, bool lanes, hipStream_t s) {
        if (lanes)
            hipLaunchKernelGGL(tb_lane_kernel<K>,
                               dim3((nseq + kTbLaneSeqs - 1) / kTbLaneSeqs), dim3(kTbLaneSeqs),
                               0, s, (const uint8_t*)bp, nseq, send, nsteps, stop, shift, sout,
                               states, trellis);
        else
            hipLaunchKernelGGL(tb_kernel<K>, dim3(nseq), dim3(kTbThreads), 0, s,
                               (const uint8_t*)bp, send, nsteps, stop, shift, sout, states,
                               trellis);
        return hipGetLastError();
    }
};

template <int K>
struct DecL {
    static hipError_t run(const int16_t* tr, int tk, int tn, const float* lut,
                          float* of, uint16_t* oh, hipStream_t s) {
        hipLaunchKernelGGL(decode_kernel<K>, dim3(tk * tn), dim3(256), 0, s, tr, tn, lut,
                           of, oh);
        return hipGetLastError();
    }
};

template <int K>
struct PackL {
    static hipError_t run(const int32_t* st, int nt, int16_t* tr, hipStream_t s) {
        hipLaunchKernelGGL(pack_kernel<K>, dim3(nt), dim3(64), 0, s, st, tr);
        return hipGetLastError();
    }
};

template <int K>
struct UnpackL {
    static hipError_t run(const int16_t* tr, int nt, int32_t* st, hipStream_t s) {
        hipLaunchKernelGGL(unpack_kernel<K>, dim3(nt), dim3(256), 0, s, tr, st);
        return hipGetLastError();
    }
};

template <int K>
struct StepBytes {
    static hipError_t run(size_t* out) {
        *out = (size_t)Geom<K>::BPSTEP;
        return hipSuccess;
    }
};

}  // namespace

#ifdef XTQ_FWD_K3_TU
hipError_t launch_forward_k3(const float* X, int xstride, int xlen, int nseq,
                             const float* lut, int roll, int nsteps, int store_lo,
                             const int32_t* ov_in, void* bp, int32_t* send, uint32_t* err,
                             int group, hipStream_t stream) {
    return FwdL<3>::run(X, xstride, xlen, nseq, lut, roll, nsteps, store_lo, ov_in, bp, send,
                        err, group, stream);
}
#else
size_t bp_step_bytes(int K) {
    size_t b = 0;
    if (dispatch_k<StepBytes>(K, &b) != hipSuccess) return 0;
    return b;
}

int forward_group(int K, int nseq, int ncu) {
    int T = 1;
    if (dispatch_k<GroupSel>(K, nseq, ncu, &T) != hipSuccess) return 1;
    return T;
}

hipError_t launch_forward(int K, const float* X, int xstride, int xlen, int nseq,
                          const float* lut, int roll, int nsteps, int store_lo,
                          const int32_t* ov_in, void* bp, int32_t* send, uint32_t* err,
                          int group, hipStream_t stream) {
    if (nseq <= 0) return hipSuccess;
    if (xlen < 1 || xlen > kSteps || nsteps < 1 || nsteps > kSteps || roll < 0 ||
        roll >= xlen || (roll != 0 && xlen != kSteps) || (roll == 0 && nsteps > xlen))
        return hipErrorInvalidValue;
    return dispatch_k<FwdL>(K, X, xstride, xlen, nseq, lut, roll, nsteps, store_lo, ov_in,
                            bp, send, err, group, stream);
}

hipError_t launch_tailbite_fused(int K, const float* X, int nseq, const float* lut,
                                 int pivot, int n1, void* bp, int32_t* send, int32_t* ovbuf,
                                 uint32_t* flags, int32_t* counter, uint32_t epoch,
                                 int spin_limit, uint32_t* err, hipStream_t stream) {
    if (nseq <= 0) return hipSuccess;
    if (pivot < 0 || pivot >= kSteps || n1 <= pivot || n1 > kSteps || spin_limit < 1)
        return hipErrorInvalidValue;
    return dispatch_k<FusedL>(K, X, nseq, lut, pivot, n1, bp, send, ovbuf, flags, counter,
                              epoch, spin_limit, err, stream);
}

hipError_t launch_had_left(const float* ht, const float* in, float* out, int rows, int cols,
                           hipStream_t stream) {
    if (rows <= 0 || cols <= 0) return hipSuccess;
    if (rows % 128 || rows / 128 > 65535) return hipErrorInvalidValue;
    hipLaunchKernelGGL(had_left_kernel, dim3((cols + 63) / 64, rows / 128, 2), dim3(256), 0,
                       stream, ht, in, out, cols);
    return hipGetLastError();
}

hipError_t launch_had_right(const float* h, const float* in, float* out, int rows, int cols,
                            hipStream_t stream) {
    if (rows <= 0 || cols <= 0) return hipSuccess;
    if (cols % 128) return hipErrorInvalidValue;
    const int ry = (rows + 4 * kHrRows - 1) / (4 * kHrRows);
    if (ry > 65535) return hipErrorInvalidValue;
    hipLaunchKernelGGL(had_right_kernel, dim3(cols / 64, ry), dim3(256), 0, stream, h, in, out,
                       rows, cols);
    return hipGetLastError();
}

hipError_t launch_lfac_quads(const float* L, int k, float* Lq, hipStream_t stream) {
    if (k <= 0) return hipSuccess;
    if (k % 16 || L == nullptr || Lq == nullptr) return hipErrorInvalidValue;
    const int nb = (k + 63) / 64;
    hipLaunchKernelGGL(lfac_quads_kernel, dim3(nb, nb), dim3(256), 0, stream, L, k, Lq);
    return hipGetLastError();
}

hipError_t launch_ldlq_chain(int K, const float* W, const float* Lq, int k, int n, int jc0,
                            int tnl, const float* lut, int pivot, int n1, void* bp,
                            int nwg, float* xbuf, int xdump, float* hatW, float* Eq,
                            int32_t* states, int16_t* trellis, uint32_t* flags,
                            int32_t* counter, uint32_t epoch, int spin_limit, uint32_t* err,
                            int buf_cols, hipStream_t stream) {
    if (k <= 0 || n <= 0 || tnl <= 0) return hipSuccess;
    if (k % 16 || n % 16 || jc0 < 0 || jc0 + tnl > n / 16 || pivot < 0 || pivot >= kSteps ||
        n1 <= pivot || n1 > kSteps || nwg < 1 || spin_limit < 1 || buf_cols < 16 ||
        buf_cols % 16)
        return hipErrorInvalidValue;
    return dispatch_k<ChainL>(K, W, Lq, k, n, jc0, tnl, lut, pivot, n1, bp, nwg, xbuf, xdump,
                              hatW, Eq, states, trellis, flags, counter, epoch, spin_limit, err,
                              buf_cols / 16, stream);
}

hipError_t launch_traceback(int K, const void* bp, int nseq, const int32_t* send,
                            int nsteps, int stop, int shift, int32_t* sout, int32_t* states,
                            int16_t* trellis, bool lanes, hipStream_t stream) {
    if (nseq <= 0) return hipSuccess;
    if (nsteps < 1 || nsteps > kSteps || stop < 0 || stop >= nsteps)
        return hipErrorInvalidValue;
    return dispatch_k<TbL>(K, bp, nseq, send, nsteps, stop, shift, sout, states, trellis,
                           lanes, stream);
}

hipError_t launch_decode(int K, const int16_t* trellis, int tk, int tn, const float* lut,
                         float* out_f32, uint16_t* out_f16, hipStream_t stream) {
    if (tk <= 0 || tn <= 0) return hipSuccess;
    return dispatch_k<DecL>(K, trellis, tk, tn, lut, out_f32, out_f16, stream);
}

hipError_t launch_pack(int K, const int32_t* states, int nt, int16_t* trellis,
                       hipStream_t stream) {
    if (nt <= 0) return hipSuccess;
    return dispatch_k<PackL>(K, states, nt, trellis, stream);
}

hipError_t launch_unpack(int K, const int16_t* trellis, int nt, int32_t* states,
                         hipStream_t stream) {
    if (nt <= 0) return hipSuccess;
    return dispatch_k<UnpackL>(K, trellis, nt, states, stream);
}

size_t defer_tile_bytes(int K) {
    size_t b = 0;
    if (dispatch_k<DeferBytes>(K, &b) != hipSuccess) return 0;
    return b;
}

hipError_t launch_forward_defer(int K, const float* X, int xstride, int xlen, int nseq,
                                const float* lut, int roll, int nsteps, int store_lo,
                                const int32_t* ov_in, void* bm, int32_t* send, uint32_t* err,
                                int group, hipStream_t stream) {
    if (nseq <= 0) return hipSuccess;
    if (xlen < 1 || xlen > kSteps || nsteps < 1 || nsteps > kSteps || roll < 0 ||
        roll >= xlen || (roll != 0 && xlen != kSteps) || (roll == 0 && nsteps > xlen) ||
        store_lo < 0)
        return hipErrorInvalidValue;
    return dispatch_k<FwdDeferL>(K, X, xstride, xlen, nseq, lut, roll, nsteps, store_lo,
                                 ov_in, bm, send, err, group, stream);
}

hipError_t launch_traceback_defer(int K, const void* bm, const float* X, int xstride, int xlen,
                                  int roll, const float* lut, int nseq,
                                  const int32_t* send, const int32_t* ov_in, int nsteps,
                                  int stop, int shift, int32_t* sout, int32_t* states,
                                  int16_t* trellis, hipStream_t stream) {
    if (nseq <= 0) return hipSuccess;
    if (nsteps < 1 || nsteps > kSteps || stop < 0 || stop >= nsteps || roll < 0 ||
        roll >= xlen || xlen < 1 || xlen > kSteps)
        return hipErrorInvalidValue;
    return dispatch_k<TbDeferL>(K, bm, X, xstride, xlen, roll, lut, nseq, send, ov_in,
                                nsteps, stop, shift, sout, states, trellis, stream);
}

hipError_t launch_fill_u32(uint32_t* p, uint32_t n, uint32_t v, hipStream_t stream) {
    if (n == 0) return hipSuccess;
    if (p == nullptr) return hipErrorInvalidValue;
    hipLaunchKernelGGL(fill_u32_kernel, dim3((n + 255u) / 256u), dim3(256), 0, stream, p, n, v);
    return hipGetLastError();
}

#endif  // XTQ_FWD_K3_TU

}  // namespace xtq
