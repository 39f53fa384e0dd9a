// exl3_vit_capi.hip -- C-ABI of libexl3vit.so (declared in include/exl3_vit.h).
//
// Host-side orchestration of the gfx950 trellis kernels: argument checks with
// the reference's status codes (quantize/viterbi_esimd.cpp:924-1005), the
// codebook tables, per-device grow-only scratch, chunking of large batches and
// the two-pass tail-biting schedule
//     forward(pass 1) -> traceback(pass 1: ov) -> forward(pass 2) -> traceback
// (quantize.py:323-354).
#include <hip/hip_runtime.h>

#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <mutex>
#include <vector>

#include "../../include/exl3_vit.h"
#include "viterbi_kernels.h"

namespace {

enum Code { kMul1 = 0, k3Inst = 1, kMcg = 2, k1Mad = 3, kNumCodes = 4 };

// --------------------------------------------------------- codebook tables
// fp16 bits -> double (exact).
double half_to_double(uint16_t h) {
    const int sgn = (h >> 15) & 1, e = (h >> 10) & 31, m = h & 1023;
    double v;
    if (e == 0) v = ldexp((double)m, -24);
    else if (e == 31) v = m ? NAN : INFINITY;
    else v = ldexp((double)(1024 + m), e - 25);
    return sgn ? -v : v;
}

// double -> fp16 bits, round to nearest, ties to even (finite inputs).
uint16_t double_to_half(double v) {
    uint16_t sgn = (v < 0 || (v == 0 && signbit(v))) ? 0x8000 : 0;
    double a = fabs(v);
    if (a == 0) return sgn;
    int e;
    frexp(a, &e);            // a = m * 2^e, m in [0.5, 1)
    int ue = e - 1;          // a in [2^ue, 2^(ue+1))
    if (ue < -14) {          // subnormal: quantum 2^-24
        double q = nearbyint(ldexp(a, 24));
        return sgn | (uint16_t)q;   // q == 1024 encodes the smallest normal
    }
    double q = nearbyint(ldexp(a, 10 - ue));  // in [1024, 2048]
    if (q >= 2048) { q = 1024; ++ue; }
    if (ue + 15 >= 31) return sgn | 0x7C00;
    return sgn | (uint16_t)(((ue + 15) << 10) | ((int)q - 1024));
}

// Codebook tables as the fp32 values the reference's get_lut returns,
// restating quantize.py:56-87 (_local_code_lut): the EXL3 codes round to
// fp16 (held exactly in fp32); qtip_1mad divides in double and rounds once
// to fp32, as numpy's astype(float32) does.
void make_lut(Code code, float* out) {
    for (uint32_t s = 0; s < 65536u; ++s) {
        if (code == kMul1) {
            const uint32_t x = s * 0x83DCD12Du;
            const uint32_t bs = (x & 0xFF) + ((x >> 8) & 0xFF) + ((x >> 16) & 0xFF) + (x >> 24);
            const double h = 1024.0 + bs;
            out[s] = (float)half_to_double(
                double_to_half(h * half_to_double(0x1EEE) + half_to_double(0xC931)));
        } else if (code == k1Mad) {
            const uint32_t x = s * 34038481u + 76625530u;
            const uint32_t bs = (x & 0xFF) + ((x >> 8) & 0xFF) + ((x >> 16) & 0xFF) + (x >> 24);
            out[s] = (float)(((double)bs - 510.0) / 147.800537109375);
        } else {
            uint32_t x = (code == k3Inst) ? s * 89226354u + 64248484u : s * 0xCBAC1FEDu;
            x = (x & 0x8FFF8FFFu) ^ 0x3B603B60u;
            const double lo = half_to_double((uint16_t)(x & 0xFFFF));
            const double hi = half_to_double((uint16_t)(x >> 16));
            out[s] = (float)half_to_double(double_to_half(lo + hi));
        }
    }
}

int parse_code(const char* code, Code* out) {
    if (!code) return 12;
    if (!strcmp(code, "mul1") || !strcmp(code, "exl3_mul1")) { *out = kMul1; return 0; }
    if (!strcmp(code, "3inst") || !strcmp(code, "exl3_3inst")) { *out = k3Inst; return 0; }
    if (!strcmp(code, "mcg") || !strcmp(code, "exl3_mcg")) { *out = kMcg; return 0; }
    if (!strcmp(code, "1mad") || !strcmp(code, "qtip_1mad")) { *out = k1Mad; return 0; }
    return 8;
}

// ------------------------------------------------------------ device state
// Column groups of different K in one chain call (each its own launch).
constexpr int kMaxChainGroups = 8;

struct DevCtx {
    bool ready = false;
    int ncu = 0;
    float* lut[kNumCodes] = {};               // fp32 codebook tables
    uint32_t* err = nullptr;
    void* bp = nullptr;
    size_t bp_cap = 0;
    int32_t* send = nullptr;
    int32_t* ov = nullptr;
    uint32_t* flags = nullptr;   // fused tail-bite: pass-1 -> pass-2 ready flags
    size_t seq_cap = 0;
    int32_t* counter = nullptr;  // fused tail-bite: task counter
    uint32_t epoch = 0;          // fused tail-bite: value the current launch publishes
    float* E = nullptr;          // column chains: W - What of finished tiles (quad layout)
    size_t e_cap = 0;            // floats
    float* Lt = nullptr;         // column chains: block-LDL factor (quad layout)
    size_t lt_cap = 0;           // floats
    uint32_t* cflags = nullptr;  // column chains: tile-ready flags
    size_t cflags_cap = 0;
    float* xbuf = nullptr;       // column chains: each workgroup's target row
    size_t xbuf_cap = 0;         // floats
    int32_t* ccount = nullptr;   // column chains: one task counter per concurrent launch
    hipStream_t side[kMaxChainGroups - 1] = {};   // launches of groups 1.. of a call
    hipEvent_t fork = nullptr, join[kMaxChainGroups - 1] = {};
    float* hx = nullptr;       // staging for the host-pointer entries
    int32_t* hs = nullptr;
    size_t host_cap = 0;
    // pinned host staging of the host-pointer entries' states (grow-only,
    // host memory, not counted in `owned`)
    int32_t* hpin = nullptr;
    size_t hpin_cap = 0;       // elements
    size_t owned = 0;          // device bytes held
    // Recorded on the stream of the last call that used the scratch above;
    // the next call waits for it on its own stream, and growing the scratch
    // waits for it on the host before freeing.
    hipEvent_t last = nullptr;
    // This device's copy of the no-allocation entry's scratch array (its
    // address from hipGetSymbolAddress at set-up).
    uint8_t* noalloc = nullptr;
};

std::mutex g_mu;
std::vector<DevCtx> g_dev;

// Device scratch of xtq_vit_tailbite_dev_noalloc: a file-scope array in the
// code object, one copy per device, held until the process ends.  256 MiB
// holds one call of up to 257 sequences at K=2 or 3, 513 at K=4 or 5, 1,027
// at K=6 and 2,055 at K=7 (kNoAllocHeader bytes of status words, then the
// per-sequence words and backpointer slots, see noalloc_capacity).  Host
// code uses its per-device address (DevCtx::noalloc), never the name.
constexpr size_t kNoAllocBytes = (size_t)256 << 20;
constexpr size_t kNoAllocHeader = 256;
static __device__ __align__(256) uint8_t scratch[kNoAllocBytes];

// Opt-in kernel timing: each forward/traceback launch is bracketed with HIP
// events on its stream; elapsed times are folded in after the stream syncs.
struct ProfPair { hipEvent_t a, b; int kind; double seq_steps; };
bool g_prof = false;
std::vector<ProfPair> g_prof_pending;
double g_prof_ms[2] = {0.0, 0.0};
long long g_prof_launches[2] = {0, 0};
double g_prof_seq_steps = 0.0;

// Records the start event of a timed launch (kind 0 forward, 1 traceback).
int prof_begin(hipStream_t s, int kind, double seq_steps) {
    if (!g_prof) return -1;
    ProfPair p{nullptr, nullptr, kind, seq_steps};
    if (hipEventCreate(&p.a) != hipSuccess || hipEventCreate(&p.b) != hipSuccess) return -1;
    (void)hipEventRecord(p.a, s);
    g_prof_pending.push_back(p);
    return (int)g_prof_pending.size() - 1;
}

void prof_end(int idx, hipStream_t s) {
    if (idx >= 0) (void)hipEventRecord(g_prof_pending[idx].b, s);
}

// Called after the stream has synchronised.
void prof_collect() {
    for (auto& p : g_prof_pending) {
        float ms = 0.0f;
        if (hipEventElapsedTime(&ms, p.a, p.b) == hipSuccess) {
            g_prof_ms[p.kind] += ms;
            g_prof_launches[p.kind] += 1;
            if (p.kind == 0) g_prof_seq_steps += p.seq_steps;
        }
        (void)hipEventDestroy(p.a);
        (void)hipEventDestroy(p.b);
    }
    g_prof_pending.clear();
}
// Bounds and budgets from the environment, read on every call (as the
// reference does, viterbi_esimd.cpp:924-933), so a caller may change them
// between calls.
//   host-pointer entries (xtq_vit_run, xtq_vit_run_k), the reference's
//   bounds and defaults:
//     XTQ_VIT_MAXSEQ    nseq per call (default 4096)            -> status 6
//     XTQ_VIT_MAXBYTES  nseq * 1,317,888 B, the reference's worst-case
//                       device bytes per sequence (default 6 GiB) -> status 5
//   every entry:
//     XTQ_VIT_DEV_MAXBYTES  library-owned device bytes (default 64 GiB)
//                       -> status 5
//     XTQ_VIT_SCRATCH   backpointer scratch budget; larger batches run in
//                       chunks (default 8 GiB)
//     XTQ_VIT_DEFER_SCRATCH  the same for the deferred-argmin encode's minima
//                       rows (default 48 GiB, at most half the free memory)
long long g_host_maxseq = 4096;
size_t g_host_maxbytes = (size_t)6 << 30;
size_t g_maxbytes = (size_t)64 << 30;
size_t g_scratch = (size_t)8 << 30;
size_t g_defer_scratch = (size_t)48 << 30;
// Worst-case device bytes per sequence of the reference's library (X 1 KiB,
// states 1 KiB, cost table 256 KiB, backpointers 1 MiB).
constexpr size_t kRefBytesPerSeq = 1317888;

void read_env() {
    const char* e;
    g_host_maxseq = (e = getenv("XTQ_VIT_MAXSEQ")) ? atoll(e) : 4096;
    g_host_maxbytes = (e = getenv("XTQ_VIT_MAXBYTES")) ? strtoull(e, nullptr, 10)
                                                       : (size_t)6 << 30;
    g_maxbytes = (e = getenv("XTQ_VIT_DEV_MAXBYTES")) ? strtoull(e, nullptr, 10)
                                                      : (size_t)64 << 30;
    g_scratch = (e = getenv("XTQ_VIT_SCRATCH")) ? strtoull(e, nullptr, 10) : (size_t)8 << 30;
    g_defer_scratch = (e = getenv("XTQ_VIT_DEFER_SCRATCH")) ? strtoull(e, nullptr, 10)
                                                             : (size_t)48 << 30;
}

// Makes `dev` ready on the calling thread (which must have it current).
int dev_init(int dev) {
    read_env();
    int ndev = 0;
    if (hipGetDeviceCount(&ndev) != hipSuccess || ndev <= 0) {
        fprintf(stderr, "xtq_vit: no HIP device\n");
        return 1;
    }
    if ((int)g_dev.size() < ndev) g_dev.resize(ndev);
    DevCtx& cx = g_dev[dev];
    if (cx.ready) return 0;
    if (hipDeviceGetAttribute(&cx.ncu, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
        return 1;
    std::vector<float> h(65536);
    for (int c = 0; c < kNumCodes; ++c) {
        if (hipMalloc((void**)&cx.lut[c], 65536 * sizeof(float)) != hipSuccess) return 2;
        make_lut((Code)c, h.data());
        if (hipMemcpy(cx.lut[c], h.data(), 65536 * sizeof(float), hipMemcpyHostToDevice) !=
            hipSuccess)
            return 1;
    }
    if (hipMalloc((void**)&cx.err, sizeof(uint32_t)) != hipSuccess) return 2;
    if (hipMemset(cx.err, 0, sizeof(uint32_t)) != hipSuccess) return 1;
    if (hipMalloc((void**)&cx.counter, sizeof(int32_t)) != hipSuccess) return 2;
    if (hipEventCreateWithFlags(&cx.last, hipEventDisableTiming) != hipSuccess) return 1;
    if (hipEventRecord(cx.last, 0) != hipSuccess) return 1;
    // this device's copy of the no-allocation scratch (the device is current)
    void* na = nullptr;
    if (hipGetSymbolAddress(&na, HIP_SYMBOL(scratch)) != hipSuccess || na == nullptr) {
        fprintf(stderr, "xtq_vit: no device address for the no-allocation scratch\n");
        return 1;
    }
    cx.noalloc = (uint8_t*)na;
    cx.owned = kNumCodes * 65536 * sizeof(float) + 256;
    cx.ready = true;
    return 0;
}

int current_device(int* dev) {
    return hipGetDevice(dev) == hipSuccess ? 0 : 1;
}

// Device selected by XTQ_VIT_DEVIDX (host-pointer entries), else current.
int host_entry_device(int* dev) {
    if (const char* e = getenv("XTQ_VIT_DEVIDX")) {
        int ndev = 0;
        if (hipGetDeviceCount(&ndev) != hipSuccess) return 1;
        const int idx = atoi(e);
        if (idx < 0 || idx >= ndev) {
            fprintf(stderr, "xtq_vit: XTQ_VIT_DEVIDX=%d, %d gpus\n", idx, ndev);
            return 3;
        }
        *dev = idx;
        return 0;
    }
    return current_device(dev);
}

template <typename P>
int grow(P** p, size_t* cap, size_t want, size_t elem, size_t* owned) {
    if (want <= *cap) return 0;
    if (*p) {
        (void)hipFree(*p);
        *owned -= *cap * elem;
    }
    *p = nullptr;
    *cap = 0;
    if (hipMalloc((void**)p, want * elem) != hipSuccess) {
        *p = nullptr;
        return 2;
    }
    *cap = want;
    *owned += want * elem;
    return 0;
}

// Releases a buffer whose capacity is tracked in *cap (a failed grow of a
// group of buffers sharing one capacity leaves them in step again).
template <typename P>
void release(P** p, size_t* cap, size_t elem, size_t* owned) {
    if (*p) {
        (void)hipFree(*p);
        *owned -= *cap * elem;
    }
    *p = nullptr;
    *cap = 0;
}

// K, pivot and margin of a tail-bite call.
int check_args(int K, int margin, int pivot) {
    if (K < 2 || K > 7) return 9;
    if (pivot < 0 || pivot >= xtq::kSteps || margin < 0) return 10;
    return 0;
}

// Scratch bytes per sequence: packed backpointers, or the minima rows of
// the deferred-argmin forward.
size_t scratch_per_seq(int K, bool defer) {
    return defer ? xtq::defer_tile_bytes(K) : xtq::bp_tile_bytes(K);
}

// Sequences per chunk for a scratch budget.
int chunk_size(const DevCtx& cx, int K, int nseq, bool defer = false) {
    const size_t per = scratch_per_seq(K, defer);
    size_t budget = g_scratch;
    if (defer) {
        // the minima rows take 8x the backpointers' bytes at K=4: a larger
        // budget keeps the chunks (each one latency-bound traceback launch
        // per pass) at thousands of sequences, capped at half of the device
        // memory this library could hold
        budget = g_defer_scratch;
        size_t fr = 0, tot = 0;
        if (hipMemGetInfo(&fr, &tot) == hipSuccess) {
            const size_t avail = (fr + cx.bp_cap) / 2;
            if (budget > avail) budget = avail;
        }
    }
    size_t ch = budget / per;
    if (ch < 1) ch = 1;
    const size_t round = (size_t)4 * (cx.ncu > 0 ? cx.ncu : 1);
    if (ch > round) ch -= ch % round;
    if (ch > (size_t)nseq) ch = nseq;
    return (int)ch;
}

// Grows the backpointer/final-state scratch for `chunk` sequences of K.
int reserve_scratch(DevCtx& cx, int K, int chunk, bool defer = false) {
    const size_t per = scratch_per_seq(K, defer);
    // A stream-ordered call may still be using the buffers about to be
    // replaced.
    if (((size_t)chunk * per > cx.bp_cap || (size_t)chunk > cx.seq_cap) &&
        hipEventSynchronize(cx.last) != hipSuccess)
        return 4;
    // Device bytes this call adds to what the library already holds.
    size_t add = 0;
    if ((size_t)chunk * per > cx.bp_cap) add += (size_t)chunk * per - cx.bp_cap;
    if ((size_t)chunk > cx.seq_cap) add += ((size_t)chunk - cx.seq_cap) * 3 * sizeof(int32_t);
    if (cx.owned + add > g_maxbytes) {
        fprintf(stderr, "xtq_vit: request over XTQ_VIT_DEV_MAXBYTES (%zu)\n", g_maxbytes);
        return 5;
    }
    // (the capacity follows the pointer also when the growth fails: grow
    // leaves a null pointer and a zero capacity then)
    size_t bpcap_bytes = cx.bp_cap;
    const int gb = grow((uint8_t**)&cx.bp, &bpcap_bytes, (size_t)chunk * per, 1, &cx.owned);
    cx.bp_cap = bpcap_bytes;
    if (gb) return 2;
    size_t sc = cx.seq_cap;
    if ((size_t)chunk > sc) {
        // send, ov and flags share seq_cap: each keeps its own capacity
        // while they grow, and a failure releases all three
        size_t sc2 = cx.seq_cap, sc3 = cx.seq_cap;
        int g = grow(&cx.send, &sc, (size_t)chunk, sizeof(int32_t), &cx.owned);
        if (!g) g = grow(&cx.ov, &sc2, (size_t)chunk, sizeof(int32_t), &cx.owned);
        if (!g) g = grow(&cx.flags, &sc3, (size_t)chunk, sizeof(uint32_t), &cx.owned);
        if (g) {
            release(&cx.send, &sc, sizeof(int32_t), &cx.owned);
            release(&cx.ov, &sc2, sizeof(int32_t), &cx.owned);
            release(&cx.flags, &sc3, sizeof(uint32_t), &cx.owned);
            cx.seq_cap = 0;
            return 2;
        }
        // fresh flags hold no epoch of a launch (epochs start at 1)
        if (hipMemset(cx.flags, 0, (size_t)chunk * sizeof(uint32_t)) != hipSuccess) return 4;
        cx.seq_cap = sc;
    }
    return 0;
}

// Waits for the stream and turns the device NaN flag into status 11.
int finish(DevCtx& cx, hipStream_t s) {
    uint32_t herr = 0;
    if (hipMemcpyAsync(&herr, cx.err, sizeof(herr), hipMemcpyDeviceToHost, s) != hipSuccess ||
        hipStreamSynchronize(s) != hipSuccess) {
        fprintf(stderr, "xtq_vit run: %s\n", hipGetErrorString(hipGetLastError()));
        return 4;
    }
    prof_collect();
    if (herr) {
        (void)hipMemset(cx.err, 0, sizeof(uint32_t));
        if (herr & 6u) {
            fprintf(stderr, "xtq_vit: persistent kernel %s\n",
                    (herr & 2u) ? "wait expired" : "task out of range");
            return 4;
        }
        fprintf(stderr, "xtq_vit: NaN target\n");
        return 11;
    }
    return 0;
}

int pick_group(const DevCtx& cx, int K, int n) {
    int T = xtq::forward_group(K, n, cx.ncu);
    if (const char* g = getenv("XTQ_VIT_GROUP")) {
        // Test hook: force the sequences per workgroup (1, 2, 4 or 8), clamped
        // to what the LDS footprint for K allows.
        const int want = atoi(g);
        const int cap = xtq::forward_group(K, 1 << 30, 1);
        if (want == 1 || want == 2 || want == 4 || want == 8) T = want < cap ? want : cap;
    }
    return T;
}

// Orders a call's use of the library scratch after the previous call's.
int scratch_begin(DevCtx& cx, hipStream_t s) {
    return hipStreamWaitEvent(s, cx.last, 0) == hipSuccess ? 0 : 4;
}

// Marks the end of a call's scratch use; a synchronous call then waits for
// its stream and reports the NaN flag.
int scratch_end(DevCtx& cx, hipStream_t s, bool sync) {
    if (hipEventRecord(cx.last, s) != hipSuccess) return 4;
    return sync ? finish(cx, s) : 0;
}

// Whether a chunk of n sequences runs as one fused two-pass launch:
// XTQ_VIT_FUSED=0 never, =1 always, unset: batches below 4 sequences per CU
// (where separate pass launches leave CUs idle in their last round).
bool use_fused(const DevCtx& cx, int n) {
    if (const char* e = getenv("XTQ_VIT_FUSED")) {
        if (!strcmp(e, "0")) return false;
        if (!strcmp(e, "1")) return true;
    }
    return n < 4 * (cx.ncu > 0 ? cx.ncu : 1);
}

// Whether the tracebacks of a chunk of n sequences use one lane per
// sequence: XTQ_VIT_TB_LANES=N sets the smallest such chunk (0: always,
// -1: never); default 2048 (below it, whole-row staging by one workgroup per
// sequence finishes sooner than a per-lane chain of dependent loads).
bool use_lanes(int n) {
    long long min_n = 2048;
    if (const char* e = getenv("XTQ_VIT_TB_LANES")) min_n = atoll(e);
    return min_n >= 0 && n >= min_n;
}

// Whether a tail-bite at K runs the deferred-argmin forward (group minima
// rows in HBM, argmin recomputed by the traceback): XTQ_VIT_DEFER=1 for
// K >= 4, else never.  Measured on the 348,160-tile K=4..7 workloads it is
// as fast end to end at K=4 and 2-5 % slower at K=5..7: its forward gains
// 7-12 %, its one-lane tracebacks recomputing NC candidates per link from
// scattered minima rows give it back.
bool use_defer(int K, int nseq) {
    (void)nseq;
    if (K < 4) return false;
    const char* e = getenv("XTQ_VIT_DEFER");
    return e && !strcmp(e, "1");
}

// Polls before a pass-2 wait in the fused kernel gives up (~1 us each, so
// seconds; a pass-1 task takes about a millisecond).
constexpr int kSpinLimit = 1 << 22;

// Device scratch of one tail-bite call: backpointer slots (bp_tile_bytes(K)
// per sequence of a chunk), per-sequence final state / pass-1 pin / fused
// ready flag, the fused kernel's task counter and the status word.
struct TbScratch {
    void* bp;
    int32_t* send;
    int32_t* ov;
    uint32_t* flags;
    int32_t* counter;
    uint32_t* err;
};

// The two-pass tail-biting schedule (quantize.py:323-354) over chunks of
// `chunk` sequences, enqueued on s with the buffers in w.  prof: bracket the
// launches with timing events (the benchmark's kernel timing).
int tailbite_chunks(DevCtx& cx, const TbScratch& w, int chunk, const float* dX, int nseq,
                    int K, Code code, int margin, int pivot, int32_t* d_states,
                    int16_t* d_trellis, hipStream_t s, bool prof, bool defer = false) {
    const int n1 = (margin > 0 && pivot + margin < xtq::kSteps) ? pivot + margin : xtq::kSteps;
    const float* lut = cx.lut[code];
    auto pbeg = [&](int kind, double steps) { return prof ? prof_begin(s, kind, steps) : -1; };
    for (int c0 = 0; c0 < nseq; c0 += chunk) {
        const int n = (nseq - c0) < chunk ? (nseq - c0) : chunk;
        const float* x = dX + (size_t)c0 * xtq::kSteps;
        int32_t* st = d_states ? d_states + (size_t)c0 * xtq::kSteps : nullptr;
        int16_t* tr = d_trellis ? d_trellis + (size_t)c0 * 16 * K : nullptr;
        const int T = pick_group(cx, K, n);
        hipError_t e;
        if (defer) {
            // Pass 1, free on the rolled sequence: minima rows from step
            // pivot, traced back to ov = s_pivot >> K; pass 2 pinned to ov.
            int pf = pbeg(0, (double)n * n1);
            e = xtq::launch_forward_defer(K, x, xtq::kSteps, xtq::kSteps, n, lut, pivot, n1,
                                          pivot, nullptr, w.bp, w.send, w.err, T, s);
            prof_end(pf, s);
            if (e == hipSuccess) {
                pf = pbeg(1, 0.0);
                e = xtq::launch_traceback_defer(K, w.bp, x, xtq::kSteps, xtq::kSteps, pivot, lut,
                                                n, w.send, nullptr, n1, pivot, K, w.ov, nullptr,
                                                nullptr, s);
                prof_end(pf, s);
            }
            if (e == hipSuccess) {
                pf = pbeg(0, (double)n * xtq::kSteps);
                e = xtq::launch_forward_defer(K, x, xtq::kSteps, xtq::kSteps, n, lut, 0,
                                              xtq::kSteps, 0, w.ov, w.bp, w.send, w.err, T, s);
                prof_end(pf, s);
            }
            if (e == hipSuccess) {
                pf = pbeg(1, 0.0);
                e = xtq::launch_traceback_defer(K, w.bp, x, xtq::kSteps, xtq::kSteps, 0, lut, n,
                                                w.send, w.ov, xtq::kSteps, 0, 0, nullptr, st,
                                                tr, s);
                prof_end(pf, s);
            }
            if (e != hipSuccess) {
                fprintf(stderr, "xtq_vit run: %s\n", hipGetErrorString(e));
                return 4;
            }
            continue;
        }
        if (use_fused(cx, n)) {
            if (++cx.epoch == 0) cx.epoch = 1;
            int pf = pbeg(0, (double)n * (n1 + xtq::kSteps));
            e = xtq::launch_tailbite_fused(K, x, n, lut, pivot, n1, w.bp, w.send, w.ov, w.flags,
                                           w.counter, cx.epoch, kSpinLimit, w.err, s);
            prof_end(pf, s);
            if (e == hipSuccess) {
                pf = pbeg(1, 0.0);
                e = xtq::launch_traceback(K, w.bp, n, w.send, xtq::kSteps, 0, 0, nullptr, st,
                                          tr, use_lanes(n), s);
                prof_end(pf, s);
            }
            if (e != hipSuccess) {
                fprintf(stderr, "xtq_vit run: %s\n", hipGetErrorString(e));
                return 4;
            }
            continue;
        }
        // Pass 1: free run over the sequence rolled right by pivot, n1 steps,
        // traced back to step pivot: ov = s_pivot >> K.
        int pf = pbeg(0, (double)n * n1);
        e = xtq::launch_forward(K, x, xtq::kSteps, xtq::kSteps, n, lut, pivot, n1, pivot,
                                nullptr, w.bp, w.send, w.err, T, s);
        prof_end(pf, s);
        if (e == hipSuccess) {
            pf = pbeg(1, 0.0);
            e = xtq::launch_traceback(K, w.bp, n, w.send, n1, pivot, K, w.ov, nullptr, nullptr,
                                      use_lanes(n), s);
            prof_end(pf, s);
        }
        // Pass 2: run pinned to ov on the unrolled sequence, full traceback.
        if (e == hipSuccess) {
            pf = pbeg(0, (double)n * xtq::kSteps);
            e = xtq::launch_forward(K, x, xtq::kSteps, xtq::kSteps, n, lut, 0, xtq::kSteps, 0,
                                    w.ov, w.bp, w.send, w.err, T, s);
            prof_end(pf, s);
        }
        if (e == hipSuccess) {
            pf = pbeg(1, 0.0);
            e = xtq::launch_traceback(K, w.bp, n, w.send, xtq::kSteps, 0, 0, nullptr, st, tr,
                                      use_lanes(n), s);
            prof_end(pf, s);
        }
        if (e != hipSuccess) {
            fprintf(stderr, "xtq_vit run: %s\n", hipGetErrorString(e));
            return 4;
        }
    }
    return 0;
}

// The tail-bite over the library-owned, grow-only scratch (chunked by the
// XTQ_VIT_SCRATCH budget).
int run_tailbite(DevCtx& cx, const float* dX, int nseq, int K, Code code, int margin,
                 int pivot, int32_t* d_states, int16_t* d_trellis, hipStream_t s,
                 bool sync = true) {
    const bool defer = use_defer(K, nseq);
    const int chunk = chunk_size(cx, K, nseq, defer);
    int rc = reserve_scratch(cx, K, chunk, defer);
    if (!rc) rc = scratch_begin(cx, s);
    if (rc) return rc;
    const TbScratch w{cx.bp, cx.send, cx.ov, cx.flags, cx.counter, cx.err};
    rc = tailbite_chunks(cx, w, chunk, dX, nseq, K, code, margin, pivot, d_states, d_trellis,
                         s, true, defer);
    if (rc) return rc;
    return scratch_end(cx, s, sync);
}

// --------------------------------------------- tail-bite without allocation
// Sequences of K one call of the no-allocation entry can take: a header,
// three words per sequence, up to 255 bytes of alignment, and the
// backpointer slots.
size_t noalloc_capacity(int K) {
    return (kNoAllocBytes - kNoAllocHeader - 256) / (xtq::bp_tile_bytes(K) + 3 * sizeof(int32_t));
}

// xtq_vit_tailbite_dev over the device's copy of `scratch` (its address in
// cx.noalloc, taken once at set-up): no allocation, one chunk, synchronous.
int run_tailbite_noalloc(DevCtx& cx, const float* dX, int nseq, int K, Code code, int margin,
                         int pivot, int32_t* d_states, int16_t* d_trellis, hipStream_t s) {
    const size_t cap = noalloc_capacity(K);
    if ((size_t)nseq > cap) {
        fprintf(stderr, "xtq_vit: nseq %d exceeds the no-allocation scratch (%zu sequences at "
                "K=%d)\n", nseq, cap, K);
        return 5;
    }
    uint8_t* base = cx.noalloc;
    TbScratch w;
    w.err = (uint32_t*)base;
    w.counter = (int32_t*)(base + 4);
    w.send = (int32_t*)(base + kNoAllocHeader);
    w.ov = w.send + nseq;
    w.flags = (uint32_t*)(w.ov + nseq);
    const uintptr_t bp = ((uintptr_t)(w.flags + nseq) + 255) & ~(uintptr_t)255;
    w.bp = (void*)bp;
    if (bp + (size_t)nseq * xtq::bp_tile_bytes(K) > (uintptr_t)(base + kNoAllocBytes)) return 5;
    // The array keeps the previous call's contents: the status word and the
    // fused kernel's ready flags must start at zero (epochs start at 1).
    hipError_t e = xtq::launch_fill_u32(w.err, 1, 0u, s);
    if (e == hipSuccess) e = xtq::launch_fill_u32(w.flags, (uint32_t)nseq, 0u, s);
    if (e != hipSuccess) {
        fprintf(stderr, "xtq_vit run: %s\n", hipGetErrorString(e));
        return 4;
    }
    int rc = tailbite_chunks(cx, w, nseq, dX, nseq, K, code, margin, pivot, d_states,
                             d_trellis, s, false);
    if (rc) return rc;
    uint32_t herr = 0;
    if (hipMemcpyAsync(&herr, w.err, sizeof(herr), hipMemcpyDeviceToHost, s) != hipSuccess ||
        hipStreamSynchronize(s) != hipSuccess) {
        fprintf(stderr, "xtq_vit run: %s\n", hipGetErrorString(hipGetLastError()));
        return 4;
    }
    if (herr & 6u) {
        fprintf(stderr, "xtq_vit: persistent kernel %s\n",
                (herr & 2u) ? "wait expired" : "task out of range");
        return 4;
    }
    if (herr) {
        fprintf(stderr, "xtq_vit: NaN target\n");
        return 11;
    }
    return 0;
}

// Relative cost of one tile of the chain kernel per K, for splitting the CUs
// between groups: kernel times of the 5120x5120 sweep (344 / 319 / 309 /
// 290 / 289 / 309 ms for K = 2..7), K = 7 raised by 2 % to the K=7 : K=5
// ratio measured with both running side by side (c4's q at K=5, k and v at
// K=7).
double chain_tile_cost(int K) {
    static const double c[8] = {1.0, 1.0, 1.11, 1.03, 1.0, 0.94, 0.94, 1.02};
    return (K >= 2 && K <= 7) ? c[K] : 1.0;
}

// Workgroups per group: proportional to the group's work, at most one per
// column chain, at least one, summing to at most ncu.
void split_cus(int ncu, int ng, const int* tng, const int* Kg, int tk, int* nwg) {
    if (ng == 1) {
        // more workgroups than column chains could only wait
        nwg[0] = tng[0] < ncu ? tng[0] : ncu;
        return;
    }
    double w[kMaxChainGroups], tot = 0.0;
    bool capped[kMaxChainGroups] = {};
    for (int g = 0; g < ng; ++g) tot += (w[g] = (double)tng[g] * tk * chain_tile_cost(Kg[g]));
    int left = ncu;
    // water-filling: groups with fewer chains than their share keep one
    // workgroup per chain and give the rest to the others
    for (bool again = true; again;) {
        again = false;
        double wt = 0.0;
        for (int g = 0; g < ng; ++g)
            if (!capped[g]) wt += w[g];
        for (int g = 0; g < ng; ++g) {
            if (capped[g]) continue;
            if (wt > 0 && (double)left * w[g] / wt > tng[g]) {
                capped[g] = true;
                nwg[g] = tng[g];
                left -= tng[g];
                again = true;
            }
        }
        if (!again) {
            int used = 0, big = -1;
            for (int g = 0; g < ng; ++g) {
                if (capped[g]) continue;
                nwg[g] = (int)((double)left * w[g] / (wt > 0 ? wt : 1.0));
                if (nwg[g] < 1) nwg[g] = 1;
                used += nwg[g];
                if (big < 0 || w[g] > w[big]) big = g;
            }
            if (big >= 0) nwg[big] += left - used;       // rounding remainder
            for (int g = 0; g < ng; ++g)
                if (nwg[g] < 1) nwg[g] = 1;
        }
    }
    (void)tot;
}

struct ChainGroup { int jc0, tnl, K; int16_t* trellis; };

// The BlockLDLQ sweep as column chains (see ldlq_chain_kernel): the factor
// repacked once, then one persistent launch per column group, the first on
// the caller's stream and the others concurrently on library streams, with
// the CUs split by work.  Library-owned E, tile flags, per-workgroup
// backpointer slots and target rows.
int run_ldlq_chain(DevCtx& cx, const float* W, const float* L, int k, int n,
                   const ChainGroup* grp, int ng, Code code, int margin, int pivot,
                   int buf_cols, float* hatW, int32_t* states, float* targets, hipStream_t s) {
    const int tk = k / 16;
    const size_t ntile = (size_t)tk * (size_t)(n / 16);
    int tng[kMaxChainGroups], Kg[kMaxChainGroups], nwg[kMaxChainGroups];
    for (int g = 0; g < ng; ++g) { tng[g] = grp[g].tnl; Kg[g] = grp[g].K; }
    split_cus(cx.ncu > 0 ? cx.ncu : 1, ng, tng, Kg, tk, nwg);
    size_t bp_bytes = 0, xrows = 0;
    size_t bp_off[kMaxChainGroups], x_off[kMaxChainGroups];
    for (int g = 0; g < ng; ++g) {
        bp_off[g] = bp_bytes;
        x_off[g] = xrows;
        bp_bytes += (size_t)nwg[g] * xtq::bp_tile_bytes(Kg[g]);
        xrows += (size_t)nwg[g];
    }
    const size_t need_e = (size_t)k * n, need_x = targets ? 0 : xrows * xtq::kSteps;
    const size_t need_lt = L ? (size_t)k * k : 0;
    size_t add = 0;
    if (bp_bytes > cx.bp_cap) add += bp_bytes - cx.bp_cap;
    if (need_e > cx.e_cap) add += (need_e - cx.e_cap) * sizeof(float);
    if (need_lt > cx.lt_cap) add += (need_lt - cx.lt_cap) * sizeof(float);
    if (ntile > cx.cflags_cap) add += (ntile - cx.cflags_cap) * sizeof(uint32_t);
    if (need_x > cx.xbuf_cap) add += (need_x - cx.xbuf_cap) * sizeof(float);
    if (cx.owned + add > g_maxbytes) {
        fprintf(stderr, "xtq_vit: request over XTQ_VIT_DEV_MAXBYTES (%zu)\n", g_maxbytes);
        return 5;
    }
    if (add && hipEventSynchronize(cx.last) != hipSuccess) return 4;
    {
        size_t cap = cx.bp_cap;
        const int gb = grow((uint8_t**)&cx.bp, &cap, bp_bytes, 1, &cx.owned);
        cx.bp_cap = cap;
        if (gb) return 2;
    }
    if (grow(&cx.E, &cx.e_cap, need_e, sizeof(float), &cx.owned)) return 2;
    if (grow(&cx.Lt, &cx.lt_cap, need_lt, sizeof(float), &cx.owned)) return 2;
    if (ntile > cx.cflags_cap) {
        if (grow(&cx.cflags, &cx.cflags_cap, ntile, sizeof(uint32_t), &cx.owned)) return 2;
        if (hipMemset(cx.cflags, 0, ntile * sizeof(uint32_t)) != hipSuccess) return 4;
    }
    if (grow(&cx.xbuf, &cx.xbuf_cap, need_x, sizeof(float), &cx.owned)) return 2;
    if (!cx.ccount) {
        if (hipMalloc((void**)&cx.ccount, kMaxChainGroups * sizeof(int32_t)) != hipSuccess)
            return 2;
        cx.owned += kMaxChainGroups * sizeof(int32_t);
    }
    for (int g = 1; g < ng; ++g) {
        if (!cx.side[g - 1] &&
            (hipStreamCreateWithFlags(&cx.side[g - 1], hipStreamNonBlocking) != hipSuccess ||
             hipEventCreateWithFlags(&cx.join[g - 1], hipEventDisableTiming) != hipSuccess))
            return 1;
    }
    if (ng > 1 && !cx.fork && hipEventCreateWithFlags(&cx.fork, hipEventDisableTiming) != hipSuccess)
        return 1;
    int rc = scratch_begin(cx, s);
    if (rc) return rc;
    if (++cx.epoch == 0) cx.epoch = 1;
    const int n1 = (margin > 0 && pivot + margin < xtq::kSteps) ? pivot + margin : xtq::kSteps;
    double steps = 0.0;
    for (int g = 0; g < ng; ++g) steps += (double)tk * tng[g] * (n1 + xtq::kSteps);
    const int pf = prof_begin(s, 0, steps);
    hipError_t e = hipSuccess;
    if (L) e = xtq::launch_lfac_quads(L, k, cx.Lt, s);
    if (e == hipSuccess && ng > 1 && hipEventRecord(cx.fork, s) != hipSuccess) e = hipErrorUnknown;
    for (int g = 0; g < ng && e == hipSuccess; ++g) {
        hipStream_t sg = g ? cx.side[g - 1] : s;
        if (g && hipStreamWaitEvent(sg, cx.fork, 0) != hipSuccess) {
            e = hipErrorUnknown;
            break;
        }
        e = xtq::launch_ldlq_chain(
            Kg[g], W, L ? cx.Lt : nullptr, k, n, grp[g].jc0, grp[g].tnl, cx.lut[code], pivot,
            n1, (uint8_t*)cx.bp + bp_off[g], nwg[g], targets ? targets : cx.xbuf + x_off[g] * xtq::kSteps,
            targets ? 1 : 0, hatW, cx.E, states, grp[g].trellis, cx.cflags, cx.ccount + g,
            cx.epoch, kSpinLimit, cx.err, buf_cols, sg);
        if (e == hipSuccess && g &&
            (hipEventRecord(cx.join[g - 1], sg) != hipSuccess ||
             hipStreamWaitEvent(s, cx.join[g - 1], 0) != hipSuccess))
            e = hipErrorUnknown;
    }
    prof_end(pf, s);
    if (e != hipSuccess) {
        fprintf(stderr, "xtq_vit ldlq chain: %s\n", hipGetErrorString(e));
        (void)hipDeviceSynchronize();
        return 4;
    }
    return scratch_end(cx, s, true);
}

// One Viterbi run (quantize.py:218-320) over device buffers: free or pinned,
// full traceback or only the state at back_from.
int run_viterbi(DevCtx& cx, const float* dX, int nseq, int T, int K, Code code,
                const int32_t* d_ov, int back_from, int32_t* d_out, hipStream_t s) {
    const int chunk = chunk_size(cx, K, nseq);
    int rc = reserve_scratch(cx, K, chunk);
    if (!rc) rc = scratch_begin(cx, s);
    if (rc) return rc;
    const float* lut = cx.lut[code];
    const int stop = back_from >= 0 ? back_from : 0;
    for (int c0 = 0; c0 < nseq; c0 += chunk) {
        const int n = (nseq - c0) < chunk ? (nseq - c0) : chunk;
        const int G = pick_group(cx, K, n);
        hipError_t e = xtq::launch_forward(K, dX + (size_t)c0 * T, T, T, n, lut, 0, T, stop,
                                           d_ov ? d_ov + c0 : nullptr, cx.bp, cx.send,
                                           cx.err, G, s);
        if (e == hipSuccess) {
            if (back_from >= 0)
                e = xtq::launch_traceback(K, cx.bp, n, cx.send, T, back_from, 0, d_out + c0,
                                          nullptr, nullptr, use_lanes(n), s);
            else
                e = xtq::launch_traceback(K, cx.bp, n, cx.send, T, 0, 0, nullptr,
                                          d_out + (size_t)c0 * T, nullptr, use_lanes(n), s);
        }
        if (e != hipSuccess) {
            fprintf(stderr, "xtq_vit viterbi: %s\n", hipGetErrorString(e));
            return 4;
        }
    }
    return scratch_end(cx, s, true);
}

// Host-pointer tail-bite: stage X, run, copy the states back.
int run_host(const float* X, int nseq, int K, Code code, int margin, int pivot,
             int32_t* out) {
    if (!X || !out) return 12;
    read_env();
    // the reference's bounds, in its order (viterbi_esimd.cpp:973-982)
    if (nseq <= 0 || nseq > g_host_maxseq) {
        fprintf(stderr, "xtq_vit: nseq %d over XTQ_VIT_MAXSEQ\n", nseq);
        return 6;
    }
    if ((size_t)nseq * kRefBytesPerSeq > g_host_maxbytes) {
        fprintf(stderr, "xtq_vit: nseq %d over XTQ_VIT_MAXBYTES\n", nseq);
        return 5;
    }
    int rc = check_args(K, margin, pivot);
    if (rc) return rc;
    int dev = 0, prev = 0;
    rc = host_entry_device(&dev);
    if (rc) return rc;
    if (hipGetDevice(&prev) != hipSuccess) return 1;
    if (dev != prev && hipSetDevice(dev) != hipSuccess) return 1;
    rc = dev_init(dev);
    if (!rc) {
        DevCtx& cx = g_dev[dev];
        const size_t add = (size_t)nseq > cx.host_cap
                               ? ((size_t)nseq - cx.host_cap) * 2 * xtq::kSteps * 4 : 0;
        if (cx.owned + add > g_maxbytes) {
            fprintf(stderr, "xtq_vit: nseq %d over XTQ_VIT_DEV_MAXBYTES\n", nseq);
            rc = 5;
        }
        // capacities in elements (host_cap counts sequences of kSteps)
        size_t c1 = cx.host_cap * xtq::kSteps, c2 = c1;
        if (!rc && (size_t)nseq > cx.host_cap && hipEventSynchronize(cx.last) != hipSuccess)
            rc = 4;
        if (!rc && (size_t)nseq > cx.host_cap) {
            if (grow(&cx.hx, &c1, (size_t)nseq * xtq::kSteps, sizeof(float), &cx.owned) ||
                grow(&cx.hs, &c2, (size_t)nseq * xtq::kSteps, sizeof(int32_t), &cx.owned)) {
                release(&cx.hx, &c1, sizeof(float), &cx.owned);
                release(&cx.hs, &c2, sizeof(int32_t), &cx.owned);
                cx.host_cap = 0;
                rc = 2;
            } else {
                cx.host_cap = nseq;
            }
        }
        if (!rc && hipMemcpy(cx.hx, X, (size_t)nseq * xtq::kSteps * 4, hipMemcpyHostToDevice) !=
                       hipSuccess)
            rc = 4;
        if (!rc) rc = run_tailbite(cx, cx.hx, nseq, K, code, margin, pivot, cx.hs, nullptr, 0);
        // The states come back through pinned staging (a DMA at full PCIe
        // rate, then one host copy): the runtime's pageable path copies
        // device-to-host at a few GB/s.  Without the staging (allocation
        // failed) they take that path.
        const size_t nel = (size_t)nseq * xtq::kSteps;
        if (!rc && nel > cx.hpin_cap) {
            if (cx.hpin) (void)hipHostFree(cx.hpin);
            cx.hpin = nullptr;
            cx.hpin_cap = 0;
            if (hipHostMalloc((void**)&cx.hpin, nel * sizeof(int32_t), hipHostMallocDefault) ==
                hipSuccess) {
                cx.hpin_cap = nel;
            } else {
                cx.hpin = nullptr;
                (void)hipGetLastError();   // not left for a later launch check to report
            }
        }
        if (!rc && cx.hpin) {
            if (hipMemcpy(cx.hpin, cx.hs, nel * sizeof(int32_t), hipMemcpyDeviceToHost) !=
                hipSuccess)
                rc = 4;
            else
                memcpy(out, cx.hpin, nel * sizeof(int32_t));
        } else if (!rc && hipMemcpy(out, cx.hs, nel * sizeof(int32_t), hipMemcpyDeviceToHost) !=
                              hipSuccess) {
            rc = 4;
        }
    }
    if (dev != prev) (void)hipSetDevice(prev);
    return rc;
}

}  // namespace

extern "C" {

int xtq_vit_init(void) {
    std::lock_guard<std::mutex> lk(g_mu);
    read_env();
    int dev = 0;
    int rc = host_entry_device(&dev);
    if (rc) return rc;
    int prev = 0;
    if (hipGetDevice(&prev) != hipSuccess) return 1;
    if (dev != prev && hipSetDevice(dev) != hipSuccess) return 1;
    rc = dev_init(dev);
    if (!rc) {
        hipDeviceProp_t p;
        if (hipGetDeviceProperties(&p, dev) == hipSuccess)
            fprintf(stderr, "xtq_vit: device %d %s (%s), %d CUs\n", dev, p.name, p.gcnArchName,
                    p.multiProcessorCount);
        fprintf(stderr, "xtq_vit: bounds nseq<=%lld devbytes<=%zu (library-owned <=%zu, "
                "scratch %zu)\n", g_host_maxseq, g_host_maxbytes, g_maxbytes, g_scratch);
    }
    if (dev != prev) (void)hipSetDevice(prev);
    return rc;
}

int xtq_vit_run(const float* X, int nseq, const char* code, int margin, int pivot,
                int32_t* out) {
    std::lock_guard<std::mutex> lk(g_mu);
    if (!code) return 12;
    if (!strcmp(code, "ih2x2")) {
        fprintf(stderr, "xtq_vit: code ih2x2 (V=2) is not supported\n");
        return 8;
    }
    if (strcmp(code, "mul1p") && strcmp(code, "mul1") && strcmp(code, "mul1t")) {
        fprintf(stderr, "xtq_vit: unknown code %s\n", code);
        return 8;
    }
    // The reference's kernel runs pass 1 over the whole sequence unless
    // margin > 0 (viterbi_esimd.cpp:413-414): a negative margin is margin 0.
    return run_host(X, nseq, 4, kMul1, margin < 0 ? 0 : margin, pivot, out);
}

int xtq_vit_run_k(const float* X, int nseq, int K, const char* code, int margin, int pivot,
                  int32_t* out) {
    std::lock_guard<std::mutex> lk(g_mu);
    Code c;
    int rc = parse_code(code, &c);
    if (rc) return rc;
    return run_host(X, nseq, K, c, margin, pivot, out);
}

}  // extern "C"

namespace {

// Shared body of the synchronous and stream-ordered device tail-bite entries.
int tailbite_dev(const float* dX, int nseq, int K, const char* code, int margin, int pivot,
                 int32_t* d_states, int16_t* d_trellis, void* stream, bool sync) {
    std::lock_guard<std::mutex> lk(g_mu);
    if (!dX || (!d_states && !d_trellis)) return 12;
    Code c;
    int rc = parse_code(code, &c);
    if (rc) return rc;
    read_env();
    if (nseq <= 0) return 6;
    rc = check_args(K, margin, pivot);
    if (rc) return rc;
    int dev = 0;
    if (current_device(&dev)) return 1;
    rc = dev_init(dev);
    if (rc) return rc;
    return run_tailbite(g_dev[dev], dX, nseq, K, c, margin, pivot, d_states, d_trellis,
                        (hipStream_t)stream, sync);
}

}  // namespace

extern "C" {

int xtq_vit_tailbite_dev(const float* dX, int nseq, int K, const char* code, int margin,
                         int pivot, int32_t* d_states, int16_t* d_trellis, void* stream) {
    return tailbite_dev(dX, nseq, K, code, margin, pivot, d_states, d_trellis, stream, true);
}

int xtq_vit_tailbite_dev_async(const float* dX, int nseq, int K, const char* code,
                               int margin, int pivot, int32_t* d_states, int16_t* d_trellis,
                               void* stream) {
    return tailbite_dev(dX, nseq, K, code, margin, pivot, d_states, d_trellis, stream, false);
}

int xtq_vit_tailbite_dev_noalloc(const float* dX, int nseq, int K, const char* code,
                                 int margin, int pivot, int32_t* d_states, int16_t* d_trellis,
                                 void* stream) {
    std::lock_guard<std::mutex> lk(g_mu);
    if (!dX || (!d_states && !d_trellis)) return 12;
    Code c;
    int rc = parse_code(code, &c);
    if (rc) return rc;
    read_env();
    if (nseq <= 0) return 6;
    rc = check_args(K, margin, pivot);
    if (rc) return rc;
    // Synchronous (it reads its status word back and waits for the stream),
    // so it refuses a stream under graph capture rather than invalidate the
    // caller's capture with a copy to the host and a synchronisation.
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing((hipStream_t)stream, &cs) != hipSuccess) {
        fprintf(stderr, "xtq_vit run: %s\n", hipGetErrorString(hipGetLastError()));
        return 4;
    }
    if (cs != hipStreamCaptureStatusNone) {
        fprintf(stderr, "xtq_vit: xtq_vit_tailbite_dev_noalloc is synchronous and cannot run on "
                "a stream under graph capture\n");
        return 13;
    }
    int dev = 0;
    if (current_device(&dev)) return 1;
    // Setting a device up allocates (codebook tables, status words): that is
    // the init call's job, never this entry's.
    if (dev >= (int)g_dev.size() || !g_dev[dev].ready) {
        fprintf(stderr, "xtq_vit: device %d is not set up; call xtq_vit_init (or any other "
                "entry point) on it before xtq_vit_tailbite_dev_noalloc\n", dev);
        return 1;
    }
    return run_tailbite_noalloc(g_dev[dev], dX, nseq, K, c, margin, pivot, d_states, d_trellis,
                                (hipStream_t)stream);
}

int xtq_vit_status_dev(void* stream) {
    std::lock_guard<std::mutex> lk(g_mu);
    int dev = 0;
    if (current_device(&dev)) return 1;
    int rc = dev_init(dev);
    if (rc) return rc;
    return finish(g_dev[dev], (hipStream_t)stream);
}

int xtq_ldlq_chain_dev(const float* d_W, const float* d_L, int k, int n, int K,
                       const char* code, int margin, int pivot, int buf_cols, float* d_hatW,
                       int32_t* d_states, int16_t* d_trellis, float* d_targets, void* stream) {
    int16_t* tr[1] = {d_trellis};
    return xtq_ldlq_chain_multi_dev(d_W, d_L, k, n, 1, &n, &K, code, margin, pivot, buf_cols,
                                    d_hatW, d_states, tr, d_targets, stream);
}

int xtq_ldlq_chain_multi_dev(const float* d_W, const float* d_L, int k, int n, int ngroups,
                             const int* h_ncols, const int* h_K, const char* code, int margin,
                             int pivot, int buf_cols, float* d_hatW, int32_t* d_states,
                             int16_t* const* h_trellis, float* d_targets, void* stream) {
    std::lock_guard<std::mutex> lk(g_mu);
    if (!d_W || !d_hatW || !h_ncols || !h_K || !h_trellis) return 12;
    Code c;
    int rc = parse_code(code, &c);
    if (rc) return rc;
    read_env();
    if (ngroups < 1 || ngroups > kMaxChainGroups) return 6;
    ChainGroup grp[kMaxChainGroups];
    int col = 0;
    for (int g = 0; g < ngroups; ++g) {
        if (h_K[g] < 2 || h_K[g] > 7) return 9;
        if (!h_trellis[g]) return 12;
        if (h_ncols[g] <= 0 || h_ncols[g] % 16) return 6;
        grp[g] = ChainGroup{col / 16, h_ncols[g] / 16, h_K[g], h_trellis[g]};
        col += h_ncols[g];
    }
    if (pivot < 0 || pivot >= xtq::kSteps || margin < 0) return 10;
    if (buf_cols < 16 || buf_cols % 16) return 6;
    if (d_L && ((uintptr_t)d_L & 15)) return 12;     // rows are read as float4
    if (k <= 0 || n <= 0 || k % 16 || n % 16 || col != n ||
        (long long)(k / 16) * (n / 16) > INT32_MAX || k > (1 << 22))
        return 6;
    int dev = 0;
    if (current_device(&dev)) return 1;
    rc = dev_init(dev);
    if (rc) return rc;
    return run_ldlq_chain(g_dev[dev], d_W, d_L, k, n, grp, ngroups, c, margin, pivot, buf_cols,
                          d_hatW, d_states, d_targets, (hipStream_t)stream);
}

int xtq_vit_viterbi_dev(const float* dX, int nseq, int T, int K, const char* code,
                        const int32_t* d_overlap, int back_from, int32_t* d_out,
                        void* stream) {
    std::lock_guard<std::mutex> lk(g_mu);
    if (!dX || !d_out) return 12;
    Code c;
    int rc = parse_code(code, &c);
    if (rc) return rc;
    read_env();
    if (nseq <= 0) return 6;
    if (K < 2 || K > 7) return 9;
    if (T < 1 || T > xtq::kSteps || back_from < -1 || back_from >= T) return 10;
    int dev = 0;
    if (current_device(&dev)) return 1;
    rc = dev_init(dev);
    if (rc) return rc;
    return run_viterbi(g_dev[dev], dX, nseq, T, K, c, d_overlap, back_from, d_out,
                       (hipStream_t)stream);
}

int xtq_trellis_decode_dev(const int16_t* d_trellis, int tk, int tn, int K, const char* code,
                           float* d_out_f32, uint16_t* d_out_f16, void* stream) {
    std::lock_guard<std::mutex> lk(g_mu);
    if (!d_trellis || (!d_out_f32 && !d_out_f16)) return 12;
    if (K < 2 || K > 7) return 9;
    if (tk <= 0 || tn <= 0 || (long long)tk * tn > (1LL << 31) - 1) return 6;
    Code c;
    int rc = parse_code(code, &c);
    if (rc) return rc;
    int dev = 0;
    if (current_device(&dev)) return 1;
    rc = dev_init(dev);
    if (rc) return rc;
    hipError_t e = xtq::launch_decode(K, d_trellis, tk, tn, g_dev[dev].lut[c], d_out_f32,
                                      d_out_f16, (hipStream_t)stream);
    if (e != hipSuccess) {
        fprintf(stderr, "xtq_vit decode: %s\n", hipGetErrorString(e));
        return 4;
    }
    return 0;
}

int xtq_trellis_pack_dev(const int32_t* d_states, int nt, int K, int16_t* d_trellis,
                         void* stream) {
    std::lock_guard<std::mutex> lk(g_mu);
    if (!d_states || !d_trellis) return 12;
    if (K < 2 || K > 7) return 9;
    if (nt <= 0) return 6;
    hipError_t e = xtq::launch_pack(K, d_states, nt, d_trellis, (hipStream_t)stream);
    if (e != hipSuccess) {
        fprintf(stderr, "xtq_vit pack: %s\n", hipGetErrorString(e));
        return 4;
    }
    return 0;
}

int xtq_trellis_unpack_dev(const int16_t* d_trellis, int nt, int K, int32_t* d_states,
                           void* stream) {
    std::lock_guard<std::mutex> lk(g_mu);
    if (!d_states || !d_trellis) return 12;
    if (K < 2 || K > 7) return 9;
    if (nt <= 0) return 6;
    hipError_t e = xtq::launch_unpack(K, d_trellis, nt, d_states, (hipStream_t)stream);
    if (e != hipSuccess) {
        fprintf(stderr, "xtq_vit unpack: %s\n", hipGetErrorString(e));
        return 4;
    }
    return 0;
}

int xtq_had128_left_dev(const float* d_ht, const float* d_in, float* d_out, int rows, int cols,
                        void* stream) {
    if (!d_ht || !d_in || !d_out) return 12;
    if (d_in == d_out) return 12;
    if (rows <= 0 || cols <= 0 || rows % 128 || rows / 128 > 65535) return 6;
    hipError_t e = xtq::launch_had_left(d_ht, d_in, d_out, rows, cols, (hipStream_t)stream);
    if (e != hipSuccess) {
        fprintf(stderr, "xtq_vit had128: %s\n", hipGetErrorString(e));
        return 4;
    }
    return 0;
}

int xtq_had128_right_dev(const float* d_h, const float* d_in, float* d_out, int rows, int cols,
                         void* stream) {
    if (!d_h || !d_in || !d_out) return 12;
    if (d_in == d_out) return 12;
    if (rows <= 0 || cols <= 0 || cols % 128 || (rows + 31) / 32 > 65535) return 6;
    hipError_t e = xtq::launch_had_right(d_h, d_in, d_out, rows, cols, (hipStream_t)stream);
    if (e != hipSuccess) {
        fprintf(stderr, "xtq_vit had128: %s\n", hipGetErrorString(e));
        return 4;
    }
    return 0;
}

int xtq_vit_get_lut(const char* code, float* out) {
    if (!out) return 12;
    Code c;
    int rc = parse_code(code, &c);
    if (rc) return rc;
    make_lut(c, out);
    return 0;
}

int64_t xtq_vit_scratch_per_seq(int K) {
    if (K < 2 || K > 7) return -1;
    return (int64_t)xtq::bp_tile_bytes(K);
}

int xtq_vit_chunk_seqs(int nseq, int K, int* deferred) {
    std::lock_guard<std::mutex> lk(g_mu);
    if (nseq <= 0) return -6;
    if (K < 2 || K > 7) return -9;
    read_env();
    int dev = 0;
    if (current_device(&dev)) return -1;
    const int rc = dev_init(dev);
    if (rc) return -rc;
    const bool defer = use_defer(K, nseq);
    if (deferred) *deferred = defer ? 1 : 0;
    return chunk_size(g_dev[dev], K, nseq, defer);
}

int xtq_vit_prof_enable(int on) {
    std::lock_guard<std::mutex> lk(g_mu);
    g_prof = on != 0;
    return 0;
}

int xtq_vit_prof_read(double* fwd_ms, int64_t* fwd_launches, double* fwd_seq_steps,
                      double* tb_ms, int64_t* tb_launches) {
    std::lock_guard<std::mutex> lk(g_mu);
    if (fwd_ms) *fwd_ms = g_prof_ms[0];
    if (fwd_launches) *fwd_launches = g_prof_launches[0];
    if (fwd_seq_steps) *fwd_seq_steps = g_prof_seq_steps;
    if (tb_ms) *tb_ms = g_prof_ms[1];
    if (tb_launches) *tb_launches = g_prof_launches[1];
    g_prof_ms[0] = g_prof_ms[1] = 0.0;
    g_prof_launches[0] = g_prof_launches[1] = 0;
    g_prof_seq_steps = 0.0;
    return 0;
}

const char* xtq_vit_strerror(int rc) {
    switch (rc) {
        case 0: return "ok";
        case 1: return "initialisation failed";
        case 2: return "device allocation failed";
        case 3: return "XTQ_VIT_DEVIDX names no device";
        case 4: return "HIP runtime error during a run";
        case 5: return "request exceeds XTQ_VIT_MAXBYTES or XTQ_VIT_DEV_MAXBYTES";
        case 6: return "sequence count out of range (XTQ_VIT_MAXSEQ for host pointers)";
        case 8: return "unsupported code";
        case 9: return "unsupported K";
        case 10: return "pivot or margin out of range";
        case 11: return "NaN target";
        case 12: return "null or misaligned pointer argument";
        case 13: return "synchronous entry given a stream under graph capture";
        default: return "unknown status";
    }
}

}  // extern "C"
