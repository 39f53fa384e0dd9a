// valu_probe.hip -- VALU issue-rate measurement for the forward DP's roofline
// (libxtqprobe.so, a benchmark helper: not part of the encoder library or
// its C-ABI; bound by probe/valu_probe.py).
//
// The forward DP spends four instructions per trellis candidate: the
// subtraction (v_add_f32 of -x with the codebook held in fp32 registers, or
// v_fma_mix_f32 with it held as packed fp16 pairs), v_mul_f32 (square),
// v_add_f32 (add) and v_min_f64 (min/argmin).  On gfx950 those instructions
// do not all issue at one wave64 instruction per SIMD per 4 cycles:
// independent v_mul_f32 / v_add_f32 placed next to each other issue faster.
// These kernels time each instruction alone and both four-instruction
// candidate mixes (in dependency order and grouped by opcode) on every CU, so
// the benchmark can report the kernel against the ceiling its own
// instruction mix has on the GPU it runs on.
//
// Each thread runs kChains independent chains for kIters iterations and
// writes one float; nothing else is read or written.
#include <hip/hip_runtime.h>

#include <stdint.h>


namespace {

constexpr int kIters = 500;
constexpr int kChains = 16;
constexpr int kThreads = 1024;

// ONE: the kernel also holds 96 KiB of LDS, so that one workgroup (16
// waves, 4 per SIMD) runs per CU at a time -- the forward DP's occupancy,
// whose 64 codebook VGPRs per lane leave room for no second workgroup --
// instead of two (8 waves per SIMD).
constexpr int kOneWgLds = 96 * 1024 / 4;

template <int OP, bool ONE = false>
__global__ __launch_bounds__(kThreads) void probe_kernel(float* __restrict__ out, float b) {
    __shared__ float pad[ONE ? kOneWgLds : 1];
    float x[kChains];
    double d[kChains];
    uint32_t h[kChains];
#pragma unroll
    for (int c = 0; c < kChains; ++c) {
        h[c] = 0x3c003c00u + threadIdx.x + c;      // fp16 pairs near 1.0
        x[c] = 1.0f + 1e-3f * (float)(threadIdx.x + c);
        d[c] = (double)x[c];
    }
    for (int it = 0; it < kIters; ++it) {
        if constexpr (OP == 0) {
#pragma unroll
            for (int c = 0; c < kChains; ++c) asm volatile("v_mul_f32 %0, %0, %1" : "+v"(x[c]) : "v"(b));
        } else if constexpr (OP == 1) {
#pragma unroll
            for (int c = 0; c < kChains; ++c) asm volatile("v_add_f32 %0, %0, %1" : "+v"(x[c]) : "v"(b));
        } else if constexpr (OP == 2) {
#pragma unroll
            for (int c = 0; c < kChains; ++c)
                asm volatile("v_fma_f32 %0, %0, %1, %1" : "+v"(x[c]) : "v"(b));
        } else if constexpr (OP == 3) {
#pragma unroll
            for (int c = 0; c < kChains; ++c)
                asm volatile("v_fma_mix_f32 %0, %1, 1.0, %2 op_sel_hi:[1,0,0]"
                             : "=v"(x[c]) : "v"(h[c]), "v"(x[c]));
        } else if constexpr (OP == 4) {
#pragma unroll
            for (int c = 0; c < kChains; ++c)
                asm volatile("v_min_f64 %0, %0, %1" : "+v"(d[c]) : "v"((double)b));
        } else if constexpr (OP == 7) {               // fp32-code mix, dependency order
#pragma unroll
            for (int c = 0; c < kChains; ++c) {
                asm volatile("v_add_f32 %0, %1, %2" : "=v"(x[c]) : "v"(x[c]), "v"(b));
                asm volatile("v_mul_f32 %0, %0, %0" : "+v"(x[c]));
                asm volatile("v_add_f32 %0, %0, %1" : "+v"(x[c]) : "v"(b));
                asm volatile("v_min_f64 %0, %0, %1" : "+v"(d[c]) : "v"((double)b));
            }
        } else if constexpr (OP == 8) {               // fp32-code mix, grouped by 8
#pragma unroll
            for (int g0 = 0; g0 < kChains; g0 += 8) {
#pragma unroll
                for (int c = g0; c < g0 + 8; ++c)
                    asm volatile("v_add_f32 %0, %1, %2" : "=v"(x[c]) : "v"(x[c]), "v"(b));
#pragma unroll
                for (int c = g0; c < g0 + 8; ++c) asm volatile("v_mul_f32 %0, %0, %0" : "+v"(x[c]));
#pragma unroll
                for (int c = g0; c < g0 + 8; ++c)
                    asm volatile("v_add_f32 %0, %0, %1" : "+v"(x[c]) : "v"(b));
#pragma unroll
                for (int c = g0; c < g0 + 8; ++c)
                    asm volatile("v_min_f64 %0, %0, %1" : "+v"(d[c]) : "v"((double)b));
            }
        } else if constexpr (OP == 9) {               // v_min3_f32 alone
#pragma unroll
            for (int c = 0; c < kChains; ++c)
                asm volatile("v_min3_f32 %0, %0, %1, %1" : "+v"(x[c]) : "v"(b));
        } else if constexpr (OP == 10) {              // deferred-argmin mix, grouped by 8
#pragma unroll
            for (int g0 = 0; g0 < kChains; g0 += 8) {
#pragma unroll
                for (int c = g0; c < g0 + 8; ++c)
                    asm volatile("v_add_f32 %0, %1, %2" : "=v"(x[c]) : "v"(x[c]), "v"(b));
#pragma unroll
                for (int c = g0; c < g0 + 8; ++c) asm volatile("v_mul_f32 %0, %0, %0" : "+v"(x[c]));
#pragma unroll
                for (int c = g0; c < g0 + 8; ++c)
                    asm volatile("v_add_f32 %0, %0, %1" : "+v"(x[c]) : "v"(b));
                // the 8 costs' minimum by a v_min3_f32 tree (4 instructions)
                asm volatile("v_min3_f32 %0, %0, %1, %2"
                             : "+v"(x[g0]) : "v"(x[g0 + 1]), "v"(x[g0 + 2]));
                asm volatile("v_min3_f32 %0, %0, %1, %2"
                             : "+v"(x[g0 + 3]) : "v"(x[g0 + 4]), "v"(x[g0 + 5]));
                asm volatile("v_min3_f32 %0, %0, %1, %2"
                             : "+v"(x[g0 + 6]) : "v"(x[g0 + 7]), "v"(x[g0]));
                asm volatile("v_min_f32 %0, %0, %1" : "+v"(x[g0 + 6]) : "v"(x[g0 + 3]));
            }
        } else if constexpr (OP == 5) {               // candidate mix, dependency order
#pragma unroll
            for (int c = 0; c < kChains; ++c) {
                asm volatile("v_fma_mix_f32 %0, %1, 1.0, %2 op_sel_hi:[1,0,0]"
                             : "=v"(x[c]) : "v"(h[c]), "v"(b));
                asm volatile("v_mul_f32 %0, %0, %0" : "+v"(x[c]));
                asm volatile("v_add_f32 %0, %0, %1" : "+v"(x[c]) : "v"(b));
                asm volatile("v_min_f64 %0, %0, %1" : "+v"(d[c]) : "v"((double)b));
            }
        } else {                                     // candidate mix, grouped by 8
#pragma unroll
            for (int g0 = 0; g0 < kChains; g0 += 8) {
#pragma unroll
                for (int c = g0; c < g0 + 8; ++c)
                    asm volatile("v_fma_mix_f32 %0, %1, 1.0, %2 op_sel_hi:[1,0,0]"
                                 : "=v"(x[c]) : "v"(h[c]), "v"(b));
#pragma unroll
                for (int c = g0; c < g0 + 8; ++c) asm volatile("v_mul_f32 %0, %0, %0" : "+v"(x[c]));
#pragma unroll
                for (int c = g0; c < g0 + 8; ++c)
                    asm volatile("v_add_f32 %0, %0, %1" : "+v"(x[c]) : "v"(b));
#pragma unroll
                for (int c = g0; c < g0 + 8; ++c)
                    asm volatile("v_min_f64 %0, %0, %1" : "+v"(d[c]) : "v"((double)b));
            }
        }
    }
    float s = 0.0f;
#pragma unroll
    for (int c = 0; c < kChains; ++c) s += x[c] + (float)d[c];
    if constexpr (ONE) {
        // touch the LDS block so that it is allocated
        pad[threadIdx.x] = s;
        __syncthreads();
        s += pad[kThreads - 1 - threadIdx.x];
    }
    out[(size_t)blockIdx.x * kThreads + threadIdx.x] = s;
}

// VALU instructions per chain per iteration of each probe.
constexpr double kOpsPerChain[13] = {1, 1, 1, 1, 1, 4, 4, 4, 4, 1, 3.5, 4, 3.5};

template <int OP, bool ONE = false>
hipError_t launch(int nwg, float* out, hipStream_t s) {
    hipLaunchKernelGGL((probe_kernel<OP, ONE>), dim3(nwg), dim3(kThreads), 0, s, out,
                       1.0000001f);
    return hipGetLastError();
}

hipError_t launch_any(int which, int nwg, float* out, hipStream_t s) {
    switch (which) {
        case 0: return launch<0>(nwg, out, s);
        case 1: return launch<1>(nwg, out, s);
        case 2: return launch<2>(nwg, out, s);
        case 3: return launch<3>(nwg, out, s);
        case 4: return launch<4>(nwg, out, s);
        case 5: return launch<5>(nwg, out, s);
        case 6: return launch<6>(nwg, out, s);
        case 7: return launch<7>(nwg, out, s);
        case 8: return launch<8>(nwg, out, s);
        case 9: return launch<9>(nwg, out, s);
        case 10: return launch<10>(nwg, out, s);
        case 11: return launch<8, true>(nwg, out, s);
        default: return launch<10, true>(nwg, out, s);
    }
}

}  // namespace

// Times probe `which` (0 v_mul_f32, 1 v_add_f32, 2 v_fma_f32, 3 v_fma_mix_f32,
// 4 v_min_f64, 5/6 the candidate mix with a packed fp16 codebook in
// dependency order / grouped by opcode, 7/8 the mix with an fp32 codebook in
// dependency order / grouped by opcode, 9 v_min3_f32, 10 the deferred-argmin
// mix: add, mul, add per candidate and a v_min3_f32 tree over 8 -- 3.5
// instructions per candidate; 11 and 12 the mixes of 8 and 10 at one
// workgroup per CU, the forward DP's occupancy) on every CU of the current
// device and returns its VALU lane-instructions per second.  Status: 0 ok,
// 1 no device, 2 allocation failed, 4 HIP error, 8 unknown probe, 12 null
// output.
extern "C" __attribute__((visibility("default"))) int xtq_valu_probe(int which,
                                                                     double* lane_ops_per_s) {
    if (!lane_ops_per_s) return 12;
    if (which < 0 || which > 12) return 8;
    int dev = 0, ncu = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&ncu, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        ncu <= 0)
        return 1;
    const int nwg = 8 * ncu;
    float* out = nullptr;
    if (hipMalloc((void**)&out, (size_t)nwg * kThreads * sizeof(float)) != hipSuccess) return 2;
    hipStream_t s = nullptr;
    hipEvent_t e0 = nullptr, e1 = nullptr;
    int rc = 0;
    float best = 0.0f;
    if (hipStreamCreate(&s) != hipSuccess || hipEventCreate(&e0) != hipSuccess ||
        hipEventCreate(&e1) != hipSuccess) {
        rc = 1;
    } else if (launch_any(which, nwg, out, s) != hipSuccess ||
               hipStreamSynchronize(s) != hipSuccess) {     // warm-up
        rc = 4;
    } else {
        for (int r = 0; r < 3 && !rc; ++r) {
            float ms = 0.0f;
            if (hipEventRecord(e0, s) != hipSuccess || launch_any(which, nwg, out, s) != hipSuccess ||
                hipEventRecord(e1, s) != hipSuccess || hipEventSynchronize(e1) != hipSuccess ||
                hipEventElapsedTime(&ms, e0, e1) != hipSuccess)
                rc = 4;
            else if (r == 0 || ms < best)
                best = ms;
        }
    }
    if (!rc) {
        const double ops = (double)nwg * kThreads * kIters * kChains * kOpsPerChain[which];
        *lane_ops_per_s = ops / (best * 1e-3);
    }
    if (e0) (void)hipEventDestroy(e0);
    if (e1) (void)hipEventDestroy(e1);
    if (s) (void)hipStreamDestroy(s);
    (void)hipFree(out);
    return rc;
}
