// Issue-rate probe of the units the summary pathway uses (MI355X, gfx950):
// measurement scaffolding built into its own library, libpack3d_probe.so,
// and loaded only by `bench.py --probe-rates`; the product library
// (libpack3d_hip.so) does not contain it.  It has no counterpart in the
// reference.
#include "../csrc/attn_common.hpp"

namespace p3d {
namespace {

// Issue-rate probes (kind), every operand in registers:
//   0: 16 independent v_exp_f32 chains (x = exp2(x));
//   1: 16 independent v_fma_f32 chains;
//   2: 4 bf16 32x32x16 MFMAs on 4 accumulators;
//   3: kinds 0 and 2 in one iteration, independent of each other;
//   4: the summary sweep's steady state for head_dim 48: two column blocks,
//      each tile 3 score MFMAs, 16 exponentials, 8 converts and 4 product
//      MFMAs, software-pipelined as in the sweep (one block's exponentials
//      beside the other block's MFMAs); two tiles and blocks per iteration.
// Every wave writes its shader-clock cycles and its 100 MHz wall-clock ticks
// over the loop, so the host derives the clock of the run.
template <int KIND>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(KIND == 4 ? 2 : 4)))
void k_rate_probe(int iters, long long* cycles) {
    float x[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) x[i] = (threadIdx.x + i) * 1e-6f - 1.f;
    bf16x8 a, b;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        a[j] = (__bf16)(0.01f * j);
        b[j] = (__bf16)(0.02f * j);
    }
    f32x16 c[4];
#pragma unroll
    for (int k = 0; k < 4; ++k)
#pragma unroll
        for (int r = 0; r < 16; ++r) c[k][r] = 0.f;
    f32x16 s0, s1, negm;
#pragma unroll
    for (int r = 0; r < 16; ++r) s0[r] = s1[r] = negm[r] = -20.f;
    bf16x8 p0[2] = {a, b}, p1[2] = {b, a};
    const long long t0 = clock64(), w0 = wall_clock64();
    for (int it = 0; it < iters; ++it) {
        if constexpr (KIND == 0 || KIND == 3) {
#pragma unroll
            for (int i = 0; i < 16; ++i) x[i] = __builtin_amdgcn_exp2f(x[i]);
        }
        if constexpr (KIND == 1) {
#pragma unroll
            for (int i = 0; i < 16; ++i) x[i] = fmaf(x[i], 0.999f, -0.5f);
        }
        if constexpr (KIND == 2 || KIND == 3) {
#pragma unroll
            for (int k = 0; k < 4; ++k) c[k] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c[k], 0, 0, 0);
        }
        if constexpr (KIND == 4) {
#pragma unroll
            for (int ph = 0; ph < 2; ++ph) {
                // exponentials of one block's tile beside the other block's MFMAs
                const f32x16 sx = ph ? s1 : s0;
                f32x16 sq = negm;
                bf16x8* px = ph ? p1 : p0;
                const bf16x8* py = ph ? p0 : p1;
                float p[16];
#pragma unroll
                for (int j = 0; j < 7; ++j) {
                    if (j < 3) {
                        sq = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, sq, 0, 0, 0);
                    } else {
                        const int i = j - 3;
                        c[2 * (1 - ph) + (i & 1)] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(
                            a, py[i >> 1], c[2 * (1 - ph) + (i & 1)], 0, 0, 0);
                    }
#pragma unroll
                    for (int r = 16 * j / 7; r < 16 * (j + 1) / 7; ++r) {
                        p[r] = __builtin_amdgcn_exp2f(sx[r]);
                        if (r % 8 == 7) {
#pragma unroll
                            for (int e = 0; e < 8; ++e) px[r / 8][e] = (__bf16)p[r - 7 + e];
                        }
                    }
                    __builtin_amdgcn_sched_barrier(0);
                }
                if (ph) s0 = sq; else s1 = sq;
            }
        }
    }
    const long long t1 = clock64(), w1 = wall_clock64();
    float keep = 0.f;
#pragma unroll
    for (int i = 0; i < 16; ++i) keep += x[i];
#pragma unroll
    for (int k = 0; k < 4; ++k)
#pragma unroll
        for (int r = 0; r < 16; ++r) keep += c[k][r];
    if constexpr (KIND == 4) {
#pragma unroll
        for (int i = 0; i < 16; ++i) keep += s0[i] + s1[i];
#pragma unroll
        for (int e = 0; e < 8; ++e) keep += (float)p0[0][e] + (float)p1[1][e];
    }
    if ((threadIdx.x & 63) == 0) {
        const int w = blockIdx.x * 4 + (threadIdx.x >> 6);
        cycles[2 * w] = (t1 - t0) + (keep == 12345.f);
        cycles[2 * w + 1] = w1 - w0;
    }
}

}  // namespace
}  // namespace p3d

using namespace p3d;

extern "C" int p3d_probe_issue_rates(int32_t kind, int64_t iters, int32_t blocks, long long* cycles, void* stream) {
    P3D_REQUIRE(cycles && kind >= 0 && kind <= 4 && iters >= 1 && iters < (1LL << 31) && blocks >= 1,
                "bad probe arguments");
    hipStream_t s = as_stream(stream);
    const int n = (int)iters;
    switch (kind) {
        case 0: k_rate_probe<0><<<(unsigned)blocks, 256, 0, s>>>(n, cycles); break;
        case 1: k_rate_probe<1><<<(unsigned)blocks, 256, 0, s>>>(n, cycles); break;
        case 2: k_rate_probe<2><<<(unsigned)blocks, 256, 0, s>>>(n, cycles); break;
        case 3: k_rate_probe<3><<<(unsigned)blocks, 256, 0, s>>>(n, cycles); break;
        default: k_rate_probe<4><<<(unsigned)blocks, 256, 0, s>>>(n, cycles); break;
    }
    return check_launch("p3d_probe_issue_rates");
}
