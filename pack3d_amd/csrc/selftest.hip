// Self-test entry points: the MFMA fragment / accumulator layout every
// attention kernel relies on, and the ABI struct sizes.
#include "attn_common.hpp"

namespace p3d {
namespace {

// One wave: A [32 x KS] and B [KS x 32] row-major in T; D = A B row-major fp32.
template <typename T>
__global__ void k_mfma_probe(const T* A, const T* B, float* Dout) {
    typedef Mma<T> M;
    const int lane = threadIdx.x, g = lane >> 5, i = lane & 31;
    typename M::Frag a, b;
    if constexpr (M::E == 1) {
        a = A[i * M::KS + g];
        b = B[g * 32 + i];
    } else {
#pragma unroll
        for (int j = 0; j < M::E; ++j) {
            a[j] = A[i * M::KS + M::E * g + j];
            b[j] = B[(M::E * g + j) * 32 + i];
        }
    }
    f32x16 acc;
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[r] = 0.f;
    acc = M::mfma(a, b, acc);
#pragma unroll
    for (int r = 0; r < 16; ++r) Dout[acc_row(r, g) * 32 + i] = acc[r];
}

// Issue-rate probes (kind): 0 = v_exp_f32, 1 = v_fma_f32, 2 = 32x32x16 bf16
// MFMA, 3 = per iteration 4 MFMAs and 16 exponentials, independent of each
// other (the mix of the summary pathway).  Every wave writes the shader
// clock cycles of its loop; 16 (or 4) independent chains keep the units fed.
template <int KIND>
__global__ __launch_bounds__(256) void k_rate_probe(int iters, long long* cycles) {
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
    const long long t0 = clock64();
    for (int it = 0; it < iters; ++it) {
        if constexpr (KIND == 0 || KIND == 3) {
#pragma unroll
            for (int i = 0; i < 16; ++i) x[i] = __builtin_amdgcn_exp2f(x[i]) - 1.5f;
        }
        if constexpr (KIND == 1) {
#pragma unroll
            for (int i = 0; i < 16; ++i) x[i] = fmaf(x[i], 0.999f, -0.5f);
        }
        if constexpr (KIND == 2 || KIND == 3) {
#pragma unroll
            for (int k = 0; k < 4; ++k) c[k] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c[k], 0, 0, 0);
        }
    }
    const long long t1 = clock64();
    float keep = 0.f;
#pragma unroll
    for (int i = 0; i < 16; ++i) keep += x[i];
#pragma unroll
    for (int k = 0; k < 4; ++k)
#pragma unroll
        for (int r = 0; r < 16; ++r) keep += c[k][r];
    if ((threadIdx.x & 63) == 0) cycles[blockIdx.x * 4 + (threadIdx.x >> 6)] = (t1 - t0) + (keep == 12345.f);
}

}  // namespace
}  // namespace p3d

using namespace p3d;

extern "C" int p3d_probe_issue_rates(int32_t kind, int64_t iters, int32_t blocks, long long* cycles, void* stream) {
    P3D_REQUIRE(cycles && kind >= 0 && kind <= 3 && iters >= 1 && iters < (1LL << 31) && blocks >= 1,
                "bad probe arguments");
    hipStream_t s = as_stream(stream);
    const int n = (int)iters;
    switch (kind) {
        case 0: k_rate_probe<0><<<(unsigned)blocks, 256, 0, s>>>(n, cycles); break;
        case 1: k_rate_probe<1><<<(unsigned)blocks, 256, 0, s>>>(n, cycles); break;
        case 2: k_rate_probe<2><<<(unsigned)blocks, 256, 0, s>>>(n, cycles); break;
        default: k_rate_probe<3><<<(unsigned)blocks, 256, 0, s>>>(n, cycles); break;
    }
    return check_launch("p3d_probe_issue_rates");
}

extern "C" int p3d_selftest_mfma(int32_t dtype, const void* a, const void* b, float* d, void* stream) {
    P3D_REQUIRE(a && b && d, "null argument");
    hipStream_t s = as_stream(stream);
    switch (dtype) {
        case P3D_F32: k_mfma_probe<float><<<1, 64, 0, s>>>((const float*)a, (const float*)b, d); break;
        case P3D_F16: k_mfma_probe<_Float16><<<1, 64, 0, s>>>((const _Float16*)a, (const _Float16*)b, d); break;
        case P3D_BF16: k_mfma_probe<__bf16><<<1, 64, 0, s>>>((const __bf16*)a, (const __bf16*)b, d); break;
        default: return fail(P3D_EINVAL, "unknown dtype");
    }
    return check_launch("p3d_selftest_mfma");
}

extern "C" int p3d_struct_sizes(int64_t* out) {
    P3D_REQUIRE(out, "null argument");
    out[0] = sizeof(p3d_view);
    out[1] = sizeof(p3d_rope);
    out[2] = sizeof(p3d_pool_args);
    out[3] = sizeof(p3d_attn_args);
    out[4] = sizeof(p3d_bwd_args);
    out[5] = sizeof(p3d_project_args);
    return P3D_OK;
}
