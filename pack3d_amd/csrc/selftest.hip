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

}  // namespace
}  // namespace p3d

using namespace p3d;

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
