// LayerNorm over the channel dimension of [rows, dim] tokens: the first op
// of the PACK3D layer (attention.py:64 of amilworks/Pack3D, nn.LayerNorm with
// elementwise affine).  Statistics in fp32 over the row (two passes in
// registers: mean, then the biased variance of the centred values), output
// (x - mean) / sqrt(var + eps) * w + b rounded to the storage type.
//
// Eight lanes share a row; lane j of the group holds the 16-byte pieces j,
// j + 8, ... of the row, so a wave covers 8 rows and every load and store is
// a full 16 bytes.  The affine weight and bias are staged in LDS as fp32 once
// per block; the row sums reduce over the 8 lanes through DPP.
#include "common.hpp"

namespace p3d {
namespace {

constexpr int kLanesPerRow = 8;
constexpr int kMaxPiecesPerLane = 8;
constexpr int kMaxDim = 512;

// Sum over the 8-lane group: lanes l ^ 1, l ^ 2 (quad_perm), then l ^ 7
// within 8 (row_half_mirror).
__device__ __forceinline__ float group8_sum(float x) {
    x += dpp_move<0xB1>(x);
    x += dpp_move<0x4E>(x);
    return x + dpp_move<0x141>(x);
}

template <typename T>
__global__ __launch_bounds__(256) void k_layer_norm(const T* x, const void* w, const void* b, int param_dtype,
                                                    T* y, int64_t rows, int dim, float eps) {
    constexpr int EP = Piece<T>::N;
    __shared__ __align__(16) float lw[kMaxDim], lb[kMaxDim];
    for (int c = threadIdx.x; c < dim; c += blockDim.x) {
        lw[c] = load_any(w, c, param_dtype);
        lb[c] = load_any(b, c, param_dtype);
    }
    const int lane = threadIdx.x & 63;
    const int sub = lane % kLanesPerRow;
    const int pieces = dim / EP;
    const int64_t row = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) / kLanesPerRow;
    const bool live = row < rows;
    const T* xr = x + (live ? row : 0) * dim;
    float v[kMaxPiecesPerLane][EP];
    float sum = 0.f;
#pragma unroll
    for (int i = 0; i < kMaxPiecesPerLane; ++i) {
        const int p = sub + kLanesPerRow * i;
        if (p < pieces) {
            load_piece<T>(xr + p * EP, v[i]);
#pragma unroll
            for (int e = 0; e < EP; ++e) sum += v[i][e];
        }
    }
    const float mean = group8_sum(sum) / (float)dim;
    float sq = 0.f;
#pragma unroll
    for (int i = 0; i < kMaxPiecesPerLane; ++i) {
        const int p = sub + kLanesPerRow * i;
        if (p < pieces)
#pragma unroll
            for (int e = 0; e < EP; ++e) {
                const float c = v[i][e] - mean;
                sq += c * c;
            }
    }
    const float rstd = 1.f / sqrtf(group8_sum(sq) / (float)dim + eps);
    __syncthreads();
    if (!live) return;
#pragma unroll
    for (int i = 0; i < kMaxPiecesPerLane; ++i) {
        const int p = sub + kLanesPerRow * i;
        if (p < pieces) {
            uint4 raw;
            T* o = reinterpret_cast<T*>(&raw);
#pragma unroll
            for (int e = 0; e < EP; ++e) {
                const int c = p * EP + e;
                o[e] = from_f32<T>((v[i][e] - mean) * rstd * lw[c] + lb[c]);
            }
            *reinterpret_cast<uint4*>(y + row * dim + p * EP) = raw;
        }
    }
}

}  // namespace
}  // namespace p3d

using namespace p3d;

extern "C" int p3d_layer_norm(const void* x, const void* weight, const void* bias, int32_t param_dtype, void* y,
                              int64_t rows, int32_t dim, int32_t dtype, float eps, void* stream) {
    P3D_REQUIRE(x && weight && bias && y, "null pointer argument");
    P3D_REQUIRE(dtype >= P3D_F32 && dtype <= P3D_BF16 && param_dtype >= P3D_F32 && param_dtype <= P3D_BF16,
                "unknown dtype");
    const int ep = 16 / dtype_size(dtype);
    P3D_REQUIRE(dim >= ep && dim % ep == 0 && dim / ep <= kLanesPerRow * kMaxPiecesPerLane && dim <= kMaxDim,
                "dim must be a multiple of the 16-byte piece, at most 64 pieces and 512 channels");
    P3D_REQUIRE(rows >= 1, "need at least one row");
    P3D_REQUIRE(((uintptr_t)x % 16) == 0 && ((uintptr_t)y % 16) == 0, "x and y must be 16-byte aligned");
    const int64_t threads = rows * kLanesPerRow;
    const unsigned blocks = (unsigned)cdiv(threads, 256);
    hipStream_t s = as_stream(stream);
    switch (dtype) {
        case P3D_F32:
            k_layer_norm<float><<<blocks, 256, 0, s>>>((const float*)x, weight, bias, param_dtype, (float*)y, rows,
                                                       dim, eps);
            break;
        case P3D_F16:
            k_layer_norm<_Float16><<<blocks, 256, 0, s>>>((const _Float16*)x, weight, bias, param_dtype,
                                                          (_Float16*)y, rows, dim, eps);
            break;
        default:
            k_layer_norm<__bf16><<<blocks, 256, 0, s>>>((const __bf16*)x, weight, bias, param_dtype, (__bf16*)y,
                                                        rows, dim, eps);
            break;
    }
    return check_launch("p3d_layer_norm");
}
