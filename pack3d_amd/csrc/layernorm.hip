// LayerNorm over the channel dimension of [rows, dim] tokens: the first op
// of the PACK3D layer (attention.py:64 of amilworks/Pack3D, nn.LayerNorm with
// elementwise affine).  Statistics in fp32 over the row (two passes in
// registers: mean, then the biased variance of the centred values), output
// (x - mean) / sqrt(var + eps) * w + b rounded to the storage type.
//
// LPR lanes share a row (8, or 16 for rows of more than 64 pieces: fp32
// rows of 384 or 512 channels); lane j of the group holds the 16-byte pieces
// j, j + LPR, ... of the row, so a wave covers 64 / LPR rows and every load
// and store is a full 16 bytes.  The affine weight and bias are staged in LDS
// as fp32 once per block; the row sums reduce over the 8-lane groups through
// DPP, then across groups by lane shuffles.
#include "common.hpp"

namespace p3d {
namespace {

constexpr int kLanesPerRow = 8;
constexpr int kMaxPiecesPerLane = 8;
constexpr int kMaxDim = 512;
constexpr int kMaxPieces = 128;  // fp32 rows of 512 channels

// Sum over the 8-lane group: lanes l ^ 1, l ^ 2 (quad_perm), then l ^ 7
// within 8 (row_half_mirror).
__device__ __forceinline__ float group8_sum(float x) {
    x += dpp_move<0xB1>(x);
    x += dpp_move<0x4E>(x);
    return x + dpp_move<0x141>(x);
}

// Sum over the LPR lanes of a row (LPR 8, 16 or 32, aligned groups).
template <int LPR>
__device__ __forceinline__ float lanes_sum(float x) {
    x = group8_sum(x);
    if constexpr (LPR >= 16) x += __shfl_xor(x, 8);
    if constexpr (LPR >= 32) x += __shfl_xor(x, 16);
    return x;
}

// Lanes per row of the forward kernels: 8, or 16 past 64 pieces.
__host__ __device__ constexpr int fwd_lanes(int pieces) { return pieces > 64 ? 16 : 8; }

template <typename T, int LPR>
__global__ __launch_bounds__(256) void k_layer_norm(const T* x, const void* w, const void* b, int param_dtype,
                                                    T* y, int64_t rows, int dim, float eps) {
    constexpr int EP = Piece<T>::N;
    constexpr int kLanesPerRow = LPR;
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
    const float mean = lanes_sum<LPR>(sum) / (float)dim;
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
    const float rstd = 1.f / sqrtf(lanes_sum<LPR>(sq) / (float)dim + eps);
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

// ------------------------------------------------------------ training
// The same LayerNorm with separate input and output types (fp32 tokens in,
// the 16-bit compute type out under autocast) that also writes each row's
// mean and 1/std for the backward.  A lane holds the 16-byte input pieces
// j, j + 8, ... of its row (EP input elements each) and the same channels of
// every other per-row tensor.
template <typename T, int N>
struct Vec {
    typedef T type __attribute__((ext_vector_type(N)));
};

template <typename T, int N>
__device__ __forceinline__ void load_n(const T* p, float (&out)[N]) {
    const typename Vec<T, N>::type v = *reinterpret_cast<const typename Vec<T, N>::type*>(p);
#pragma unroll
    for (int e = 0; e < N; ++e) out[e] = to_f32(v[e]);
}

template <typename T, int N>
__device__ __forceinline__ void store_n(T* p, const float (&in)[N]) {
    typename Vec<T, N>::type v;
#pragma unroll
    for (int e = 0; e < N; ++e) v[e] = from_f32<T>(in[e]);
    *reinterpret_cast<typename Vec<T, N>::type*>(p) = v;
}

template <typename TI, typename TO, int LPR>
__global__ __launch_bounds__(256) void k_layer_norm_train(const TI* x, const void* w, const void* b, int param_dtype,
                                                          TO* y, TO* x_copy, float* mean_out, float* rstd_out,
                                                          int64_t rows, int dim, float eps) {
    constexpr int EP = Piece<TI>::N;
    constexpr int kLanesPerRow = LPR;
    __shared__ __align__(16) float lw[kMaxDim], lb[kMaxDim];
    for (int c = threadIdx.x; c < dim; c += blockDim.x) {
        lw[c] = load_any(w, c, param_dtype);
        lb[c] = load_any(b, c, param_dtype);
    }
    const int sub = threadIdx.x % kLanesPerRow;
    const int pieces = dim / EP;
    const int64_t row = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) / kLanesPerRow;
    const bool live = row < rows;
    const TI* xr = x + (live ? row : 0) * dim;
    float v[kMaxPiecesPerLane][EP];
    float sum = 0.f;
#pragma unroll
    for (int i = 0; i < kMaxPiecesPerLane; ++i) {
        const int p = sub + kLanesPerRow * i;
        if (p < pieces) {
            load_n<TI, EP>(xr + p * EP, v[i]);
#pragma unroll
            for (int e = 0; e < EP; ++e) sum += v[i][e];
        }
    }
    const float mean = lanes_sum<LPR>(sum) / (float)dim;
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
    const float rstd = 1.f / sqrtf(lanes_sum<LPR>(sq) / (float)dim + eps);
    __syncthreads();
    if (!live) return;
    if (sub == 0) {
        mean_out[row] = mean;
        rstd_out[row] = rstd;
    }
#pragma unroll
    for (int i = 0; i < kMaxPiecesPerLane; ++i) {
        const int p = sub + kLanesPerRow * i;
        if (p < pieces) {
            float o[EP];
#pragma unroll
            for (int e = 0; e < EP; ++e) {
                const int c = p * EP + e;
                o[e] = (v[i][e] - mean) * rstd * lw[c] + lb[c];
            }
            store_n<TO, EP>(y + row * dim + p * EP, o);
            if (x_copy) store_n<TO, EP>(x_copy + row * dim + p * EP, v[i]);
        }
    }
}

// LayerNorm backward (torch's formula): with xhat = (x - mean) rstd and
// g = dy * w, dx = rstd (g - mean(g) - xhat mean(g xhat)) per row, and the
// affine gradients dw = sum_rows dy xhat, db = sum_rows dy.  Blocks stride
// over the rows; each writes its fp32 partial sums of dw and db to
// part[block][0 / 1][dim], summed by the caller.  LPR lanes share a row (8,
// or 32 for rows of more than 32 pieces, whose per-lane arrays would
// otherwise hold a wave to one per SIMD); PPL: pieces per lane
// (ceil(dim / EP / LPR)), which sizes the per-lane arrays.
template <typename TD, typename TI, typename TO, int PPL, int LPR>
__global__ __launch_bounds__(256) void k_layer_norm_bwd(const TD* dy, const TO* dres, const TI* x, const void* w,
                                                        int param_dtype, const float* mean_in, const float* rstd_in,
                                                        TO* dx, float* part, int64_t rows, int dim, int parts) {
    constexpr int EP = Piece<TI>::N;
    constexpr int kLanesPerRow = LPR;
    constexpr int GROUPS = 256 / kLanesPerRow;
    __shared__ __align__(16) float lw[kMaxDim];
    __shared__ float red[2][kMaxDim];
    for (int c = threadIdx.x; c < dim; c += blockDim.x) {
        lw[c] = load_any(w, c, param_dtype);
        red[0][c] = red[1][c] = 0.f;
    }
    __syncthreads();
    const int sub = threadIdx.x % kLanesPerRow, grp = threadIdx.x / kLanesPerRow;
    const int pieces = dim / EP;
    float pw[PPL][EP], pb[PPL][EP];
#pragma unroll
    for (int i = 0; i < PPL; ++i)
#pragma unroll
        for (int e = 0; e < EP; ++e) pw[i][e] = pb[i][e] = 0.f;
    const int64_t step = (int64_t)gridDim.x * GROUPS;
    for (int64_t row = (int64_t)blockIdx.x * GROUPS + grp; row < rows; row += step) {
        const float mean = mean_in[row], rstd = rstd_in[row];
        float xh[PPL][EP], g[PPL][EP], rr[PPL][EP];
        float sg = 0.f, sgx = 0.f;
#pragma unroll
        for (int i = 0; i < PPL; ++i) {
            const int p = sub + kLanesPerRow * i;
            if (p < pieces) {
                float xv[EP], dv[EP];
                load_n<TI, EP>(x + row * dim + p * EP, xv);
                load_n<TD, EP>(dy + row * dim + p * EP, dv);
                // The residual gradient is loaded with x and dy, so a row costs
                // one round trip to memory rather than two.
                if (dres) load_n<TO, EP>(dres + row * dim + p * EP, rr[i]);
#pragma unroll
                for (int e = 0; e < EP; ++e) {
                    xh[i][e] = (xv[e] - mean) * rstd;
                    g[i][e] = dv[e] * lw[p * EP + e];
                    sg += g[i][e];
                    sgx += g[i][e] * xh[i][e];
                    pw[i][e] += dv[e] * xh[i][e];
                    pb[i][e] += dv[e];
                }
            }
        }
        const float mg = lanes_sum<LPR>(sg) / (float)dim, mgx = lanes_sum<LPR>(sgx) / (float)dim;
#pragma unroll
        for (int i = 0; i < PPL; ++i) {
            const int p = sub + kLanesPerRow * i;
            if (p < pieces) {
                float o[EP];
#pragma unroll
                for (int e = 0; e < EP; ++e) o[e] = rstd * (g[i][e] - mg - xh[i][e] * mgx);
                if (dres) {
#pragma unroll
                    for (int e = 0; e < EP; ++e) o[e] += rr[i][e];
                }
                store_n<TO, EP>(dx + row * dim + p * EP, o);
            }
        }
    }
    // Partial affine gradients of this block: the row groups in turn (fixed order).
    for (int k = 0; k < GROUPS; ++k) {
        if (grp == k)
#pragma unroll
            for (int i = 0; i < PPL; ++i) {
                const int p = sub + kLanesPerRow * i;
                if (p < pieces)
#pragma unroll
                    for (int e = 0; e < EP; ++e) {
                        red[0][p * EP + e] += pw[i][e];
                        red[1][p * EP + e] += pb[i][e];
                    }
            }
        __syncthreads();
    }
    for (int c = threadIdx.x; c < dim; c += blockDim.x) {
        part[((int64_t)blockIdx.x * 2 + 0) * dim + c] = red[0][c];
        part[((int64_t)blockIdx.x * 2 + 1) * dim + c] = red[1][c];
    }
    // Partial rows past the launched grid hold zeros, so the caller's sum
    // over all `parts` rows is the same whatever grid ran.
    for (int q = blockIdx.x + gridDim.x; q < parts; q += gridDim.x)
        for (int c = threadIdx.x; c < 2 * dim; c += blockDim.x) part[(int64_t)q * 2 * dim + c] = 0.f;
}

template <typename TI, typename TO>
int launch_ln_train(const void* x, const void* w, const void* b, int pdt, void* y, void* xc, float* mean, float* rstd,
                    int64_t rows, int dim, float eps, hipStream_t s) {
    if (fwd_lanes(dim / Piece<TI>::N) == 16) {
        const unsigned blocks = (unsigned)cdiv(rows * 16, 256);
        k_layer_norm_train<TI, TO, 16><<<blocks, 256, 0, s>>>((const TI*)x, w, b, pdt, (TO*)y, (TO*)xc, mean, rstd,
                                                              rows, dim, eps);
    } else {
        const unsigned blocks = (unsigned)cdiv(rows * 8, 256);
        k_layer_norm_train<TI, TO, 8><<<blocks, 256, 0, s>>>((const TI*)x, w, b, pdt, (TO*)y, (TO*)xc, mean, rstd,
                                                             rows, dim, eps);
    }
    return check_launch("p3d_layer_norm_train");
}

template <typename TI>
int dispatch_ln_train(const void* x, const void* w, const void* b, int pdt, void* y, void* xc, float* mean,
                      float* rstd, int64_t rows, int dim, int y_dtype, float eps, hipStream_t s) {
    switch (y_dtype) {
        case P3D_F32: return launch_ln_train<TI, float>(x, w, b, pdt, y, xc, mean, rstd, rows, dim, eps, s);
        case P3D_F16: return launch_ln_train<TI, _Float16>(x, w, b, pdt, y, xc, mean, rstd, rows, dim, eps, s);
        default: return launch_ln_train<TI, __bf16>(x, w, b, pdt, y, xc, mean, rstd, rows, dim, eps, s);
    }
}

template <typename TD, typename TI, typename TO>
int launch_ln_bwd(const void* dy, const void* dres, const void* x, const void* w, int pdt, const float* mean,
                  const float* rstd, void* dx, float* part, int64_t rows, int dim, int parts, hipStream_t s) {
    const int pieces = dim / Piece<TI>::N;
    const int ppl = (int)cdiv(pieces, kLanesPerRow);
    // At most one round of resident blocks: the blocks stride over the rows,
    // and a partly filled second round would leave most of the GPU idle.
    int dev = 0, cus = 0;
    (void)hipGetDevice(&dev);
    (void)hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
    auto grid_for = [&](const void* kernel) {
        int per_cu = 0;
        (void)hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kernel, 256, 0);
        const int64_t resident = (int64_t)(cus > 0 ? cus : 1) * (per_cu > 0 ? per_cu : 1);
        return (unsigned)(parts < resident ? parts : resident);
    };
    if (ppl > 4) {
        // 32 lanes per row: up to 4 pieces per lane (128 pieces).
        switch ((int)cdiv(pieces, 32)) {
#define CASE(P)                                                                                                  \
    case P:                                                                                                      \
        k_layer_norm_bwd<TD, TI, TO, P, 32>                                                                      \
            <<<grid_for(reinterpret_cast<const void*>(k_layer_norm_bwd<TD, TI, TO, P, 32>)), 256, 0, s>>>(      \
                (const TD*)dy, (const TO*)dres, (const TI*)x, w, pdt, mean, rstd, (TO*)dx, part, rows, dim,      \
                parts);                                                                                          \
        break;
            CASE(2) CASE(3) CASE(4)
#undef CASE
            default: return fail(P3D_EUNSUPPORTED, "dim too large for the LayerNorm backward");
        }
        return check_launch("p3d_layer_norm_bwd");
    }
    switch (ppl) {
#define CASE(P)                                                                                                  \
    case P:                                                                                                      \
        k_layer_norm_bwd<TD, TI, TO, P, 8>                                                                       \
            <<<grid_for(reinterpret_cast<const void*>(k_layer_norm_bwd<TD, TI, TO, P, 8>)), 256, 0, s>>>(       \
                (const TD*)dy, (const TO*)dres, (const TI*)x, w, pdt, mean, rstd, (TO*)dx, part, rows, dim,      \
                parts);                                                                                          \
        break;
        CASE(1) CASE(2) CASE(3) CASE(4)
#undef CASE
        default: return fail(P3D_EUNSUPPORTED, "dim too large for the LayerNorm backward");
    }
    return check_launch("p3d_layer_norm_bwd");
}

// Type dispatch of the backward: dy and dx in {the 16-bit type of the
// forward output, fp32}, x in {fp32, fp16, bf16}.
template <typename TD, typename TI>
int dispatch_ln_bwd_out(const void* dy, const void* dres, const void* x, const void* w, int pdt, const float* mean,
                        const float* rstd, void* dx, float* part, int64_t rows, int dim, int parts, int dx_dtype,
                        hipStream_t s) {
    switch (dx_dtype) {
        case P3D_F32:
            return launch_ln_bwd<TD, TI, float>(dy, dres, x, w, pdt, mean, rstd, dx, part, rows, dim, parts, s);
        case P3D_F16:
            return launch_ln_bwd<TD, TI, _Float16>(dy, dres, x, w, pdt, mean, rstd, dx, part, rows, dim, parts, s);
        default:
            return launch_ln_bwd<TD, TI, __bf16>(dy, dres, x, w, pdt, mean, rstd, dx, part, rows, dim, parts, s);
    }
}

template <typename TD>
int dispatch_ln_bwd_x(const void* dy, const void* dres, const void* x, const void* w, int pdt, const float* mean,
                      const float* rstd, void* dx, float* part, int64_t rows, int dim, int parts, int x_dtype,
                      int dx_dtype, hipStream_t s) {
    switch (x_dtype) {
        case P3D_F32:
            return dispatch_ln_bwd_out<TD, float>(dy, dres, x, w, pdt, mean, rstd, dx, part, rows, dim, parts,
                                                  dx_dtype, s);
        case P3D_F16:
            return dispatch_ln_bwd_out<TD, _Float16>(dy, dres, x, w, pdt, mean, rstd, dx, part, rows, dim, parts,
                                                     dx_dtype, s);
        default:
            return dispatch_ln_bwd_out<TD, __bf16>(dy, dres, x, w, pdt, mean, rstd, dx, part, rows, dim, parts,
                                                   dx_dtype, s);
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
    P3D_REQUIRE(dim >= ep && dim % ep == 0 && dim / ep <= kMaxPieces && dim <= kMaxDim,
                "dim must be a multiple of the 16-byte piece and at most 512 channels");
    P3D_REQUIRE(rows >= 1, "need at least one row");
    P3D_REQUIRE(((uintptr_t)x % 16) == 0 && ((uintptr_t)y % 16) == 0, "x and y must be 16-byte aligned");
    hipStream_t s = as_stream(stream);
    switch (dtype) {
        case P3D_F32:
            if (fwd_lanes(dim / ep) == 16)
                k_layer_norm<float, 16><<<(unsigned)cdiv(rows * 16, 256), 256, 0, s>>>(
                    (const float*)x, weight, bias, param_dtype, (float*)y, rows, dim, eps);
            else
                k_layer_norm<float, 8><<<(unsigned)cdiv(rows * 8, 256), 256, 0, s>>>(
                    (const float*)x, weight, bias, param_dtype, (float*)y, rows, dim, eps);
            break;
        case P3D_F16:
            k_layer_norm<_Float16, 8><<<(unsigned)cdiv(rows * 8, 256), 256, 0, s>>>(
                (const _Float16*)x, weight, bias, param_dtype, (_Float16*)y, rows, dim, eps);
            break;
        default:
            k_layer_norm<__bf16, 8><<<(unsigned)cdiv(rows * 8, 256), 256, 0, s>>>(
                (const __bf16*)x, weight, bias, param_dtype, (__bf16*)y, rows, dim, eps);
            break;
    }
    return check_launch("p3d_layer_norm");
}

extern "C" int p3d_layer_norm_train(const void* x, const void* weight, const void* bias, int32_t param_dtype, void* y,
                                    void* x_copy, float* mean, float* rstd, int64_t rows, int32_t dim,
                                    int32_t x_dtype, int32_t y_dtype, float eps, void* stream) {
    P3D_REQUIRE(x && weight && bias && y && mean && rstd, "null pointer argument");
    P3D_REQUIRE(x_dtype >= P3D_F32 && x_dtype <= P3D_BF16 && y_dtype >= P3D_F32 && y_dtype <= P3D_BF16 &&
                    param_dtype >= P3D_F32 && param_dtype <= P3D_BF16,
                "unknown dtype");
    const int ep = 16 / dtype_size(x_dtype);
    P3D_REQUIRE(dim >= ep && dim % ep == 0 && dim / ep <= kMaxPieces && dim <= kMaxDim,
                "dim must be a multiple of the 16-byte piece of x and at most 512 channels");
    P3D_REQUIRE(rows >= 1, "need at least one row");
    P3D_REQUIRE(aligned16(x) && aligned16(y), "x and y must be 16-byte aligned");
    P3D_REQUIRE(!x_copy || aligned16(x_copy), "x_copy must be 16-byte aligned");
    hipStream_t s = as_stream(stream);
    switch (x_dtype) {
        case P3D_F32: return dispatch_ln_train<float>(x, weight, bias, param_dtype, y, x_copy, mean, rstd, rows, dim,
                                                      y_dtype, eps, s);
        case P3D_F16: return dispatch_ln_train<_Float16>(x, weight, bias, param_dtype, y, x_copy, mean, rstd, rows,
                                                         dim, y_dtype, eps, s);
        default: return dispatch_ln_train<__bf16>(x, weight, bias, param_dtype, y, x_copy, mean, rstd, rows, dim,
                                                  y_dtype, eps, s);
    }
}

extern "C" int p3d_layer_norm_bwd(const void* dy, const void* dres, const void* x, const void* weight, int32_t param_dtype,
                                  const float* mean, const float* rstd, void* dx, float* partial, int64_t rows,
                                  int32_t dim, int32_t dy_dtype, int32_t x_dtype, int32_t dx_dtype, int32_t parts,
                                  void* stream) {
    P3D_REQUIRE(dy && x && weight && mean && rstd && dx && partial, "null pointer argument");
    P3D_REQUIRE(dy_dtype >= P3D_F32 && dy_dtype <= P3D_BF16 && x_dtype >= P3D_F32 && x_dtype <= P3D_BF16 &&
                    dx_dtype >= P3D_F32 && dx_dtype <= P3D_BF16 && param_dtype >= P3D_F32 && param_dtype <= P3D_BF16,
                "unknown dtype");
    const int ep = 16 / dtype_size(x_dtype);
    P3D_REQUIRE(dim >= ep && dim % ep == 0 && dim / ep <= kMaxPieces && dim <= kMaxDim,
                "dim must be a multiple of the 16-byte piece of x and at most 512 channels");
    P3D_REQUIRE(rows >= 1 && parts >= 1 && parts < 65536, "need at least one row and one part");
    P3D_REQUIRE(aligned16(dy) && aligned16(x) && aligned16(dx), "dy, x and dx must be 16-byte aligned");
    P3D_REQUIRE(!dres || aligned16(dres), "dres must be 16-byte aligned");
    hipStream_t s = as_stream(stream);
    switch (dy_dtype) {
        case P3D_F32: return dispatch_ln_bwd_x<float>(dy, dres, x, weight, param_dtype, mean, rstd, dx, partial, rows,
                                                      dim, parts, x_dtype, dx_dtype, s);
        case P3D_F16: return dispatch_ln_bwd_x<_Float16>(dy, dres, x, weight, param_dtype, mean, rstd, dx, partial,
                                                         rows, dim, parts, x_dtype, dx_dtype, s);
        default: return dispatch_ln_bwd_x<__bf16>(dy, dres, x, weight, param_dtype, mean, rstd, dx, partial, rows,
                                                  dim, parts, x_dtype, dx_dtype, s);
    }
}
