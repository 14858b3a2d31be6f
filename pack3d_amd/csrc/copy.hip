// Strided row copy: a [B, H, N, d] tensor from one view to another whose
// rows of d elements are contiguous and 16-byte aligned (the core's dense
// gradients into the head-interleaved projection layout [B, N, H, d] that the
// layer's to_q / to_kv outputs use, attention.py:64-67 of amilworks/Pack3D).
// One 16-byte piece per thread, in destination order: the heads of a token
// are adjacent in the projection layout, so a block writes whole token rows
// (heads * d elements) and reads d-element rows of the source.
#include "common.hpp"

namespace p3d {
namespace {

template <typename T>
__global__ __launch_bounds__(256) void k_copy_rows(const T* src, int64_t ssb, int64_t ssh, int64_t ssn, T* dst,
                                                   int64_t dsb, int64_t dsh, int64_t dsn, int H, int N, int ppr) {
    constexpr int EP = Piece<T>::N;
    const int b = blockIdx.y;
    const int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const int per_token = H * ppr;
    if (e >= (int64_t)N * per_token) return;
    const int n = (int)(e / per_token);
    const int r = (int)(e - (int64_t)n * per_token), h = r / ppr, p = r - h * ppr;
    *reinterpret_cast<uint4*>(dst + b * dsb + h * dsh + n * dsn + p * EP) =
        *reinterpret_cast<const uint4*>(src + b * ssb + h * ssh + n * ssn + p * EP);
}

}  // namespace
}  // namespace p3d

using namespace p3d;

extern "C" int p3d_copy_rows(p3d_view src, p3d_view dst, int64_t batch, int32_t heads, int64_t tokens,
                             int32_t head_dim, int32_t dtype, void* stream) {
    P3D_REQUIRE(src.data && dst.data, "null pointer argument");
    P3D_REQUIRE(dtype >= P3D_F32 && dtype <= P3D_BF16, "unknown dtype");
    const int es = dtype_size(dtype);
    P3D_REQUIRE(batch >= 1 && heads >= 1 && tokens >= 1 && batch < 65536 && tokens * heads * head_dim < (1LL << 40),
                "bad batch/head/token counts");
    P3D_REQUIRE(head_dim >= 1 && (head_dim * es) % 16 == 0, "rows must be whole 16-byte pieces");
    P3D_REQUIRE(view_ok(src, es) && view_ok(dst, es), "rows must be 16-byte aligned");
    const int ppr = head_dim * es / 16;
    P3D_REQUIRE(tokens < (1LL << 31), "too many tokens");
    const dim3 grid((unsigned)cdiv(tokens * heads * ppr, 256), (unsigned)batch);
    hipStream_t s = as_stream(stream);
    switch (dtype) {
        case P3D_F32:
            k_copy_rows<float><<<grid, 256, 0, s>>>((const float*)src.data, src.sb, src.sh, src.sn, (float*)dst.data,
                                                   dst.sb, dst.sh, dst.sn, heads, (int)tokens, ppr);
            break;
        case P3D_F16:
            k_copy_rows<_Float16><<<grid, 256, 0, s>>>((const _Float16*)src.data, src.sb, src.sh, src.sn,
                                                      (_Float16*)dst.data, dst.sb, dst.sh, dst.sn, heads, (int)tokens,
                                                      ppr);
            break;
        default:
            k_copy_rows<__bf16><<<grid, 256, 0, s>>>((const __bf16*)src.data, src.sb, src.sh, src.sn,
                                                    (__bf16*)dst.data, dst.sb, dst.sh, dst.sn, heads, (int)tokens, ppr);
            break;
    }
    return check_launch("p3d_copy_rows");
}
