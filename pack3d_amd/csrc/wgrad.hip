// Weight gradients of the PACK3D layer's linear maps (to_q, to_kv, gate and
// to_out of attention.py:64-67,85,89 of amilworks/Pack3D): for y = x W^T,
// dW[o][i] = sum over tokens n of dy[n][o] x[n][i], accumulated in fp32.
// The contraction runs over all tokens (262,144 at 64^3) while W is small
// (at most a few hundred rows), so the tokens are split across workgroups
// and each writes an fp32 partial; a second kernel sums the partials in a
// fixed order (deterministic).
//
// A workgroup owns 256 output rows (8 waves x 32) and a token range, taken
// TOK tokens per stage.  A stage of dy [TOK tokens x 256 rows] and of x [TOK
// tokens x I] is loaded with 16-byte row pieces (the next stage in flight
// while the current one is multiplied) and stored row-major in LDS.  The
// pass is bound by the bytes in flight per CU: from I = 128 on, one
// workgroup fits per CU and its stages take 64 tokens (32-token stages ran
// 15% slower at I = 192); narrower x keeps 32-token stages and several
// workgroups per CU.  The MFMA operands need 8 consecutive tokens of one column per lane; they come
// out of the row-major tiles through ds_read_b64_tr_b16, two 8-byte
// transposed reads per fragment, so nothing is transposed on the way in.
// Each wave then multiplies its 32 x 16-token A fragment with the I / 32
// shared x fragments: D = dy^T x, 32 rows by I columns per wave.
#include "common.hpp"

namespace p3d {
namespace {

constexpr int kWgWaves = 8;
constexpr int kWgRows = 32 * kWgWaves;  // output rows per workgroup
// Tokens per stage for x of 32 IT columns.
template <int IT>
constexpr int wg_tok() { return IT >= 4 ? 64 : 32; }
constexpr int kWgTokMax = 64;
constexpr int kWgMaxCols = 256;  // input columns per workgroup

// Row stride (elements of a 16-bit type) of an LDS tile w elements wide: the
// stride in dwords is 16 mod 32, so the four consecutive rows that a 16-lane
// block reads through one transposed load start in four distinct 16-bank
// ranges; rows stay 16-byte aligned.
constexpr int tile_stride(int w) { return w + 2 * ((16 - (w / 2) % 32 + 32) % 32); }

typedef short v4s __attribute__((ext_vector_type(4)));
typedef short v8s __attribute__((ext_vector_type(8)));

// MFMA operand fragment (32x32x16 layout: lane L holds index L % 32 of the
// M or N dimension and contraction indices 8 (L / 32) .. + 8) from a
// row-major LDS tile whose rows are the contraction index (tokens): rows
// k0 + 8 (L / 32) + t, column c0 + L % 32.  ds_read_b64_tr_b16 hands lane
// B + 4a + e of each 16-lane block element e of the 8-byte windows addressed
// by lanes B + a + 4j (j = 0..3) as its values j, so lane L addresses row
// k0 + 8 (L / 32) + (L % 16) / 4 (four rows further for the second read) at
// column c0 + 16 ((L / 16) % 2) + 4 (L % 4).
template <typename T>
__device__ __forceinline__ typename Mma<T>::Frag frag_tr(const T* tile, int stride, int k0, int c0, int lane) {
    const int row = k0 + 8 * (lane >> 5) + ((lane & 15) >> 2);
    const int col = c0 + 16 * ((lane >> 4) & 1) + 4 * (lane & 3);
    typedef __attribute__((address_space(3))) v4s* lds_v4s;
    const v4s lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4s)(tile + row * stride + col));
    const v4s hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4s)(tile + (row + 4) * stride + col));
    const v8s v = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
    return __builtin_bit_cast(typename Mma<T>::Frag, v);
}

template <int IT>
constexpr int wgrad_stage_elems() { return wg_tok<IT>() * (tile_stride(kWgRows) + tile_stride(32 * IT)); }

// dy as up to three column blocks of output rows: rows [0, end[0]) from
// src[0], [end[0], end[1]) from src[1], [end[1], O) from src[2], each with its
// own row stride (a single dy has end[0] = end[1] = O).
template <typename T>
struct WgSrc {
    const T* src[3];
    int64_t ld[3];
    int end[2];
};

// Partial dW of token range [blockIdx.y * per, + per) for output rows
// [blockIdx.x * rpb, + rpb) (rpb a multiple of 32, at most 256: the rows are
// spread evenly over the row blocks, so that a last block of a few rows does
// not cost a whole workgroup's pass) and input columns [blockIdx.z * I, + I)
// of I_total, written to part[blockIdx.y][o][blockIdx.z * I + i].  Two
// stages of dynamic LDS (2 * wgrad_stage_elems<IT>() elements).
template <typename T, int IT>
__global__ __launch_bounds__(64 * kWgWaves) void k_wgrad(WgSrc<T> dy, const T* x, int64_t ldx, float* part,
                                                        int64_t rows, int O, int rpb, int64_t per, int I_total) {
    typedef Mma<T> M;
    constexpr int I = 32 * IT;
    constexpr int SA = tile_stride(kWgRows), SB = tile_stride(I);
    constexpr int STAGE = wgrad_stage_elems<IT>();         // elements
    constexpr int kWgTok = wg_tok<IT>();
    constexpr int PA = kWgTok * (kWgRows / 8) / (64 * kWgWaves);            // dy pieces per thread
    constexpr int BP = kWgTok * (I / 8);                                     // x pieces per stage
    constexpr int PB = (BP + 64 * kWgWaves - 1) / (64 * kWgWaves);           // x pieces per thread
    static_assert(PA * 64 * kWgWaves == kWgTok * (kWgRows / 8), "dy stage pieces must divide evenly");
    extern __shared__ __align__(16) unsigned char wg_smem[];
    T* lds = reinterpret_cast<T*>(wg_smem);
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, g = lane >> 5;
    const int ob = blockIdx.x * rpb;
    const int64_t n0 = (int64_t)blockIdx.y * per, n1 = min(rows, n0 + per);
    x += (int64_t)blockIdx.z * I;  // this workgroup's input columns
    const bool active = 32 * wave < rpb && ob + 32 * wave < O;  // wave-uniform

    u32x4 ra[PA], rb[PB];
    auto fetch = [&](int64_t t0) __attribute__((always_inline)) {
#pragma unroll
        for (int i = 0; i < PA; ++i) {
            const int p = tid + i * 64 * kWgWaves, r = p / (kWgRows / 8), c = (p % (kWgRows / 8)) * 8;
            const int64_t n = t0 + r;
            const int o = ob + c;  // 8 rows of one source (the blocks are multiples of 8)
            const int sel = o < dy.end[0] ? 0 : (o < dy.end[1] ? 1 : 2);
            const int o_src = o - (sel == 0 ? 0 : dy.end[sel - 1]);
            ra[i] = u32x4{0, 0, 0, 0};
            if (n < n1 && c < rpb && o < O)
                ra[i] = *reinterpret_cast<const u32x4*>(dy.src[sel] + n * dy.ld[sel] + o_src);
        }
#pragma unroll
        for (int i = 0; i < PB; ++i) {
            const int p = tid + i * 64 * kWgWaves, r = p / (I / 8), c = (p % (I / 8)) * 8;
            const int64_t n = t0 + r;
            rb[i] = u32x4{0, 0, 0, 0};
            if (p < BP && n < n1) rb[i] = *reinterpret_cast<const u32x4*>(x + n * ldx + c);
        }
    };
    auto stage = [&](T* st) __attribute__((always_inline)) {
#pragma unroll
        for (int i = 0; i < PA; ++i) {
            const int p = tid + i * 64 * kWgWaves, r = p / (kWgRows / 8), c = (p % (kWgRows / 8)) * 8;
            *reinterpret_cast<u32x4*>(st + r * SA + c) = ra[i];
        }
#pragma unroll
        for (int i = 0; i < PB; ++i) {
            const int p = tid + i * 64 * kWgWaves, r = p / (I / 8), c = (p % (I / 8)) * 8;
            if (p < BP) *reinterpret_cast<u32x4*>(st + kWgTok * SA + r * SB + c) = rb[i];
        }
    };

    f32x16 acc[IT];
#pragma unroll
    for (int t = 0; t < IT; ++t)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[t][r] = 0.f;
    if (n0 < n1) {
        fetch(n0);
        stage(lds);
        __syncthreads();
        int buf = 0;
        for (int64_t t0 = n0; t0 < n1; t0 += kWgTok) {
            const bool more = t0 + kWgTok < n1;
            if (more) fetch(t0 + kWgTok);
            const T* cur = lds + buf * STAGE;
            // Waves past the block's last output row multiply the zero columns
            // of the dy tile: no branch around the MFMAs, whose accumulators would
            // otherwise be copied between register files at the join.
#pragma unroll
            for (int ks = 0; ks < kWgTok / 16; ++ks) {
                const typename M::Frag fa = frag_tr<T>(cur, SA, 16 * ks, 32 * wave, lane);
#pragma unroll
                for (int t = 0; t < IT; ++t)
                    acc[t] = M::mfma(fa, frag_tr<T>(cur + kWgTok * SA, SB, 16 * ks, 32 * t, lane), acc[t]);
            }
            if (more) stage(lds + (buf ^ 1) * STAGE);
            __syncthreads();
            buf ^= 1;
        }
    }
    if (!active) return;
    // D row acc_row(r, g) is output row ob + 32 wave + that; column lane % 32 of tile t is input 32 t + lane % 32.
    float* out = part + (int64_t)blockIdx.y * O * I_total + (int64_t)blockIdx.z * I;
#pragma unroll
    for (int t = 0; t < IT; ++t)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const int o = ob + 32 * wave + acc_row(r, g);
            if (o < O) out[(int64_t)o * I_total + 32 * t + (lane & 31)] = acc[t][r];
        }
}

// dw[e] = sum over splits of part[s][e] in a fixed order: thread group j of
// a block (64 elements x 4 groups) sums splits j, j + 4, ... in increasing
// order, then group 0 adds the four partial sums in order (deterministic).
constexpr int kRedElems = 64, kRedGroups = 4;
__global__ __launch_bounds__(kRedElems * kRedGroups) void k_wgrad_reduce(const float* part, float* dw, int64_t count,
                                                                         int splits) {
    __shared__ float sums[kRedGroups][kRedElems];
    const int le = threadIdx.x % kRedElems, grp = threadIdx.x / kRedElems;
    const int64_t e = (int64_t)blockIdx.x * kRedElems + le;
    float s = 0.f;
    if (e < count)
        for (int k = grp; k < splits; k += kRedGroups) s += part[(int64_t)k * count + e];
    sums[grp][le] = s;
    __syncthreads();
    if (grp == 0 && e < count) {
        float t = sums[0][le];
#pragma unroll
        for (int j = 1; j < kRedGroups; ++j) t += sums[j][le];
        dw[e] = t;
    }
}

// Input widths the kernel takes: a multiple of 32 up to 256 (one column
// block), or a multiple of 256 up to 2048 (column blocks of 256).
inline bool wgrad_cols_ok(int I) {
    return (I >= 32 && I % 32 == 0 && I <= kWgMaxCols) || (I > kWgMaxCols && I % kWgMaxCols == 0 && I <= 2048);
}

template <typename T>
int launch_wgrad(const WgSrc<T>& dy, const void* x, int64_t ldx, float* dw, float* part, int64_t rows, int O, int I,
                 int splits, hipStream_t s) {
    const int64_t per = cdiv(cdiv(rows, splits), kWgTokMax) * kWgTokMax;
    const int used = (int)cdiv(rows, per);
    // Past 256 input columns the columns go to blocks of 256 (grid z), each
    // with its own accumulators; dy is read once per block.
    const int cbs = I > kWgMaxCols ? I / kWgMaxCols : 1, Ib = I / cbs;
    const int nrb = (int)cdiv(O, kWgRows), rpb = 32 * (int)cdiv(cdiv(O, nrb), 32);
    const dim3 grid((unsigned)nrb, (unsigned)used, (unsigned)cbs);
    switch (Ib / 32) {
#define CASE(IT)                                                                                                  \
    case IT:                                                                                                      \
        k_wgrad<T, IT><<<grid, 64 * kWgWaves, 2 * wgrad_stage_elems<IT>() * sizeof(T), s>>>(                      \
            dy, (const T*)x, ldx, part, rows, O, rpb, per, I);                                                         \
        break;
        CASE(1) CASE(2) CASE(3) CASE(4) CASE(5) CASE(6) CASE(7) CASE(8)
#undef CASE
        default: return fail(P3D_EUNSUPPORTED, "in_features must be a multiple of 32, at most 256");
    }
    const int64_t count = (int64_t)O * I;
    k_wgrad_reduce<<<(unsigned)cdiv(count, kRedElems), kRedElems * kRedGroups, 0, s>>>(part, dw, count, used);
    return check_launch("p3d_weight_grad");
}

}  // namespace
}  // namespace p3d

using namespace p3d;

extern "C" int p3d_weight_grad(const void* dy, int64_t ldy, const void* x, int64_t ldx, float* dw, float* workspace,
                               int64_t rows, int32_t out_features, int32_t in_features, int32_t splits, int32_t dtype,
                               void* stream) {
    P3D_REQUIRE(dy && x && dw && workspace, "null pointer argument");
    P3D_REQUIRE(dtype == P3D_F16 || dtype == P3D_BF16, "dtype must be fp16 or bf16");
    P3D_REQUIRE(rows >= 1 && splits >= 1, "need at least one row and one split");
    P3D_REQUIRE(out_features >= 8 && out_features % 8 == 0, "out_features must be a positive multiple of 8");
    P3D_REQUIRE(wgrad_cols_ok(in_features),
                "in_features must be a multiple of 32 up to 256, or a multiple of 256 up to 2048");
    P3D_REQUIRE(ldy >= out_features && ldy % 8 == 0 && ldx >= in_features && ldx % 8 == 0,
                "row strides must cover the rows and keep 16-byte alignment");
    P3D_REQUIRE(aligned16(dy) && aligned16(x), "dy and x must be 16-byte aligned");
    P3D_REQUIRE(cdiv(out_features, kWgRows) < 65536 && splits < 65536, "grid too large");
    if (dtype == P3D_F16) {
        const WgSrc<_Float16> src{{(const _Float16*)dy, nullptr, nullptr}, {ldy, 0, 0}, {out_features, out_features}};
        return launch_wgrad<_Float16>(src, x, ldx, dw, workspace, rows, out_features, in_features, splits,
                                      as_stream(stream));
    }
    const WgSrc<__bf16> src{{(const __bf16*)dy, nullptr, nullptr}, {ldy, 0, 0}, {out_features, out_features}};
    return launch_wgrad<__bf16>(src, x, ldx, dw, workspace, rows, out_features, in_features, splits,
                                as_stream(stream));
}

extern "C" int p3d_weight_grad3(const void* dy0, int64_t ld0, int32_t out0, const void* dy1, int64_t ld1,
                                int32_t out1, const void* dy2, int64_t ld2, int32_t out2, const void* x, int64_t ldx,
                                float* dw, float* workspace, int64_t rows, int32_t in_features, int32_t splits,
                                int32_t dtype, void* stream) {
    P3D_REQUIRE(dy0 && dy1 && dy2 && x && dw && workspace, "null pointer argument");
    P3D_REQUIRE(dtype == P3D_F16 || dtype == P3D_BF16, "dtype must be fp16 or bf16");
    P3D_REQUIRE(rows >= 1 && splits >= 1, "need at least one row and one split");
    P3D_REQUIRE(out0 >= 8 && out1 >= 8 && out2 >= 8 && out0 % 8 == 0 && out1 % 8 == 0 && out2 % 8 == 0 &&
                    (int64_t)out0 + out1 + out2 < (1 << 24),
                "out features must be positive multiples of 8");
    P3D_REQUIRE(wgrad_cols_ok(in_features),
                "in_features must be a multiple of 32 up to 256, or a multiple of 256 up to 2048");
    P3D_REQUIRE(ld0 >= out0 && ld1 >= out1 && ld2 >= out2 && ld0 % 8 == 0 && ld1 % 8 == 0 && ld2 % 8 == 0 &&
                    ldx >= in_features && ldx % 8 == 0,
                "row strides must cover the rows and keep 16-byte alignment");
    P3D_REQUIRE(aligned16(dy0) && aligned16(dy1) && aligned16(dy2) && aligned16(x), "dy and x must be 16-byte aligned");
    const int O = out0 + out1 + out2;
    P3D_REQUIRE(cdiv(O, kWgRows) < 65536 && splits < 65536, "grid too large");
    if (dtype == P3D_F16) {
        const WgSrc<_Float16> src{{(const _Float16*)dy0, (const _Float16*)dy1, (const _Float16*)dy2},
                                  {ld0, ld1, ld2},
                                  {out0, out0 + out1}};
        return launch_wgrad<_Float16>(src, x, ldx, dw, workspace, rows, O, in_features, splits, as_stream(stream));
    }
    const WgSrc<__bf16> src{{(const __bf16*)dy0, (const __bf16*)dy1, (const __bf16*)dy2}, {ld0, ld1, ld2},
                            {out0, out0 + out1}};
    return launch_wgrad<__bf16>(src, x, ldx, dw, workspace, rows, O, in_features, splits, as_stream(stream));
}
