// Fused projections of the PACK3D layer (attention.py:64-67,85,89 of
// amilworks/Pack3D).  k_project: LayerNorm, the to_q, to_kv and gate linear
// maps of the normalised tokens as one MFMA GEMM with contraction length
// dim, and the gate's two-way softmax (softmax(-1)[..., 1]), in one pass
// over the tokens.  k_out_residual: x + to_out(y).
//
// A wave owns 32 tokens.  Lane l holds token l % 32 and, for every 16-channel
// k-step, channels 8 (l / 32) .. +8 of it: the B operand of the 32x32x16
// MFMA.  It loads them as 16-byte pieces, forms the LayerNorm statistics
// together with lane l ^ 32 (which holds the other half of the row),
// normalises in fp32 and rounds to the storage type, as torch's LayerNorm
// output is, and keeps them in registers for the whole GEMM.  The weights
// come 32 output rows at a time as the A operand: the 8 waves of a
// workgroup stage each 32-row block in LDS once (double-buffered, the next
// block's loads in flight while the current one is multiplied), so the
// weights cross the cache hierarchy once per 256 tokens.  D = W X^T then holds,
// in lane l, register r, output 32 ob + acc_row(r, l / 32) of token l % 32.
// A wave writes its 32 x 32 block of q / kv outputs into a private LDS tile
// and stores it back as rows, four lanes per token, so every token's 64
// bytes leave as one coalesced 64-byte piece rather than as 16-byte
// fragments of 32 different rows.  Outputs are rounded to the storage type,
// as the linear maps' outputs are; the gate bias is added before that
// rounding and the pair softmax runs in fp32 on the rounded logits.
#include "common.hpp"

namespace p3d {
namespace {

constexpr int kProjMaxDim = 512;
constexpr int kProjWaves = 8;

struct ProjDev {
    const char* x;
    const void *ln_w, *ln_b;
    const char *wq, *wkv, *wg;
    const void* gate_bias;
    char *q, *kv, *gate;
    int64_t rows;
    int dim, q_out, kv_out, heads;
    int ln_dtype, gate_bias_dtype;
    float eps;
};

template <typename T>
__device__ __forceinline__ void store4(T* dst, const float (&v)[4]) {
    typedef __attribute__((ext_vector_type(4))) T T4;
    T4 o;
#pragma unroll
    for (int i = 0; i < 4; ++i) o[i] = from_f32<T>(v[i]);
    *reinterpret_cast<T4*>(dst) = o;
}

// Waves per SIMD: 4 up to dim 128, 3 at dim 192 (the 168 registers that
// leaves hold the GEMM without spilling; at 4 it spilled 16), else 2.
template <typename T, int KS>
__global__ __launch_bounds__(64 * kProjWaves)
__attribute__((amdgpu_waves_per_eu(KS <= 8 ? 4 : (KS <= 12 ? 3 : 2)))) void k_project(ProjDev a) {
    typedef Mma<T> M;
    typedef typename M::Frag Frag;
    constexpr int DIM = 16 * KS;
    constexpr int WS = DIM + 8;                     // LDS weight-row stride (elements), 16-byte pad
    constexpr int PIECES = 32 * DIM / 8;            // 16-byte pieces of a 32-row weight block
    constexpr int PPT = (PIECES + 64 * kProjWaves - 1) / (64 * kProjWaves);  // per thread
    __shared__ __align__(16) float lw[DIM], lb[DIM];
    constexpr int OS = 32 + 8;                      // output tile row stride (elements)
    __shared__ __align__(16) T wbuf[2][32 * WS];
    __shared__ __align__(16) T otile[kProjWaves][32 * OS];
    for (int c = threadIdx.x; c < DIM; c += blockDim.x) {
        lw[c] = load_any(a.ln_w, c, a.ln_dtype);
        lb[c] = load_any(a.ln_b, c, a.ln_dtype);
    }
    const int gbase = a.q_out + a.kv_out, nout = gbase + 2 * a.heads;
    const int nblocks = (nout + 31) / 32;
    // Weight row o of the concatenation [Wq; Wkv; Wg] (rows past nout are zero).
    auto wrow = [&](int o) __attribute__((always_inline)) -> const T* {
        return o < a.q_out ? reinterpret_cast<const T*>(a.wq) + (int64_t)o * DIM
               : o < gbase ? reinterpret_cast<const T*>(a.wkv) + (int64_t)(o - a.q_out) * DIM
                           : reinterpret_cast<const T*>(a.wg) + (int64_t)(o - gbase) * DIM;
    };
    u32x4 wreg[PPT];
    auto fetch = [&](int ob) __attribute__((always_inline)) {
#pragma unroll
        for (int i = 0; i < PPT; ++i) {
            const int pc = threadIdx.x + i * 64 * kProjWaves, r = pc / (DIM / 8), c = (pc % (DIM / 8)) * 8;
            const int o = 32 * ob + r;
            wreg[i] = (pc < PIECES && o < nout) ? *reinterpret_cast<const u32x4*>(wrow(o) + c) : u32x4{0u, 0u, 0u, 0u};
        }
    };
    auto stage = [&](int buf) __attribute__((always_inline)) {
#pragma unroll
        for (int i = 0; i < PPT; ++i) {
            const int pc = threadIdx.x + i * 64 * kProjWaves, r = pc / (DIM / 8), c = (pc % (DIM / 8)) * 8;
            if (pc < PIECES) *reinterpret_cast<u32x4*>(&wbuf[buf][r * WS + c]) = wreg[i];
        }
    };
    fetch(0);
    stage(0);
    if (nblocks > 1) fetch(1);
    __syncthreads();

    const int lane = threadIdx.x & 63, g = lane >> 5, t = lane & 31;
    const int64_t tok0 = ((int64_t)blockIdx.x * kProjWaves + (threadIdx.x >> 6)) * 32, tok = tok0 + t;
    T* tile = otile[threadIdx.x >> 6];
    const bool live = tok < a.rows;
    const T* xr = reinterpret_cast<const T*>(a.x) + (live ? tok : 0) * DIM + 8 * g;

    // ---- LayerNorm of the lane's half row (channels 16 ks + 8 g + j)
    u32x4 raw[KS];
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) raw[ks] = *reinterpret_cast<const u32x4*>(xr + 16 * ks);
    float sum = 0.f;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
        const T* v = reinterpret_cast<const T*>(&raw[ks]);
#pragma unroll
        for (int j = 0; j < 8; ++j) sum += to_f32(v[j]);
    }
    const float mean = (sum + lane_xor32(sum)) / (float)DIM;
    float sq = 0.f;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
        const T* v = reinterpret_cast<const T*>(&raw[ks]);
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const float c = to_f32(v[j]) - mean;
            sq += c * c;
        }
    }
    const float rstd = 1.f / sqrtf((sq + lane_xor32(sq)) / (float)DIM + a.eps);
    Frag xf[KS];
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
        const T* v = reinterpret_cast<const T*>(&raw[ks]);
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const int c = 16 * ks + 8 * g + j;
            xf[ks][j] = from_f32<T>((to_f32(v[j]) - mean) * rstd * lw[c] + lb[c]);
        }
    }

    // ---- D = W X^T, 32 outputs at a time
    T* go = reinterpret_cast<T*>(a.gate) + tok * a.heads;
    for (int ob = 0; ob < nblocks; ++ob) {
        const T* wb = &wbuf[ob & 1][t * WS + 8 * g];
        f32x16 d;
#pragma unroll
        for (int r = 0; r < 16; ++r) d[r] = 0.f;
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) d = M::mfma(*reinterpret_cast<const Frag*>(wb + 16 * ks), xf[ks], d);
        if (32 * ob < gbase) {
            // q / kv outputs of the block through the tile: row t, columns
            // acc_row(4 qd, g) .. +3, then 16-byte pieces (token tt, outputs
            // 8 pp .. +7) with four consecutive lanes per token.
#pragma unroll
            for (int qd = 0; qd < 4; ++qd) {
                const float v[4] = {d[4 * qd], d[4 * qd + 1], d[4 * qd + 2], d[4 * qd + 3]};
                store4<T>(tile + t * OS + acc_row(4 * qd, g), v);
            }
            wave_lds_sync();
#pragma unroll
            for (int i = 0; i < 2; ++i) {
                const int tt = 16 * i + (lane >> 2), pp = lane & 3, o0 = 32 * ob + 8 * pp;
                const int64_t tk = tok0 + tt;
                if (tk < a.rows && o0 < gbase) {
                    const u32x4 piece = *reinterpret_cast<const u32x4*>(tile + tt * OS + 8 * pp);
                    T* dst = o0 < a.q_out ? reinterpret_cast<T*>(a.q) + tk * a.q_out + o0
                                          : reinterpret_cast<T*>(a.kv) + tk * a.kv_out + (o0 - a.q_out);
                    *reinterpret_cast<u32x4*>(dst) = piece;
                }
            }
            wave_lds_sync();  // the next block's tile writes follow these reads
        }
        if (live && 32 * ob + 32 > gbase) {
#pragma unroll
            for (int qd = 0; qd < 4; ++qd) {
                const int o0 = 32 * ob + acc_row(4 * qd, g);  // outputs o0 .. o0 + 3
                float v[4] = {d[4 * qd], d[4 * qd + 1], d[4 * qd + 2], d[4 * qd + 3]};
                if (o0 >= gbase && o0 < nout) {
                    // Logit pairs (2h, 2h + 1) of heads h = (o0 - gbase) / 2 + {0, 1}.
#pragma unroll
                    for (int p = 0; p < 2; ++p) {
                        const int j = o0 - gbase + 2 * p;
                        if (j + 1 >= 2 * a.heads) break;
                        const float l0 =
                            to_f32(from_f32<T>(v[2 * p] + load_any(a.gate_bias, j, a.gate_bias_dtype)));
                        const float l1 =
                            to_f32(from_f32<T>(v[2 * p + 1] + load_any(a.gate_bias, j + 1, a.gate_bias_dtype)));
                        const float m = fmaxf(l0, l1);
                        const float e0 = expf(l0 - m), e1 = expf(l1 - m);
                        go[j / 2] = from_f32<T>(e1 / (e0 + e1));
                    }
                }
            }
        }
        if (ob + 1 < nblocks) {
            stage((ob + 1) & 1);
            if (ob + 2 < nblocks) fetch(ob + 2);
        }
        __syncthreads();
    }
}

// Output projection with the residual (attention.py:89): out = x + y Wo^T
// for y [rows, K] (the core's output, heads concatenated), Wo [dim, K] and
// x, out [rows, dim]: the same tiling as k_project without the LayerNorm (y
// is the B operand as loaded), 32 outputs per block.  The block's fp32
// accumulators go through the wave's tile, and the store phase adds the
// residual piece and rounds once, as a GEMM with the residual as its C
// operand does.
template <typename T, int KS>
__global__ __launch_bounds__(64 * kProjWaves) __attribute__((amdgpu_waves_per_eu(KS <= 12 ? 4 : 2)))
void k_out_residual(const T* __restrict__ y, const T* __restrict__ wo, const T* __restrict__ x, T* __restrict__ out,
                    int64_t rows, int dim) {
    typedef Mma<T> M;
    typedef typename M::Frag Frag;
    constexpr int K = 16 * KS;
    constexpr int WS = K + 8;
    constexpr int PIECES = 32 * K / 8;
    constexpr int PPT = (PIECES + 64 * kProjWaves - 1) / (64 * kProjWaves);
    constexpr int OS = 32 + 4;                      // fp32 output tile row stride
    __shared__ __align__(16) T wbuf[2][32 * WS];
    __shared__ __align__(16) float otile[kProjWaves][32 * OS];
    const int nblocks = dim / 32;
    u32x4 wreg[PPT];
    auto fetch = [&](int ob) __attribute__((always_inline)) {
#pragma unroll
        for (int i = 0; i < PPT; ++i) {
            const int pc = threadIdx.x + i * 64 * kProjWaves, r = pc / (K / 8), c = (pc % (K / 8)) * 8;
            wreg[i] = pc < PIECES ? *reinterpret_cast<const u32x4*>(wo + (int64_t)(32 * ob + r) * K + c)
                                  : u32x4{0u, 0u, 0u, 0u};
        }
    };
    auto stage = [&](int buf) __attribute__((always_inline)) {
#pragma unroll
        for (int i = 0; i < PPT; ++i) {
            const int pc = threadIdx.x + i * 64 * kProjWaves, r = pc / (K / 8), c = (pc % (K / 8)) * 8;
            if (pc < PIECES) *reinterpret_cast<u32x4*>(&wbuf[buf][r * WS + c]) = wreg[i];
        }
    };
    fetch(0);
    stage(0);
    if (nblocks > 1) fetch(1);
    __syncthreads();

    const int lane = threadIdx.x & 63, g = lane >> 5, t = lane & 31;
    const int64_t tok0 = ((int64_t)blockIdx.x * kProjWaves + (threadIdx.x >> 6)) * 32, tok = tok0 + t;
    const bool live = tok < rows;
    float* tile = otile[threadIdx.x >> 6];
    const T* yr = y + (live ? tok : 0) * K + 8 * g;
    Frag yf[KS];
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) yf[ks] = __builtin_bit_cast(Frag, *reinterpret_cast<const u32x4*>(yr + 16 * ks));

    for (int ob = 0; ob < nblocks; ++ob) {
        const T* wb = &wbuf[ob & 1][t * WS + 8 * g];
        f32x16 d;
#pragma unroll
        for (int r = 0; r < 16; ++r) d[r] = 0.f;
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) d = M::mfma(*reinterpret_cast<const Frag*>(wb + 16 * ks), yf[ks], d);
#pragma unroll
        for (int qd = 0; qd < 4; ++qd)
            *reinterpret_cast<f32x4*>(tile + t * OS + acc_row(4 * qd, g)) =
                f32x4{d[4 * qd], d[4 * qd + 1], d[4 * qd + 2], d[4 * qd + 3]};
        wave_lds_sync();
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const int tt = 16 * i + (lane >> 2), pp = lane & 3, o0 = 32 * ob + 8 * pp;
            const int64_t tk = tok0 + tt;
            if (tk < rows) {
                const f32x4 lo = *reinterpret_cast<const f32x4*>(tile + tt * OS + 8 * pp);
                const f32x4 hi = *reinterpret_cast<const f32x4*>(tile + tt * OS + 8 * pp + 4);
                const u32x4 res = *reinterpret_cast<const u32x4*>(x + tk * dim + o0);
                const T* rv = reinterpret_cast<const T*>(&res);
                u32x4 o;
                T* ov = reinterpret_cast<T*>(&o);
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    ov[e] = from_f32<T>(lo[e] + to_f32(rv[e]));
                    ov[4 + e] = from_f32<T>(hi[e] + to_f32(rv[4 + e]));
                }
                *reinterpret_cast<u32x4*>(out + tk * dim + o0) = o;
            }
        }
        wave_lds_sync();
        if (ob + 1 < nblocks) {
            stage((ob + 1) & 1);
            if (ob + 2 < nblocks) fetch(ob + 2);
        }
        __syncthreads();
    }
}

template <typename T>
int launch_project(const ProjDev& d, hipStream_t s) {
    const unsigned blocks = (unsigned)cdiv(cdiv(d.rows, 32), kProjWaves);
    switch (d.dim) {
#define CASE(DIM)                                                                     \
    case DIM:                                                                         \
        k_project<T, DIM / 16><<<blocks, 64 * kProjWaves, 0, s>>>(d);                 \
        break;
        CASE(64) CASE(96) CASE(128) CASE(192) CASE(256) CASE(384) CASE(512)
#undef CASE
        default: return fail(P3D_EUNSUPPORTED, "dim must be one of 64, 96, 128, 192, 256, 384, 512");
    }
    return check_launch("p3d_project");
}

template <typename T>
int launch_out_residual(const void* y, const void* wo, const void* x, void* out, int64_t rows, int k, int dim,
                        hipStream_t s) {
    const unsigned blocks = (unsigned)cdiv(cdiv(rows, 32), kProjWaves);
    switch (k) {
#define CASE(KK)                                                                                               \
    case KK:                                                                                                   \
        k_out_residual<T, KK / 16><<<blocks, 64 * kProjWaves, 0, s>>>((const T*)y, (const T*)wo, (const T*)x, \
                                                                      (T*)out, rows, dim);                     \
        break;
        CASE(64) CASE(96) CASE(128) CASE(192) CASE(256) CASE(384) CASE(512)
#undef CASE
        default: return fail(P3D_EUNSUPPORTED, "heads * head_dim must be one of 64, 96, 128, 192, 256, 384, 512");
    }
    return check_launch("p3d_out_residual");
}

}  // namespace
}  // namespace p3d

using namespace p3d;

extern "C" int p3d_out_residual(const void* y, const void* wo, const void* x, void* out, int64_t rows, int32_t k,
                                int32_t dim, int32_t dtype, void* stream) {
    P3D_REQUIRE(y && wo && x && out, "null pointer argument");
    P3D_REQUIRE(dtype == P3D_F16 || dtype == P3D_BF16, "dtype must be fp16 or bf16");
    P3D_REQUIRE(rows >= 1, "need at least one row");
    P3D_REQUIRE(dim >= 32 && dim % 32 == 0 && dim <= kProjMaxDim, "dim must be a multiple of 32, at most 512");
    P3D_REQUIRE(aligned16(y) && aligned16(wo) && aligned16(x) && aligned16(out), "pointers must be 16-byte aligned");
    P3D_REQUIRE(cdiv(rows, 32 * kProjWaves) < (1LL << 31), "too many rows");
    hipStream_t s = as_stream(stream);
    return dtype == P3D_F16 ? launch_out_residual<_Float16>(y, wo, x, out, rows, k, dim, s)
                            : launch_out_residual<__bf16>(y, wo, x, out, rows, k, dim, s);
}

extern "C" int p3d_project(const p3d_project_args* args, void* stream) {
    P3D_REQUIRE(args, "null args");
    const p3d_project_args& a = *args;
    P3D_REQUIRE(a.dtype == P3D_F16 || a.dtype == P3D_BF16, "dtype must be fp16 or bf16");
    P3D_REQUIRE(a.ln_dtype >= P3D_F32 && a.ln_dtype <= P3D_BF16 && a.gate_bias_dtype >= P3D_F32 &&
                    a.gate_bias_dtype <= P3D_BF16,
                "unknown parameter dtype");
    P3D_REQUIRE(a.x && a.ln_weight && a.ln_bias && a.wq && a.wkv && a.wg && a.gate_bias && a.q && a.kv && a.gate,
                "null pointer argument");
    P3D_REQUIRE(a.rows >= 1 && a.heads >= 1, "empty projection problem");
    P3D_REQUIRE(a.dim >= 16 && a.dim <= kProjMaxDim && a.dim % 16 == 0, "dim must be a multiple of 16, at most 512");
    P3D_REQUIRE(a.q_out >= 16 && a.q_out % 16 == 0 && a.kv_out >= 16 && a.kv_out % 16 == 0,
                "q_out and kv_out must be positive multiples of 16");
    P3D_REQUIRE(aligned16(a.x) && aligned16(a.wq) && aligned16(a.wkv) && aligned16(a.wg),
                "x and the weights must be 16-byte aligned");
    P3D_REQUIRE(aligned16(a.q) && aligned16(a.kv), "q and kv must be 16-byte aligned");
    P3D_REQUIRE(cdiv(a.rows, 32 * kProjWaves) < (1LL << 31), "too many rows");
    ProjDev d;
    d.x = (const char*)a.x;
    d.ln_w = a.ln_weight;
    d.ln_b = a.ln_bias;
    d.wq = (const char*)a.wq;
    d.wkv = (const char*)a.wkv;
    d.wg = (const char*)a.wg;
    d.gate_bias = a.gate_bias;
    d.q = (char*)a.q;
    d.kv = (char*)a.kv;
    d.gate = (char*)a.gate;
    d.rows = a.rows;
    d.dim = a.dim;
    d.q_out = a.q_out;
    d.kv_out = a.kv_out;
    d.heads = a.heads;
    d.ln_dtype = a.ln_dtype;
    d.gate_bias_dtype = a.gate_bias_dtype;
    d.eps = a.eps;
    hipStream_t s = as_stream(stream);
    return a.dtype == P3D_F16 ? launch_project<_Float16>(d, s) : launch_project<__bf16>(d, s);
}
