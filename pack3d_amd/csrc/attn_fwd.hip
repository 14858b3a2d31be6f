// Fused PACK3D attention forward (reference.py:16-31 of amilworks/Pack3D).
//
// Grid kernel (complete-grid layouts): a workgroup of 4 waves owns a
// 4 x 8 x 8 (z, y, x) brick of queries of one (batch, head); each wave owns a
// 4 x 4 x 4 sub-brick, split into two 2 x 4 x 4 column blocks of 32 queries.
//   1. Queries are gathered through the raster->packed map and rotated on
//      load (axial RoPE fused), rounded to the storage type.
//   2. Local pathway: the halo of the brick is streamed plane by plane
//      (z), each plane 12 x 12 keys with K rotated on load; each wave scores
//      its 8 x 8 key footprint (two 32-key tiles) against its queries on
//      MFMA and masks the (2rz+1)(2ry+1)(2rx+1) stencil and the grid border
//      from coordinates, so the neighbour table is never read.
//   3. Global pathway: all summaries are streamed through LDS in stages of
//      64 and scored on MFMA with a second online-softmax state.
//   4. Epilogue: y = sl * o_L + gate * sg * o_G, stored in the storage type.
// Rows kernel (any validated geometry): the same global pathway and epilogue
// for 64 packed rows per wave, with the local branch read from a buffer.
#include "attn_common.hpp"

namespace p3d {
namespace {

constexpr int kWaves = 4;
constexpr int kPlane = 12;                 // plane side for radius <= 2 and an 8 x 8 brick face
constexpr int kPlaneKeys = kPlane * kPlane;
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;

struct AttnDev {
    int B, H, G, N, M, Mp;
    int Z, Y, X, rz, ry, rx;
    int bricks_y, bricks_x;
    int gate_dtype;
    const char *q, *kl, *vl, *gate;
    int64_t qsb, qsh, qsn, ksb, ksh, ksn, vsb, vsh, vsn, gsb, gsh, gsn;
    const float *sl, *sg;
    const char *sk, *svt;
    RopeDev rope;
    const int32_t* map;
    const float* o_local_in;
    char* y;
    int64_t ysb, ysh, ysn;
    float *lse_l, *lse_g;
    char *o_l, *o_g;
    float scale_log2;  // log2(e) / sqrt(D)
};

template <typename T>
__device__ __forceinline__ const T* tp(const char* p) { return reinterpret_cast<const T*>(p); }

// Load and rotate this lane's query channels into score-MFMA B fragments.
template <typename C>
__device__ __forceinline__ void load_q(const typename C::T_* row, bool valid, const RopeDev& rope,
                                       const int64_t pos[3], int g, typename C::Frag* qf) {
    typedef typename C::T_ T;
#pragma unroll
    for (int t = 0; t < C::NT; ++t) {
        if constexpr (C::E == 8) {
            float x[8];
            const int c0 = t * C::KS + 8 * g;
            if (valid) {
                load_piece<T>(row + c0, x);
                rope_apply(rope, pos, c0, x, 8);
            } else {
#pragma unroll
                for (int j = 0; j < 8; ++j) x[j] = 0.f;
            }
#pragma unroll
            for (int j = 0; j < 8; ++j) qf[t][j] = from_f32<T>(x[j]);
        } else {
            float x[2] = {0.f, 0.f};
            const int c0 = t * C::KS;
            if (valid) {
                x[0] = to_f32(row[c0]);
                x[1] = to_f32(row[c0 + 1]);
                rope_apply(rope, pos, c0, x, 2);
            }
            qf[t] = x[g];
        }
    }
}

// Stage summaries [base, base + 64) of one KV head: K rows (natural order)
// and V transposed, in LDS.  The padded summary rows of sk / svt are zero.
template <typename C>
__device__ __forceinline__ void stage_summaries(const AttnDev& a, int64_t bg, int base, typename C::T_* Ks,
                                                typename C::T_* Vs, int vstride) {
    typedef typename C::T_ T;
    constexpr int EP = Piece<T>::N;
    constexpr int D = C::D;
    const int rows = min(64, a.Mp - base);
    const T* sk = tp<T>(a.sk) + ((int64_t)bg * a.Mp + base) * D;
    for (int p = threadIdx.x; p < rows * (D / EP); p += 64 * kWaves) {
        const int r = p / (D / EP), c = (p - r * (D / EP)) * EP;
        *reinterpret_cast<uint4*>(Ks + r * C::KSTR + c) = *reinterpret_cast<const uint4*>(sk + r * D + c);
    }
    const T* svt = tp<T>(a.svt) + ((int64_t)bg * (a.Mp / 32) + base / 32) * D * 32;
    const int tiles = rows / 32;
    for (int p = threadIdx.x; p < tiles * D * (32 / EP); p += 64 * kWaves) {
        const int tt = p / (D * (32 / EP));
        const int rem = p - tt * D * (32 / EP);
        const int ch = rem / (32 / EP), k = (rem - ch * (32 / EP)) * EP;
        *reinterpret_cast<uint4*>(Vs + ch * vstride + 32 * tt + k) =
            *reinterpret_cast<const uint4*>(svt + ((int64_t)tt * D + ch) * 32 + k);
    }
}

// One global stage on this wave's two column blocks.
template <typename C>
__device__ __forceinline__ void global_stage(const AttnDev& a, int base, const typename C::T_* Ks,
                                             const typename C::T_* Vs, int vstride,
                                             const typename C::Frag (*qf)[C::NT], Soft<C::MB>* st, int lane) {
    typedef typename C::T_ T;
    const int g = lane >> 5, qi = lane & 31;
#pragma unroll
    for (int tt = 0; tt < 2; ++tt) {
        const int first = base + 32 * tt;
        if (first >= a.M) break;
        const T* krow = Ks + (32 * tt + kperm<C::E, C::KS>(qi)) * C::KSTR + C::E * g;
        auto vload = [&](int mb, int ks) -> typename C::Frag {
            const int ch = 32 * mb + qi;
            const T* p = Vs + min(ch, C::D - 1) * vstride + 32 * tt + ks * C::KS + C::E * g;
            typename C::Frag f = frag_load16<T>(p);
            if (32 * mb + 32 > C::D && ch >= C::D) f = frag_fill<T>((C::ONES && ch == C::D) ? 1.f : 0.f);
            return f;
        };
#pragma unroll
        for (int nb = 0; nb < 2; ++nb) {
            f32x16 s = score_tile<C>(krow, qf[nb]);
            if (first + 32 > a.M) {
#pragma unroll
                for (int r = 0; r < 16; ++r)
                    if (first + kperm<C::E, C::KS>(acc_row(r, g)) >= a.M) s[r] = -INFINITY;
            }
            soft_update<C>(st[nb], s, a.scale_log2, vload);
        }
    }
}

// Channels of accumulator register r in lane group g of block mb.
__device__ __forceinline__ int acc_channel(int mb, int r, int g) { return 32 * mb + acc_row(r, g); }

template <typename C>
__device__ __forceinline__ void store_quad(typename C::T_* dst, const float* v) {
    typedef typename C::T_ T;
#pragma unroll
    for (int i = 0; i < 4; ++i) dst[i] = from_f32<T>(v[i]);
}

template <typename C>
__device__ __forceinline__ void epilogue(const AttnDev& a, int b, int h, int64_t row, bool valid, int g,
                                         const Soft<C::MB>& sg_state, const float (*ylocal)[16]) {
    typedef typename C::T_ T;
    const float den = soft_denominator<C>(sg_state, g);
    if (!valid) return;
    const float inv = 1.f / den;
    const int64_t bh = (int64_t)b * a.H + h;
    const float gate = load_any(a.gate, b * a.gsb + h * a.gsh + row * a.gsn, a.gate_dtype);
    T* y = reinterpret_cast<T*>(a.y) + b * a.ysb + h * a.ysh + row * a.ysn;
    T* og = a.o_g ? reinterpret_cast<T*>(a.o_g) + (bh * a.N + row) * C::D : nullptr;
#pragma unroll
    for (int mb = 0; mb < C::MB; ++mb)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            if (32 * mb + 8 * q >= C::D) continue;
            const int ch0 = acc_channel(mb, 4 * q, g);
            float out[4], o[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                o[i] = sg_state.acc[mb][4 * q + i] * inv;
                out[i] = ylocal[mb][4 * q + i] + gate * a.sg[ch0 + i] * o[i];
            }
            store_quad<C>(y + ch0, out);
            if (og) store_quad<C>(og + ch0, o);
        }
    if (a.lse_g) a.lse_g[bh * a.N + row] = sg_state.m * kLn2 + __logf(den);
}

// Finish the local state: ylocal = sl * o_L; optionally save o_L and its LSE.
template <typename C>
__device__ __forceinline__ void finish_local(const AttnDev& a, int b, int h, int64_t row, bool valid, int g,
                                             const Soft<C::MB>& st, float (*ylocal)[16]) {
    typedef typename C::T_ T;
    const float den = soft_denominator<C>(st, g);
    const float inv = den > 0.f ? 1.f / den : 0.f;  // an all-masked row gives 0
    const int64_t bh = (int64_t)b * a.H + h;
    T* ol = (a.o_l && valid) ? reinterpret_cast<T*>(a.o_l) + (bh * a.N + row) * C::D : nullptr;
#pragma unroll
    for (int mb = 0; mb < C::MB; ++mb)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            if (32 * mb + 8 * q >= C::D) continue;
            const int ch0 = acc_channel(mb, 4 * q, g);
            float o[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                o[i] = st.acc[mb][4 * q + i] * inv;
                ylocal[mb][4 * q + i] = a.sl[ch0 + i] * o[i];
            }
            if (ol) store_quad<C>(ol + ch0, o);
        }
    if (a.lse_l && valid) a.lse_l[bh * a.N + row] = den > 0.f ? st.m * kLn2 + __logf(den) : -INFINITY;
}

template <typename T, int D>
__global__ __launch_bounds__(64 * kWaves, 2) void k_attn_grid(AttnDev a) {
    typedef Cfg<T, D> C;
    constexpr int EP = Piece<T>::N;
    constexpr int VPS = kPlaneKeys + EP;  // plane V row stride (elements)
    constexpr int VGS = 64 + EP;          // summary V row stride (elements)
    extern __shared__ __align__(16) unsigned char smem[];
    T* Kp = reinterpret_cast<T*>(smem);
    T* Vp = Kp + kPlaneKeys * C::KSTR;
    T* Ks = reinterpret_cast<T*>(smem);  // global stages reuse the plane buffer
    T* Vs = Ks + 64 * C::KSTR;

    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, g = lane >> 5, qi = lane & 31;
    const int bh = blockIdx.y, b = bh / a.H, h = bh % a.H, kvh = h / (a.H / a.G);
    const int64_t bg = (int64_t)b * a.G + kvh;
    const int brick = blockIdx.x;
    const int Z0 = 4 * (brick / (a.bricks_y * a.bricks_x));
    const int Y0 = 8 * ((brick / a.bricks_x) % a.bricks_y);
    const int X0 = 8 * (brick % a.bricks_x);
    const int wy = wave >> 1, wx = wave & 1;
    const int qy = (qi >> 2) & 3, qx = qi & 3;  // within the wave footprint

    // ---- queries
    typename C::Frag qf[2][C::NT];
    int64_t qrow[2];
    bool qok[2];
#pragma unroll
    for (int nb = 0; nb < 2; ++nb) {
        const int gz = Z0 + 2 * nb + (qi >> 4), gy = Y0 + 4 * wy + qy, gx = X0 + 4 * wx + qx;
        qok[nb] = gz < a.Z && gy < a.Y && gx < a.X;
        const int64_t raster = ((int64_t)gz * a.Y + gy) * a.X + gx;
        qrow[nb] = qok[nb] ? (a.map ? (int64_t)a.map[raster] : raster) : 0;
        int64_t pos[3] = {gz, gy, gx};
        if (a.rope.packed) pos[0] = qrow[nb], pos[1] = 0, pos[2] = 0;
        const T* row = tp<T>(a.q) + b * a.qsb + h * a.qsh + qrow[nb] * a.qsn;
        load_q<C>(row, qok[nb], a.rope, pos, g, qf[nb]);
    }

    Soft<C::MB> st[2];
    st[0].reset();
    st[1].reset();

    // ---- local pathway
    const T* KL = tp<T>(a.kl) + b * a.ksb + kvh * a.ksh;
    const T* VL = tp<T>(a.vl) + b * a.vsb + kvh * a.vsh;
    const int planes = 4 + 2 * a.rz;
    for (int hz = 0; hz < planes; ++hz) {
        __syncthreads();
        const int gz = Z0 - a.rz + hz;
        // Stage the 12 x 12 plane: K rotated, V transposed; keys outside the
        // grid or the footprint are zero (they are masked below).
        for (int p = tid; p < kPlaneKeys * (D / EP); p += 64 * kWaves) {
            const int key = p / (D / EP), c0 = (p - key * (D / EP)) * EP;
            const int ky = key / kPlane, kx = key - ky * kPlane;
            const int gy = Y0 - a.ry + ky, gx = X0 - a.rx + kx;
            const bool in = gz >= 0 && gz < a.Z && gy >= 0 && gy < a.Y && gx >= 0 && gx < a.X &&
                            ky < 8 + 2 * a.ry && kx < 8 + 2 * a.rx;
            float kv[EP], vv[EP];
            if (in) {
                const int64_t raster = ((int64_t)gz * a.Y + gy) * a.X + gx;
                const int64_t row = a.map ? (int64_t)a.map[raster] : raster;
                load_piece<T>(KL + row * a.ksn + c0, kv);
                load_piece<T>(VL + row * a.vsn + c0, vv);
                int64_t pos[3] = {gz, gy, gx};
                if (a.rope.packed) pos[0] = row, pos[1] = 0, pos[2] = 0;
                rope_apply(a.rope, pos, c0, kv, EP);
            } else {
#pragma unroll
                for (int e = 0; e < EP; ++e) kv[e] = vv[e] = 0.f;
            }
            T kt[EP];
#pragma unroll
            for (int e = 0; e < EP; ++e) {
                kt[e] = from_f32<T>(kv[e]);
                Vp[(c0 + e) * VPS + key] = from_f32<T>(vv[e]);
            }
            *reinterpret_cast<uint4*>(Kp + key * C::KSTR + c0) = *reinterpret_cast<const uint4*>(kt);
        }
        __syncthreads();
#pragma unroll
        for (int nb = 0; nb < 2; ++nb) {
            const int qz = 2 * nb + (qi >> 4);
            if (hz < 2 * nb || hz > 2 * nb + 1 + 2 * a.rz) continue;  // plane out of reach
            const bool zok = hz - qz >= 0 && hz - qz <= 2 * a.rz;
#pragma unroll
            for (int c = 0; c < 2; ++c) {
                if (4 * c >= 4 + 2 * a.ry) continue;
                const int kap = kperm<C::E, C::KS>(qi);
                const T* krow = Kp + ((4 * wy + 4 * c + kap / 8) * kPlane + 4 * wx + kap % 8) * C::KSTR + C::E * g;
                f32x16 s = score_tile<C>(krow, qf[nb]);
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const int kr = kperm<C::E, C::KS>(acc_row(r, g));
                    const int ky = 4 * c + kr / 8, kx = kr % 8;  // within the wave footprint
                    const int dy = ky - qy, dx = kx - qx;
                    const int gy = Y0 + 4 * wy - a.ry + ky, gx = X0 + 4 * wx - a.rx + kx;
                    const bool ok = zok && (unsigned)dy <= (unsigned)(2 * a.ry) &&
                                    (unsigned)dx <= (unsigned)(2 * a.rx) && (unsigned)gy < (unsigned)a.Y &&
                                    (unsigned)gx < (unsigned)a.X && (unsigned)gz < (unsigned)a.Z;
                    if (!ok) s[r] = -INFINITY;
                }
                auto vload = [&](int mb, int ks) -> typename C::Frag {
                    const int ch = 32 * mb + qi;
                    const int k0 = ks * C::KS + C::E * g;
                    const T* p = Vp + min(ch, D - 1) * VPS + (4 * wy + 4 * c + k0 / 8) * kPlane + 4 * wx + k0 % 8;
                    typename C::Frag f = frag_load8<T>(p);
                    if (32 * mb + 32 > D && ch >= D) f = frag_fill<T>((C::ONES && ch == D) ? 1.f : 0.f);
                    return f;
                };
                soft_update<C>(st[nb], s, a.scale_log2, vload);
            }
        }
    }

    float ylocal[2][C::MB][16];
#pragma unroll
    for (int nb = 0; nb < 2; ++nb) {
        finish_local<C>(a, b, h, qrow[nb], qok[nb], g, st[nb], ylocal[nb]);
        st[nb].reset();
    }

    // ---- global pathway
    for (int base = 0; base < a.M; base += 64) {
        __syncthreads();
        stage_summaries<C>(a, bg, base, Ks, Vs, VGS);
        __syncthreads();
        global_stage<C>(a, base, Ks, Vs, VGS, qf, st, lane);
    }

#pragma unroll
    for (int nb = 0; nb < 2; ++nb) epilogue<C>(a, b, h, qrow[nb], qok[nb], g, st[nb], ylocal[nb]);
}

template <typename T, int D>
__global__ __launch_bounds__(64 * kWaves, 2) void k_attn_rows(AttnDev a) {
    typedef Cfg<T, D> C;
    constexpr int EP = Piece<T>::N;
    constexpr int VGS = 64 + EP;
    extern __shared__ __align__(16) unsigned char smem[];
    T* Ks = reinterpret_cast<T*>(smem);
    T* Vs = Ks + 64 * C::KSTR;

    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, g = lane >> 5, qi = lane & 31;
    const int bh = blockIdx.y, b = bh / a.H, h = bh % a.H, kvh = h / (a.H / a.G);
    const int64_t bg = (int64_t)b * a.G + kvh;

    typename C::Frag qf[2][C::NT];
    int64_t qrow[2];
    bool qok[2];
    float ylocal[2][C::MB][16];
#pragma unroll
    for (int nb = 0; nb < 2; ++nb) {
        const int64_t row = (int64_t)blockIdx.x * 64 * kWaves + 64 * wave + 32 * nb + qi;
        qok[nb] = row < a.N;
        qrow[nb] = qok[nb] ? row : 0;
        int64_t pos[3];
        rope_position(a.rope, qrow[nb], pos);
        load_q<C>(tp<T>(a.q) + b * a.qsb + h * a.qsh + qrow[nb] * a.qsn, qok[nb], a.rope, pos, g, qf[nb]);
        const float* ol = a.o_local_in + (((int64_t)b * a.H + h) * a.N + qrow[nb]) * D;
#pragma unroll
        for (int mb = 0; mb < C::MB; ++mb)
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                if (32 * mb + 8 * q >= D) continue;
                const int ch0 = acc_channel(mb, 4 * q, g);
#pragma unroll
                for (int i = 0; i < 4; ++i) ylocal[nb][mb][4 * q + i] = qok[nb] ? a.sl[ch0 + i] * ol[ch0 + i] : 0.f;
            }
    }

    Soft<C::MB> st[2];
    st[0].reset();
    st[1].reset();
    for (int base = 0; base < a.M; base += 64) {
        __syncthreads();
        stage_summaries<C>(a, bg, base, Ks, Vs, VGS);
        __syncthreads();
        global_stage<C>(a, base, Ks, Vs, VGS, qf, st, lane);
    }
#pragma unroll
    for (int nb = 0; nb < 2; ++nb) epilogue<C>(a, b, h, qrow[nb], qok[nb], g, st[nb], ylocal[nb]);
}

// Indexed local attention on VALU: one wave per (batch, head, query row);
// lanes own neighbour columns for the scores and channels for the output.
template <typename T>
__global__ __launch_bounds__(64) void k_local_indexed(AttnDev a, const int32_t* nb, int W, int D,
                                                     float* out, float scale) {
    __shared__ float qs[128];
    __shared__ float ps[128];
    __shared__ int ids[128];
    const int lane = threadIdx.x;
    const int64_t item = blockIdx.x;
    const int64_t row = item % a.N;
    const int64_t bh = item / a.N;
    const int b = (int)(bh / a.H), h = (int)(bh % a.H), kvh = h / (a.H / a.G);
    const T* q = tp<T>(a.q) + b * a.qsb + h * a.qsh + row * a.qsn;
    for (int c = lane; c < D; c += 64) qs[c] = to_f32(q[c]);
    float s[2];
    int idx[2];
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        const int w = lane + 64 * j;
        idx[j] = w < W ? nb[row * W + w] : -1;
        ids[w] = idx[j];
    }
    __syncthreads();
    const T* K = tp<T>(a.kl) + b * a.ksb + kvh * a.ksh;
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        s[j] = -INFINITY;
        if (idx[j] >= 0) {
            const T* k = K + idx[j] * a.ksn;
            float dot = 0.f;
            for (int c = 0; c < D; ++c) dot += qs[c] * to_f32(k[c]);
            s[j] = dot * scale;
        }
    }
    const float mx = wave_max(fmaxf(s[0], s[1]));
    const bool any = mx != -INFINITY;
    float e[2], tot;
#pragma unroll
    for (int j = 0; j < 2; ++j) e[j] = idx[j] >= 0 ? expf(s[j] - mx) : 0.f;
    tot = wave_sum(e[0] + e[1]);
#pragma unroll
    for (int j = 0; j < 2; ++j) ps[lane + 64 * j] = any ? e[j] / tot : 0.f;
    __syncthreads();
    const T* V = tp<T>(a.vl) + b * a.vsb + kvh * a.vsh;
    float* o = out + (bh * a.N + row) * D;
    for (int c = lane; c < D; c += 64) {
        float acc = 0.f;
        for (int w = 0; w < W; ++w) {
            const int t = ids[w];
            if (t >= 0) acc += ps[w] * to_f32(V[t * a.vsn + c]);
        }
        o[c] = acc;
    }
    if (a.lse_l && lane == 0) a.lse_l[bh * a.N + row] = any ? mx + __logf(tot) : -INFINITY;
}

int fill_dev(const p3d_attn_args& x, AttnDev& d) {
    const int es = dtype_size(x.dtype);
    P3D_REQUIRE(x.dtype >= P3D_F32 && x.dtype <= P3D_BF16, "unknown dtype");
    P3D_REQUIRE(x.batch >= 1 && x.heads >= 1 && x.kv_heads >= 1 && x.heads % x.kv_heads == 0 && x.tokens >= 1,
                "bad batch/head/token counts");
    P3D_REQUIRE(x.summaries >= 1, "need at least one summary");
    P3D_REQUIRE(view_ok(x.q, es) && view_ok(x.kl, es) && view_ok(x.vl, es) && view_ok(x.y, es),
                "q/k/v/y rows must be 16-byte aligned");
    P3D_REQUIRE(x.gate.data && x.local_scale && x.global_scale && x.sk && x.svt, "null pointer argument");
    P3D_REQUIRE(x.rope.table && x.rope.pairs && (x.rope.packed || x.rope.coords), "bad rope arguments");
    d = AttnDev{};
    d.B = x.batch, d.H = x.heads, d.G = x.kv_heads, d.N = x.tokens, d.M = x.summaries;
    d.Mp = (int)cdiv(x.summaries, 32) * 32;
    d.gate_dtype = x.gate_dtype;
    d.q = (const char*)x.q.data, d.qsb = x.q.sb, d.qsh = x.q.sh, d.qsn = x.q.sn;
    d.kl = (const char*)x.kl.data, d.ksb = x.kl.sb, d.ksh = x.kl.sh, d.ksn = x.kl.sn;
    d.vl = (const char*)x.vl.data, d.vsb = x.vl.sb, d.vsh = x.vl.sh, d.vsn = x.vl.sn;
    d.gate = (const char*)x.gate.data, d.gsb = x.gate.sb, d.gsh = x.gate.sh, d.gsn = x.gate.sn;
    d.sl = x.local_scale, d.sg = x.global_scale;
    d.sk = (const char*)x.sk, d.svt = (const char*)x.svt;
    d.rope = rope_dev(x.rope);
    d.map = x.raster_to_packed;
    d.o_local_in = x.o_local_in;
    d.y = (char*)x.y.data, d.ysb = x.y.sb, d.ysh = x.y.sh, d.ysn = x.y.sn;
    d.lse_l = x.lse_local, d.lse_g = x.lse_global;
    d.o_l = (char*)x.o_local, d.o_g = (char*)x.o_global;
    d.scale_log2 = kLog2e / sqrtf((float)x.head_dim);
    return P3D_OK;
}

template <int D>
size_t lds_grid(int es) {
    const int ep = 16 / es;
    const size_t plane = (size_t)kPlaneKeys * (D + ep) + (size_t)D * (kPlaneKeys + ep);
    const size_t stage = (size_t)64 * (D + ep) + (size_t)D * (64 + ep);
    return (plane > stage ? plane : stage) * es;
}

template <int D>
size_t lds_rows(int es) {
    const int ep = 16 / es;
    return ((size_t)64 * (D + ep) + (size_t)D * (64 + ep)) * es;
}

template <int D>
int launch_grid(const AttnDev& d, int dtype, dim3 grid, hipStream_t s) {
    const size_t smem = lds_grid<D>(dtype_size(dtype));
    switch (dtype) {
        case P3D_F32: k_attn_grid<float, D><<<grid, 64 * kWaves, smem, s>>>(d); break;
        case P3D_F16: k_attn_grid<_Float16, D><<<grid, 64 * kWaves, smem, s>>>(d); break;
        default: k_attn_grid<__bf16, D><<<grid, 64 * kWaves, smem, s>>>(d); break;
    }
    return check_launch("p3d_attn_fwd_grid");
}

template <int D>
int launch_rows(const AttnDev& d, int dtype, dim3 grid, hipStream_t s) {
    const size_t smem = lds_rows<D>(dtype_size(dtype));
    switch (dtype) {
        case P3D_F32: k_attn_rows<float, D><<<grid, 64 * kWaves, smem, s>>>(d); break;
        case P3D_F16: k_attn_rows<_Float16, D><<<grid, 64 * kWaves, smem, s>>>(d); break;
        default: k_attn_rows<__bf16, D><<<grid, 64 * kWaves, smem, s>>>(d); break;
    }
    return check_launch("p3d_attn_fwd_rows");
}

#define P3D_HEAD_DIMS(X) X(16) X(32) X(48) X(64) X(128)

}  // namespace
}  // namespace p3d

using namespace p3d;

extern "C" int p3d_attn_fwd_grid(const p3d_attn_args* args, void* stream) {
    P3D_REQUIRE(args, "null args");
    AttnDev d;
    int rc = fill_dev(*args, d);
    if (rc) return rc;
    for (int i = 0; i < 3; ++i) P3D_REQUIRE(args->radius[i] >= 0 && args->radius[i] <= 2, "grid kernel radius must be <= 2");
    P3D_REQUIRE((int64_t)args->grid[0] * args->grid[1] * args->grid[2] == args->tokens, "grid does not match tokens");
    d.Z = args->grid[0], d.Y = args->grid[1], d.X = args->grid[2];
    d.rz = args->radius[0], d.ry = args->radius[1], d.rx = args->radius[2];
    d.bricks_y = (int)cdiv(d.Y, 8), d.bricks_x = (int)cdiv(d.X, 8);
    const int64_t bricks = cdiv(d.Z, 4) * d.bricks_y * d.bricks_x;
    P3D_REQUIRE(bricks < (1LL << 31) && (int64_t)d.B * d.H < 65536, "launch grid too large");
    dim3 grid((unsigned)bricks, (unsigned)(d.B * d.H));
    hipStream_t s = as_stream(stream);
    switch (args->head_dim) {
#define CASE(DD) \
    case DD: return launch_grid<DD>(d, args->dtype, grid, s);
        P3D_HEAD_DIMS(CASE)
#undef CASE
        default: return fail(P3D_EUNSUPPORTED, "head_dim must be one of 16, 32, 48, 64, 128");
    }
}

extern "C" int p3d_attn_fwd_rows(const p3d_attn_args* args, void* stream) {
    P3D_REQUIRE(args, "null args");
    AttnDev d;
    int rc = fill_dev(*args, d);
    if (rc) return rc;
    P3D_REQUIRE(args->o_local_in, "rows kernel needs o_local_in");
    P3D_REQUIRE((int64_t)d.B * d.H < 65536, "launch grid too large");
    dim3 grid((unsigned)cdiv(d.N, 64 * kWaves), (unsigned)(d.B * d.H));
    hipStream_t s = as_stream(stream);
    switch (args->head_dim) {
#define CASE(DD) \
    case DD: return launch_rows<DD>(d, args->dtype, grid, s);
        P3D_HEAD_DIMS(CASE)
#undef CASE
        default: return fail(P3D_EUNSUPPORTED, "head_dim must be one of 16, 32, 48, 64, 128");
    }
}

extern "C" int p3d_local_fwd_indexed(const p3d_attn_args* args, const int32_t* neighbors, int32_t width,
                                     float* o_local, void* stream) {
    P3D_REQUIRE(args && neighbors && o_local, "null argument");
    AttnDev d;
    int rc = fill_dev(*args, d);
    if (rc) return rc;
    P3D_REQUIRE(width >= 1 && width <= 128, "width must be in [1, 128]");
    P3D_REQUIRE(args->head_dim <= 128, "head_dim must be <= 128");
    const int64_t items = (int64_t)d.B * d.H * d.N;
    P3D_REQUIRE(items < (1LL << 31), "too many rows");
    const float scale = 1.f / sqrtf((float)args->head_dim);
    hipStream_t s = as_stream(stream);
    switch (args->dtype) {
        case P3D_F32: k_local_indexed<float><<<(unsigned)items, 64, 0, s>>>(d, neighbors, width, args->head_dim, o_local, scale); break;
        case P3D_F16: k_local_indexed<_Float16><<<(unsigned)items, 64, 0, s>>>(d, neighbors, width, args->head_dim, o_local, scale); break;
        default: k_local_indexed<__bf16><<<(unsigned)items, 64, 0, s>>>(d, neighbors, width, args->head_dim, o_local, scale); break;
    }
    return check_launch("p3d_local_fwd_indexed");
}
