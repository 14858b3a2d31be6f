// Indexed local attention for any validated graph (reference.py:23-30 of
// amilworks/Pack3D): forward, dQ and dK/dV over the neighbour table and its
// reverse adjacency.  The reference's GPU kernels for the same math are
// kernels.py:43-66 (_local_fwd), :130-151 (_local_dq) and :154-181
// (_local_dkv).  Complete-grid layouts take the brick kernels instead; these
// serve every other geometry.
//
// Work layout.  A row slot is one (row, head) pair.  LPR consecutive lanes
// own a slot, each holding PPL 16-byte channel pieces of it (pieces p,
// p + LPR, ...), so a neighbour row is gathered as LPR contiguous 16-byte
// loads and a dot product is PPL * EP fused multiply-adds plus a log2(LPR)
// step DPP sum.  A wave holds 64 / LPR slots.  In the query kernels these are
// R heads of one kv group for 64 / (LPR R) consecutive rows, so a gathered
// key / value row serves R heads from one load instruction (the R slots read
// the same address).  Gathers are issued CE edges at a time: CE * PPL loads of
// each operand are in flight per lane before the first is used.
//
// Scores stay in fp32 (q pre-multiplied by log2(e)/sqrt(d), so the softmax
// runs in exp2 with a lazily moved running max); the backward computes dS
// in fp32 as the reference's indexed kernels do.
#include "attn_common.hpp"

namespace p3d {
namespace {

constexpr int kWaves = 4;
constexpr int kCE = 4;  // edges per gather batch
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;

template <typename T, int D>
struct GCfg {
    static constexpr int EP = Piece<T>::N;                 // elements per 16-byte piece
    static constexpr int NP = D / EP;                      // pieces per row
    static constexpr int PPL = (NP % 3 == 0) ? 3 : 2;      // pieces per lane
    static constexpr int LPR = NP / PPL;                   // lanes per row slot (power of two)
    static constexpr int SLOTS = 64 / LPR;                 // row slots per wave
    static constexpr int CH = PPL * EP;                    // channels per lane
    static_assert(NP % PPL == 0 && (LPR & (LPR - 1)) == 0 && LPR <= 16, "unsupported head_dim");
};

// Sum over the LPR lanes of a slot (quad_perm, row_half_mirror, row_mirror);
// every lane of the group ends with the same bits.
template <int LPR>
__device__ __forceinline__ float group_sum(float x) {
    if constexpr (LPR >= 2) x += dpp_move<0xB1>(x);
    if constexpr (LPR >= 4) x += dpp_move<0x4E>(x);
    if constexpr (LPR >= 8) x += dpp_move<0x141>(x);
    if constexpr (LPR >= 16) x += dpp_move<0x140>(x);
    return x;
}

template <typename T>
__device__ __forceinline__ uint4 load16(const T* p) { return *reinterpret_cast<const uint4*>(p); }

template <typename T>
__device__ __forceinline__ float elem(const uint4& raw, int e) { return to_f32(reinterpret_cast<const T*>(&raw)[e]); }

template <typename T>
__device__ __forceinline__ void store16(T* dst, const float* x) {
    uint4 raw;
    T* v = reinterpret_cast<T*>(&raw);
#pragma unroll
    for (int e = 0; e < Piece<T>::N; ++e) v[e] = from_f32<T>(x[e]);
    *reinterpret_cast<uint4*>(dst) = raw;
}

// Channel of element e of this lane's piece i.
template <typename C>
__device__ __forceinline__ int chan(int part, int i, int e) { return (part + C::LPR * i) * C::EP + e; }

template <typename T, typename C>
__device__ __forceinline__ float dot_pieces(const float (&x)[C::CH], const uint4 (&raw)[C::PPL]) {
    float s = 0.f;
#pragma unroll
    for (int i = 0; i < C::PPL; ++i)
#pragma unroll
        for (int e = 0; e < C::EP; ++e) s = fmaf(x[i * C::EP + e], elem<T>(raw[i], e), s);
    return s;
}

template <typename T, typename C>
__device__ __forceinline__ void axpy_pieces(float (&acc)[C::CH], float a, const uint4 (&raw)[C::PPL]) {
#pragma unroll
    for (int i = 0; i < C::PPL; ++i)
#pragma unroll
        for (int e = 0; e < C::EP; ++e) acc[i * C::EP + e] = fmaf(a, elem<T>(raw[i], e), acc[i * C::EP + e]);
}

template <typename T, typename C>
__device__ __forceinline__ void gather(const T* base, int64_t stride, int idx, int part, uint4 (&out)[C::PPL]) {
    const T* row = base + (int64_t)(idx < 0 ? 0 : idx) * stride;
#pragma unroll
    for (int i = 0; i < C::PPL; ++i) out[i] = load16(row + (part + C::LPR * i) * C::EP);
}

// Workgroups are dispatched round-robin over the 8 XCDs: give each XCD a
// contiguous run of row tiles, so that the neighbour rows its tiles gather
// overlap in its own L2 (5% faster at 64^3 radius 2 than the dispatch order).
__device__ __forceinline__ int xcd_run(int id, int count) {
    const int q = count / 8, r = count % 8;
    const int xcd = id % 8, slot = id / 8;
    return xcd < r ? xcd * (q + 1) + slot : r * (q + 1) + (xcd - r) * q + slot;
}

struct GDev {
    int B, H, G, N, W, R;
    const char *q, *kl, *vl;
    int64_t qsb, qsh, qsn, ksb, ksh, ksn, vsb, vsh, vsn;
    const int32_t* nb;  // [N, W] (query kernels) or the reverse table [N, W] (key kernel)
    RopeDev rope;       // forward: rotation of q on load
    const float* sl;
    char* y;
    int64_t ysb, ysh, ysn;
    char* o_l;       // forward, optional: [B,H,N,D] storage type
    float* lse_l;    // forward output (optional) / backward input: [B,H,N]
    const char* dol;      // backward: dO_L [B,H,N,D] storage type
    const float* delta;   // backward: Delta_L [B,H,N]
    float* dq;            // backward: [B,H,N,D] fp32
    float* dk;            // backward: [B,G,N,D] fp32
    char* dv;             // backward: view, storage type
    int64_t dvsb, dvsh, dvsn;
    float scale_log2;  // log2(e) / sqrt(D)
    float scale;       // 1 / sqrt(D)
};

// Slot of this lane in a query kernel: batch, head, row (or -1).
struct QSlot {
    int b, h, kvh, part;
    int64_t row;
    bool ok;
};

template <typename C>
__device__ __forceinline__ QSlot query_slot(const GDev& a) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int slot = lane / C::LPR;
    const int rep = a.H / a.G, groups = rep / a.R;
    const int by = blockIdx.y;
    const int b = by / (a.G * groups), rem = by - b * a.G * groups;
    const int g = rem / groups, hg = rem - g * groups;
    QSlot s;
    s.part = lane % C::LPR;
    s.b = b;
    s.kvh = g;
    s.h = g * rep + hg * a.R + slot % a.R;
    const int rows_per_wave = C::SLOTS / a.R;
    s.row = ((int64_t)xcd_run(blockIdx.x, gridDim.x) * kWaves + wave) * rows_per_wave + slot / a.R;
    s.ok = s.row < a.N;
    if (!s.ok) s.row = 0;
    return s;
}

// ------------------------------------------------------------------ forward
// y = sl * o_L in the storage type (the epilogue of the rows kernel adds the
// global branch), o_L and its log-sum-exp optionally saved for backward.
template <typename T, int D>
__global__ __launch_bounds__(64 * kWaves) void k_local_gather_fwd(GDev a) {
    typedef GCfg<T, D> C;
    const QSlot sl = query_slot<C>(a);
    float q[C::CH];
    {
        const T* qrow = reinterpret_cast<const T*>(a.q) + sl.b * a.qsb + sl.h * a.qsh + sl.row * a.qsn;
        int64_t pos[3];
        rope_position(a.rope, sl.row, pos);
#pragma unroll
        for (int i = 0; i < C::PPL; ++i) {
            const int c0 = chan<C>(sl.part, i, 0);
            const uint4 raw = load16(qrow + c0);
#pragma unroll
            for (int e = 0; e < C::EP; ++e) q[i * C::EP + e] = elem<T>(raw, e);
            rope_apply(a.rope, pos, c0, q + i * C::EP, C::EP);
        }
        // The rotated q is rounded to the storage type, as rope.py:48 returns
        // it and as the backward (which recomputes P from the saved log-sum-exp
        // on the rounded copy) sees it.
#pragma unroll
        for (int c = 0; c < C::CH; ++c) q[c] = to_f32(from_f32<T>(q[c])) * a.scale_log2;
    }
    const T* K = reinterpret_cast<const T*>(a.kl) + sl.b * a.ksb + sl.kvh * a.ksh;
    const T* V = reinterpret_cast<const T*>(a.vl) + sl.b * a.vsb + sl.kvh * a.vsh;
    const int32_t* nbr = a.nb + sl.row * a.W;
    float acc[C::CH];
#pragma unroll
    for (int c = 0; c < C::CH; ++c) acc[c] = 0.f;
    float m = -INFINITY, l = 0.f;
    for (int w0 = 0; w0 < a.W; w0 += kCE) {
        int idx[kCE];
        uint4 kr[kCE][C::PPL], vr[kCE][C::PPL];
#pragma unroll
        for (int e = 0; e < kCE; ++e) idx[e] = (sl.ok && w0 + e < a.W) ? nbr[w0 + e] : -1;
#pragma unroll
        for (int e = 0; e < kCE; ++e) gather<T, C>(K, a.ksn, idx[e], sl.part, kr[e]);
#pragma unroll
        for (int e = 0; e < kCE; ++e) gather<T, C>(V, a.vsn, idx[e], sl.part, vr[e]);
        float s[kCE];
        float mx = -INFINITY;
#pragma unroll
        for (int e = 0; e < kCE; ++e) {
            s[e] = group_sum<C::LPR>(dot_pieces<T, C>(q, kr[e]));
            s[e] = idx[e] >= 0 ? s[e] : -INFINITY;
            mx = fmaxf(mx, s[e]);
        }
        // The running max moves only when a batch exceeds it by 8 (log2
        // units): probabilities stay below 2^8, and the accumulator is rarely
        // rescaled.
        if (mx > m + 8.f || (m == -INFINITY && mx > -INFINITY)) {
            const float alpha = m == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(m - mx);
#pragma unroll
            for (int c = 0; c < C::CH; ++c) acc[c] *= alpha;
            l *= alpha;
            m = mx;
        }
        const float base = m == -INFINITY ? 0.f : m;
#pragma unroll
        for (int e = 0; e < kCE; ++e) {
            const float p = __builtin_amdgcn_exp2f(s[e] - base);
            l += p;
            axpy_pieces<T, C>(acc, p, vr[e]);
        }
    }
    if (!sl.ok) return;
    const float inv = l > 0.f ? 1.f / l : 0.f;  // an all-masked row gives 0
    const int64_t bh = (int64_t)sl.b * a.H + sl.h;
    T* y = reinterpret_cast<T*>(a.y) + sl.b * a.ysb + sl.h * a.ysh + sl.row * a.ysn;
    T* ol = a.o_l ? reinterpret_cast<T*>(a.o_l) + (bh * a.N + sl.row) * D : nullptr;
#pragma unroll
    for (int i = 0; i < C::PPL; ++i) {
        const int c0 = chan<C>(sl.part, i, 0);
        float o[C::EP], yl[C::EP];
#pragma unroll
        for (int e = 0; e < C::EP; ++e) {
            o[e] = acc[i * C::EP + e] * inv;
            yl[e] = a.sl[c0 + e] * o[e];
        }
        store16<T>(y + c0, yl);
        if (ol) store16<T>(ol + c0, o);
    }
    if (a.lse_l && sl.part == 0) a.lse_l[bh * a.N + sl.row] = l > 0.f ? m * kLn2 + __logf(l) : -INFINITY;
}

// ---------------------------------------------------------------- local dQ
// P = 2^(s log2(e)/sqrt(d) - lse log2(e)) from the saved log-sum-exp,
// dS = P (dO_L . v - Delta_L), dQ = sum dS k / sqrt(d).  q is rotated.
template <typename T, int D>
__global__ __launch_bounds__(64 * kWaves) void k_local_gather_dq(GDev a) {
    typedef GCfg<T, D> C;
    const QSlot sl = query_slot<C>(a);
    const int64_t bh = (int64_t)sl.b * a.H + sl.h;
    const int64_t qi = bh * a.N + sl.row;
    float q[C::CH], dox[C::CH];
    {
        const T* qrow = reinterpret_cast<const T*>(a.q) + sl.b * a.qsb + sl.h * a.qsh + sl.row * a.qsn;
        const T* drow = reinterpret_cast<const T*>(a.dol) + qi * D;
#pragma unroll
        for (int i = 0; i < C::PPL; ++i) {
            const int c0 = chan<C>(sl.part, i, 0);
            const uint4 rq = load16(qrow + c0), rd = load16(drow + c0);
#pragma unroll
            for (int e = 0; e < C::EP; ++e) {
                q[i * C::EP + e] = elem<T>(rq, e) * a.scale_log2;
                dox[i * C::EP + e] = elem<T>(rd, e);
            }
        }
    }
    const float lse = a.lse_l[qi];
    const bool live = sl.ok && lse != -INFINITY;  // an all-masked row has no local gradient
    const float lse2 = live ? lse * kLog2e : 0.f;
    const float delta = a.delta[qi];
    const T* K = reinterpret_cast<const T*>(a.kl) + sl.b * a.ksb + sl.kvh * a.ksh;
    const T* V = reinterpret_cast<const T*>(a.vl) + sl.b * a.vsb + sl.kvh * a.vsh;
    const int32_t* nbr = a.nb + sl.row * a.W;
    float acc[C::CH];
#pragma unroll
    for (int c = 0; c < C::CH; ++c) acc[c] = 0.f;
    for (int w0 = 0; w0 < a.W; w0 += kCE) {
        int idx[kCE];
        uint4 kr[kCE][C::PPL], vr[kCE][C::PPL];
#pragma unroll
        for (int e = 0; e < kCE; ++e) idx[e] = (live && w0 + e < a.W) ? nbr[w0 + e] : -1;
#pragma unroll
        for (int e = 0; e < kCE; ++e) gather<T, C>(K, a.ksn, idx[e], sl.part, kr[e]);
#pragma unroll
        for (int e = 0; e < kCE; ++e) gather<T, C>(V, a.vsn, idx[e], sl.part, vr[e]);
#pragma unroll
        for (int e = 0; e < kCE; ++e) {
            const float s = group_sum<C::LPR>(dot_pieces<T, C>(q, kr[e]));
            const float dp = group_sum<C::LPR>(dot_pieces<T, C>(dox, vr[e]));
            const float p = idx[e] >= 0 ? __builtin_amdgcn_exp2f(s - lse2) : 0.f;
            axpy_pieces<T, C>(acc, p * (dp - delta), kr[e]);
        }
    }
    if (!sl.ok) return;
    float* dq = a.dq + qi * D;
#pragma unroll
    for (int i = 0; i < C::PPL; ++i) {
        const int c0 = chan<C>(sl.part, i, 0);
        float o[C::EP];
#pragma unroll
        for (int e = 0; e < C::EP; ++e) o[e] = acc[i * C::EP + e] * a.scale;
#pragma unroll
        for (int e = 0; e < C::EP; e += 4)
            *reinterpret_cast<float4*>(dq + c0 + e) = float4{o[e], o[e + 1], o[e + 2], o[e + 3]};
    }
}

// ------------------------------------------------------------- local dK / dV
// One slot per (kv head, key row j); the queries listing j come from the
// reverse adjacency and every query head of the kv group contributes:
// dK_j = sum dS q / sqrt(d), dV_j = sum P dO_L.
template <typename T, int D>
__global__ __launch_bounds__(64 * kWaves) void k_local_gather_dkv(GDev a) {
    typedef GCfg<T, D> C;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int part = lane % C::LPR;
    const int bg = blockIdx.y, b = bg / a.G, g = bg - b * a.G, rep = a.H / a.G;
    int64_t row = ((int64_t)xcd_run(blockIdx.x, gridDim.x) * kWaves + wave) * C::SLOTS + lane / C::LPR;
    const bool ok = row < a.N;
    if (!ok) row = 0;
    float k[C::CH], v[C::CH];
    {
        const T* krow = reinterpret_cast<const T*>(a.kl) + b * a.ksb + g * a.ksh + row * a.ksn;
        const T* vrow = reinterpret_cast<const T*>(a.vl) + b * a.vsb + g * a.vsh + row * a.vsn;
#pragma unroll
        for (int i = 0; i < C::PPL; ++i) {
            const int c0 = chan<C>(part, i, 0);
            const uint4 rk = load16(krow + c0), rv = load16(vrow + c0);
#pragma unroll
            for (int e = 0; e < C::EP; ++e) {
                k[i * C::EP + e] = elem<T>(rk, e) * a.scale_log2;
                v[i * C::EP + e] = elem<T>(rv, e);
            }
        }
    }
    const int32_t* rv = a.nb + row * a.W;
    float dk[C::CH], dv[C::CH];
#pragma unroll
    for (int c = 0; c < C::CH; ++c) dk[c] = dv[c] = 0.f;
    for (int hh = 0; hh < rep; ++hh) {
        const int h = g * rep + hh;
        const int64_t bh = (int64_t)b * a.H + h;
        const T* Q = reinterpret_cast<const T*>(a.q) + b * a.qsb + h * a.qsh;
        const T* DO = reinterpret_cast<const T*>(a.dol) + bh * a.N * D;
        const float* LSE = a.lse_l + bh * a.N;
        const float* DL = a.delta + bh * a.N;
        for (int w0 = 0; w0 < a.W; w0 += kCE) {
            int idx[kCE];
            float l2[kCE], dl[kCE];
            uint4 qr[kCE][C::PPL], dr[kCE][C::PPL];
#pragma unroll
            for (int e = 0; e < kCE; ++e) idx[e] = (ok && w0 + e < a.W) ? rv[w0 + e] : -1;
#pragma unroll
            for (int e = 0; e < kCE; ++e) {
                const int i = idx[e] < 0 ? 0 : idx[e];
                const float lse = LSE[i];
                // All-masked rows and absent edges carry no gradient.
                l2[e] = (idx[e] < 0 || lse == -INFINITY) ? INFINITY : lse * kLog2e;
                dl[e] = DL[i];
            }
#pragma unroll
            for (int e = 0; e < kCE; ++e) gather<T, C>(Q, a.qsn, idx[e], part, qr[e]);
#pragma unroll
            for (int e = 0; e < kCE; ++e) gather<T, C>(DO, D, idx[e], part, dr[e]);
#pragma unroll
            for (int e = 0; e < kCE; ++e) {
                const float s = group_sum<C::LPR>(dot_pieces<T, C>(k, qr[e]));
                const float dp = group_sum<C::LPR>(dot_pieces<T, C>(v, dr[e]));
                const float p = __builtin_amdgcn_exp2f(s - l2[e]);
                axpy_pieces<T, C>(dk, p * (dp - dl[e]), qr[e]);
                axpy_pieces<T, C>(dv, p, dr[e]);
            }
        }
    }
    if (!ok) return;
    float* dko = a.dk + ((int64_t)bg * a.N + row) * D;
    T* dvo = reinterpret_cast<T*>(a.dv) + b * a.dvsb + g * a.dvsh + row * a.dvsn;
#pragma unroll
    for (int i = 0; i < C::PPL; ++i) {
        const int c0 = chan<C>(part, i, 0);
        float ko[C::EP], vo[C::EP];
#pragma unroll
        for (int e = 0; e < C::EP; ++e) {
            ko[e] = dk[i * C::EP + e] * a.scale;
            vo[e] = dv[i * C::EP + e];
        }
#pragma unroll
        for (int e = 0; e < C::EP; e += 4)
            *reinterpret_cast<float4*>(dko + c0 + e) = float4{ko[e], ko[e + 1], ko[e + 2], ko[e + 3]};
        store16<T>(dvo + c0, vo);
    }
}

// Heads of a kv group that share one wave's gathers: the largest power of
// two dividing H / G that fits the wave's slots.
int heads_per_group(int rep, int slots) {
    int r = 1;
    while (r * 2 <= slots && rep % (r * 2) == 0) r *= 2;
    return r;
}

// Query kernels (forward, dQ): grid x over row tiles, y over (batch, kv
// head, group of R heads).
template <typename T, int D, bool FWD>
int launch_query(GDev d, hipStream_t s) {
    typedef GCfg<T, D> C;
    d.R = heads_per_group(d.H / d.G, C::SLOTS);
    const int64_t rows_per_block = (int64_t)kWaves * (C::SLOTS / d.R);
    const int64_t gy = (int64_t)d.B * d.G * ((d.H / d.G) / d.R);
    if (gy > 65535) return fail(P3D_EUNSUPPORTED, "batch * heads exceeds the launch grid");
    const dim3 grid((unsigned)cdiv(d.N, rows_per_block), (unsigned)gy);
    if constexpr (FWD)
        k_local_gather_fwd<T, D><<<grid, 64 * kWaves, 0, s>>>(d);
    else
        k_local_gather_dq<T, D><<<grid, 64 * kWaves, 0, s>>>(d);
    return P3D_OK;
}

// Key kernel (dK, dV): grid x over row tiles, y over (batch, kv head).
template <typename T, int D>
int launch_key(GDev d, hipStream_t s) {
    typedef GCfg<T, D> C;
    if ((int64_t)d.B * d.G > 65535) return fail(P3D_EUNSUPPORTED, "batch * kv_heads exceeds the launch grid");
    const dim3 grid((unsigned)cdiv(d.N, (int64_t)kWaves * C::SLOTS), (unsigned)(d.B * d.G));
    k_local_gather_dkv<T, D><<<grid, 64 * kWaves, 0, s>>>(d);
    return P3D_OK;
}

enum class Pass { fwd, dq, dkv };

template <typename T, int D>
int launch_pass(Pass pass, const GDev& d, hipStream_t s) {
    switch (pass) {
        case Pass::fwd: return launch_query<T, D, true>(d, s);
        case Pass::dq: return launch_query<T, D, false>(d, s);
        default: return launch_key<T, D>(d, s);
    }
}

template <typename T>
int launch_head_dim(Pass pass, const GDev& d, int D, hipStream_t s) {
    switch (D) {
        case 16: return launch_pass<T, 16>(pass, d, s);
        case 32: return launch_pass<T, 32>(pass, d, s);
        case 48: return launch_pass<T, 48>(pass, d, s);
        case 64: return launch_pass<T, 64>(pass, d, s);
        case 128: return launch_pass<T, 128>(pass, d, s);
        default: return fail(P3D_EUNSUPPORTED, "head_dim must be one of 16, 32, 48, 64, 128");
    }
}

int launch(Pass pass, const GDev& d, int dtype, int D, hipStream_t s) {
    switch (dtype) {
        case P3D_F32: return launch_head_dim<float>(pass, d, D, s);
        case P3D_F16: return launch_head_dim<_Float16>(pass, d, D, s);
        default: return launch_head_dim<__bf16>(pass, d, D, s);
    }
}

bool head_dim_ok(int d) { return d == 16 || d == 32 || d == 48 || d == 64 || d == 128; }

}  // namespace
}  // namespace p3d

using namespace p3d;

extern "C" int p3d_local_fwd_indexed(const p3d_attn_args* args, const int32_t* neighbors, int32_t width,
                                     void* stream) {
    P3D_REQUIRE(args && neighbors, "null argument");
    const p3d_attn_args& x = *args;
    const int es = dtype_size(x.dtype);
    P3D_REQUIRE(x.dtype >= P3D_F32 && x.dtype <= P3D_BF16, "unknown dtype");
    P3D_REQUIRE(head_dim_ok(x.head_dim), "head_dim must be one of 16, 32, 48, 64, 128");
    P3D_REQUIRE(x.batch >= 1 && x.heads >= 1 && x.kv_heads >= 1 && x.heads % x.kv_heads == 0 && x.tokens >= 1,
                "bad batch/head/token counts");
    P3D_REQUIRE(width >= 1 && width <= 128, "width must be in [1, 128]");
    P3D_REQUIRE(view_ok(x.q, es) && view_ok(x.kl, es) && view_ok(x.vl, es) && view_ok(x.y, es),
                "q/k/v/y rows must be 16-byte aligned");
    P3D_REQUIRE(x.local_scale && x.rope.table && x.rope.pairs && (x.rope.packed || x.rope.coords),
                "null pointer argument");
    P3D_REQUIRE(!x.o_local || aligned16(x.o_local), "o_local must be 16-byte aligned");
    GDev d{};
    d.B = x.batch, d.H = x.heads, d.G = x.kv_heads, d.N = x.tokens, d.W = width;
    d.q = (const char*)x.q.data, d.qsb = x.q.sb, d.qsh = x.q.sh, d.qsn = x.q.sn;
    d.kl = (const char*)x.kl.data, d.ksb = x.kl.sb, d.ksh = x.kl.sh, d.ksn = x.kl.sn;
    d.vl = (const char*)x.vl.data, d.vsb = x.vl.sb, d.vsh = x.vl.sh, d.vsn = x.vl.sn;
    d.nb = neighbors;
    d.rope = rope_dev(x.rope);
    d.sl = x.local_scale;
    d.y = (char*)x.y.data, d.ysb = x.y.sb, d.ysh = x.y.sh, d.ysn = x.y.sn;
    d.o_l = (char*)x.o_local;
    d.lse_l = x.lse_local;
    d.scale_log2 = kLog2e / sqrtf((float)x.head_dim);
    d.scale = 1.f / sqrtf((float)x.head_dim);
    if (int rc = launch(Pass::fwd, d, x.dtype, x.head_dim, as_stream(stream))) return rc;
    return check_launch("p3d_local_fwd_indexed");
}

extern "C" int p3d_local_bwd_indexed(const p3d_bwd_args* args, const int32_t* neighbors, int32_t width,
                                     const int32_t* reverse, int32_t rwidth, void* stream) {
    P3D_REQUIRE(args, "null args");
    const p3d_bwd_args& x = *args;
    const int es = dtype_size(x.dtype);
    P3D_REQUIRE(x.dtype >= P3D_F32 && x.dtype <= P3D_BF16, "unknown dtype");
    P3D_REQUIRE(head_dim_ok(x.head_dim), "head_dim must be 16, 32, 48, 64 or 128");
    P3D_REQUIRE(x.batch >= 1 && x.heads >= 1 && x.kv_heads >= 1 && x.heads % x.kv_heads == 0 && x.tokens >= 1,
                "bad batch/head/token counts");
    P3D_REQUIRE(neighbors && reverse && width >= 1 && width <= 128 && rwidth >= 1 && rwidth <= 128,
                "neighbour tables must have 1..128 columns");
    P3D_REQUIRE(view_ok(x.q, es) && view_ok(x.kl, es) && view_ok(x.vl, es), "q/k/v rows must be 16-byte aligned");
    P3D_REQUIRE(x.dol && x.lse_local && x.delta_local && x.dq_local && x.dk_local && view_ok(x.dv_local, es),
                "null pointer argument or misaligned dv_local");
    P3D_REQUIRE(aligned16(x.dol) && aligned16(x.dq_local) && aligned16(x.dk_local), "misaligned gradient buffers");
    GDev d{};
    d.B = x.batch, d.H = x.heads, d.G = x.kv_heads, d.N = x.tokens;
    d.q = (const char*)x.q.data, d.qsb = x.q.sb, d.qsh = x.q.sh, d.qsn = x.q.sn;
    d.kl = (const char*)x.kl.data, d.ksb = x.kl.sb, d.ksh = x.kl.sh, d.ksn = x.kl.sn;
    d.vl = (const char*)x.vl.data, d.vsb = x.vl.sb, d.vsh = x.vl.sh, d.vsn = x.vl.sn;
    d.lse_l = const_cast<float*>(x.lse_local);
    d.dol = (const char*)x.dol;
    d.delta = x.delta_local;
    d.dq = x.dq_local;
    d.dk = x.dk_local;
    d.dv = (char*)x.dv_local.data, d.dvsb = x.dv_local.sb, d.dvsh = x.dv_local.sh, d.dvsn = x.dv_local.sn;
    d.scale_log2 = kLog2e / sqrtf((float)x.head_dim);
    d.scale = 1.f / sqrtf((float)x.head_dim);
    hipStream_t s = as_stream(stream);
    GDev dq = d;
    dq.nb = neighbors, dq.W = width;
    if (int rc = launch(Pass::dq, dq, x.dtype, x.head_dim, s)) return rc;
    GDev dkv = d;
    dkv.nb = reverse, dkv.W = rwidth;
    if (int rc = launch(Pass::dkv, dkv, x.dtype, x.head_dim, s)) return rc;
    return check_launch("p3d_local_bwd_indexed");
}
