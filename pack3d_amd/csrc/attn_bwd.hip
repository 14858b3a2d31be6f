// PACK3D core backward: the vector-Jacobian product of
// y = sl * o_L + gate * sg * o_G (reference.py:16-31 of amilworks/Pack3D),
// split into the same passes as the reference's GPU backward
// (backends/triton/kernels.py:106-356): the fusion step, local dQ, local
// dK/dV through the reverse adjacency, global dQ, and global dK/dV in query
// splits (reduced, with the pooling backward, in pool.hip).
//
// Rounding points follow the reference: dO_L = dy * sl and dO_G = dy * gate * sg
// are rounded to the storage type before Delta is formed (kernels.py:118-120),
// dS is rounded to the storage type before the global dQ / dK products, and
// dQ = round(round(dQ_L) + round(dQ_G)) (kernels.py:202-206), rotated back
// with R^T and rounded again (the rotation's own backward).
//
// All q / k inputs here are already rotated (the host rotates them once);
// summary keys are stored times log2(e)/sqrt(d) as in the forward.
#include <type_traits>

#include "attn_common.hpp"

namespace p3d {
namespace {

constexpr int kWaves = 4;
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;

struct BwdDev {
    int B, H, G, N, M, Mp;
    int gate_dtype, parts, splits;
    const char *q, *kl, *vl, *gate;
    int64_t qsb, qsh, qsn, ksb, ksh, ksn, vsb, vsh, vsn, gsb, gsh, gsn;
    const float *sl, *sg;
    const char *sk, *svt;
    float key_scale;
    const char *o_l, *o_g;
    const float *lse_l, *lse_g;
    const char* dy;
    int64_t dsb, dsh, dsn;
    char *dol, *dog;
    float *dl, *dg;
    char* dgate;
    float *dsl_part, *dsg_part;
    char *sv_rows, *skt;
    float *dq_l, *dq_g, *dk_l;
    char* dv_l;
    int64_t dvsb, dvsh, dvsn;
    float *dsk_part, *dsv_part;
    const char *q_t, *dog_t;  // optional: q and dO_G transposed, [B*H][D][N]
};

template <typename T>
__device__ __forceinline__ const T* tp(const char* p) { return reinterpret_cast<const T*>(p); }

template <typename T>
__device__ __forceinline__ void store_piece(T* dst, const float* x) {
    constexpr int N = Piece<T>::N;
    uint4 raw;
    T* v = reinterpret_cast<T*>(&raw);
#pragma unroll
    for (int e = 0; e < N; ++e) v[e] = from_f32<T>(x[e]);
    *reinterpret_cast<uint4*>(dst) = raw;
}

template <typename T>
__device__ __forceinline__ float round_to(float x) { return to_f32(from_f32<T>(x)); }

// ------------------------------------------------------------------- fusion
// dO_L, dO_G (rounded), Delta_L = sum dO_L o_L, Delta_G = sum dO_G o_G,
// dgate = sum dy sg o_G, and per-block partial sums of dsl = sum dy o_L and
// dsg = sum dy gate o_G (kernels.py:106-127).  LG lanes per row, one
// 16-byte piece per lane; blocks stride over the rows.
template <typename T, int D>
__global__ __launch_bounds__(256) void k_mix_bwd(BwdDev a) {
    constexpr int EP = Piece<T>::N, PPR = D / EP;
    constexpr int LG = PPR <= 2 ? 2 : (PPR <= 4 ? 4 : (PPR <= 8 ? 8 : (PPR <= 16 ? 16 : 32)));
    static_assert(PPR <= 32, "a row must fit in half a wave");
    constexpr int RPW = 64 / LG;
    __shared__ float red[2][kWaves][D];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int sub = lane % LG, grp = lane / LG;
    const bool act = sub < PPR;
    const int c0 = (act ? sub : 0) * EP;
    float sl[EP], sg[EP], psl[EP], psg[EP];
#pragma unroll
    for (int e = 0; e < EP; ++e) {
        sl[e] = a.sl[c0 + e];
        sg[e] = a.sg[c0 + e];
        psl[e] = psg[e] = 0.f;
    }
    const int64_t rows = (int64_t)a.B * a.H * a.N;
    const int64_t step = (int64_t)gridDim.x * kWaves * RPW;
    for (int64_t r = ((int64_t)blockIdx.x * kWaves + wave) * RPW + grp; r < rows; r += step) {
        const int64_t bh = r / a.N, n = r - bh * a.N;
        const int b = (int)(bh / a.H), h = (int)(bh - (int64_t)b * a.H);
        float dy[EP], ol[EP], og[EP];
        load_piece<T>(tp<T>(a.dy) + b * a.dsb + h * a.dsh + n * a.dsn + c0, dy);
        load_piece<T>(tp<T>(a.o_l) + r * D + c0, ol);
        load_piece<T>(tp<T>(a.o_g) + r * D + c0, og);
        const float gate = load_any(a.gate, b * a.gsb + h * a.gsh + n * a.gsn, a.gate_dtype);
        float dol[EP], dog[EP], sdl = 0.f, sdg = 0.f, sgt = 0.f;
#pragma unroll
        for (int e = 0; e < EP; ++e) {
            dol[e] = round_to<T>(dy[e] * sl[e]);
            dog[e] = round_to<T>(dy[e] * gate * sg[e]);
            sdl += dol[e] * ol[e];
            sdg += dog[e] * og[e];
            sgt += dy[e] * og[e] * sg[e];
            if (act) {
                psl[e] += dy[e] * ol[e];
                psg[e] += dy[e] * og[e] * gate;
            }
        }
        if (act) {
            store_piece<T>(reinterpret_cast<T*>(a.dol) + r * D + c0, dol);
            store_piece<T>(reinterpret_cast<T*>(a.dog) + r * D + c0, dog);
        }
        if (!act) sdl = sdg = sgt = 0.f;
#pragma unroll
        for (int o = 1; o < LG; o <<= 1) {
            sdl += __shfl_xor(sdl, o);
            sdg += __shfl_xor(sdg, o);
            sgt += __shfl_xor(sgt, o);
        }
        if (sub == 0) {
            a.dl[r] = sdl;
            a.dg[r] = sdg;
            switch (a.gate_dtype) {
                case P3D_F32: reinterpret_cast<float*>(a.dgate)[r] = sgt; break;
                case P3D_F16: reinterpret_cast<_Float16*>(a.dgate)[r] = (_Float16)sgt; break;
                default: reinterpret_cast<__bf16*>(a.dgate)[r] = (__bf16)sgt; break;
            }
        }
    }
    // Partial dsl / dsg of this block: over the row groups of each wave, then the waves.
#pragma unroll
    for (int o = LG; o < 64; o <<= 1)
#pragma unroll
        for (int e = 0; e < EP; ++e) {
            psl[e] += __shfl_xor(psl[e], o);
            psg[e] += __shfl_xor(psg[e], o);
        }
    if (grp == 0 && act)
#pragma unroll
        for (int e = 0; e < EP; ++e) {
            red[0][wave][c0 + e] = psl[e];
            red[1][wave][c0 + e] = psg[e];
        }
    __syncthreads();
    for (int c = threadIdx.x; c < D; c += blockDim.x) {
        float s0 = 0.f, s1 = 0.f;
#pragma unroll
        for (int w = 0; w < kWaves; ++w) {
            s0 += red[0][w][c];
            s1 += red[1][w][c];
        }
        a.dsl_part[(int64_t)blockIdx.x * D + c] = s0;
        a.dsg_part[(int64_t)blockIdx.x * D + c] = s1;
    }
}


// ------------------------------------------------------------ summaries
// sv rows [B,G,Mp,D] from svt, and skt [B,G,Mp/32,D,32] from sk (both the
// storage type; tiny).
template <typename T>
__global__ void k_summary_transpose(BwdDev a, int D) {
    const int64_t total = (int64_t)a.B * a.G * a.Mp * D;
    const int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (e >= total) return;
    const int c = (int)(e % D);
    const int64_t bm = e / D;  // bg * Mp + m
    const int m = (int)(bm % a.Mp);
    const int64_t bg = bm / a.Mp;
    const int64_t t_off = ((bg * (a.Mp / 32) + m / 32) * D + c) * 32 + (m & 31);
    reinterpret_cast<T*>(a.sv_rows)[e] = tp<T>(a.svt)[t_off];
    reinterpret_cast<T*>(a.skt)[t_off] = tp<T>(a.sk)[e];
}

// Layout of a stage of SK summaries (64, or 32 when two stages of 64 would
// not fit in LDS) for the global dQ pass: sk rows and sv rows (row stride
// KSTR) and sk transposed (row stride SK + EP, zero padding rows up to
// 32 * MB).  Double-buffered.
template <typename C, int SK>
struct DqStage {
    typedef typename C::T_ T;
    static constexpr int EP = Piece<T>::N;
    static constexpr int TGS = SK + EP;
    static constexpr int SIZE = 2 * SK * C::KSTR + 32 * C::MB * TGS;  // elements
};

// A dQ stage copied by the LDS DMA: sk rows, sv rows and sk^T in DqStage's
// layout, each copy covering whole padded rows (lanes on padding
// slots fetch a piece of the same row), the last copy of a region starting 64
// slots before its end, and sources clamped into the rows present.  Copies
// are split evenly over the waves (a wave with fewer repeats the last one).
template <typename C, int SK>
struct DqDma {
    typedef typename C::T_ T;
    typedef DqStage<C, SK> S;
    static constexpr int EP = Piece<T>::N;
    static constexpr int KROW = C::KSTR / EP, TROW = S::TGS / EP;  // 16-byte slots per padded row
    static constexpr int RSLOTS = SK * KROW, TSLOTS = C::D * TROW;
    static constexpr int RCH = (RSLOTS + 63) / 64, TCH = (TSLOTS + 63) / 64;
    static constexpr int CH = 2 * RCH + TCH, PER = (CH + kWaves - 1) / kWaves;
    static_assert(C::KSTR % EP == 0 && S::TGS % EP == 0 && RSLOTS >= 64 && TSLOTS >= 64, "stage layout");
    uint32_t off[PER];  // byte offset of this lane's source piece in the stage's block
    int wave;

    __device__ __forceinline__ static int chunk(int w, int i) { return min(w * PER + i, CH - 1); }
    __device__ __forceinline__ static int region(int c) { return c < RCH ? 0 : (c < 2 * RCH ? 1 : 2); }
    __device__ __forceinline__ static int first_slot(int c) {
        const int r = region(c);
        return r < 2 ? min(64 * (c - r * RCH), RSLOTS - 64) : min(64 * (c - 2 * RCH), TSLOTS - 64);
    }

    __device__ __forceinline__ DqDma() {
        wave = __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6);
        const int lane = threadIdx.x & 63;
#pragma unroll
        for (int i = 0; i < PER; ++i) {
            const int c = chunk(wave, i), slot = first_slot(c) + lane;
            int e;
            if (region(c) < 2) {
                const int row = slot / KROW, p = slot % KROW;
                e = row * C::D + (p < C::D / EP ? p : 0) * EP;
            } else {
                const int ch = slot / TROW, p = slot % TROW, dp = p < SK / EP ? p : 0;
                e = (dp / (32 / EP)) * C::D * 32 + ch * 32 + (dp % (32 / EP)) * EP;
            }
            off[i] = (uint32_t)e * sizeof(T);
        }
    }

    __device__ __forceinline__ void copy(const BwdDev& a, int64_t bg, int base, T* stage) const {
        const uint32_t last = (uint32_t)(min(SK, a.Mp - base) * C::D - EP) * sizeof(T);
        const int64_t e0 = ((int64_t)bg * a.Mp + base) * C::D;
        const uint32_t lds0 = lds_address(stage);
#pragma unroll
        for (int i = 0; i < PER; ++i) {
            const int c = chunk(wave, i), r = region(c);
            const T* src = r == 0 ? tp<T>(a.sk) + e0 : (r == 1 ? tp<T>(a.sv_rows) + e0 : tp<T>(a.skt) + e0);
            dma_copy16(src, min(off[i], last), lds0 + (uint32_t)(r * RSLOTS + first_slot(c)) * 16u);
        }
    }
};

// Stage depth: 64 rows when two stages fit in the 160 KiB of LDS, else 32.
template <typename C, template <typename, int> class Stage>
constexpr int stage_rows() {
    return 2 * Stage<C, 64>::SIZE * (int)sizeof(typename C::T_) <= 160 * 1024 ? 64 : 32;
}

// Zero rows [D, 32 * MB) of a transposed buffer (rows of `stride` elements).
template <typename C>
__device__ __forceinline__ void zero_padding_rows(typename C::T_* buf, int stride, int cols) {
    const int rows = 32 * C::MB - C::D;
    for (int i = threadIdx.x; i < rows * cols; i += blockDim.x) {
        const int r = i / cols, c = i - r * cols;
        buf[(C::D + r) * stride + c] = from_f32<typename C::T_>(0.f);
    }
}

// Fragments of one lane's row (query or key) for the score MFMAs, no rotation.
template <typename C>
__device__ __forceinline__ void load_row_frags(const typename C::T_* row, bool valid, int g, typename C::Frag* f) {
    typedef typename C::T_ T;
#pragma unroll
    for (int t = 0; t < C::NT; ++t) {
        if constexpr (C::E == 8) {
            f[t] = valid ? frag_load16<T>(row + t * C::KS + 8 * g) : frag_fill<T>(0.f);
        } else {
            f[t] = valid ? row[t * C::KS + g] : 0.f;
        }
    }
}

// Global dQ: per query, over all summaries, S = q . sk (log2 units), P =
// 2^(S - lse_G log2 e), dP = dO_G . sv, dS = P (dP - Delta_G), dQ = ln 2 *
// sum dS sk_stored (sk_stored = sk log2(e)/sqrt(d), so ln 2 * sk_stored =
// sk / sqrt(d)) (kernels.py:184-206).  Transposed tiles as in the forward:
// lane = query; dS feeds the dQ^T = sk^T dS^T MFMA as its B operand.
template <typename T, int D>
__global__ __launch_bounds__(64 * kWaves, 2) void k_global_dq(BwdDev a) {
    typedef Cfg<T, D> C;
    constexpr int SK = stage_rows<C, DqStage>();
    typedef DqStage<C, SK> S;
    extern __shared__ __align__(16) unsigned char smem[];
    T* lds = reinterpret_cast<T*>(smem);
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, g = lane >> 5, qi = lane & 31;
    const int bh = blockIdx.y, b = bh / a.H, h = bh % a.H, kvh = h / (a.H / a.G);
    const int64_t bg = (int64_t)b * a.G + kvh;

    typename C::Frag qf[2][C::NT], df[2][C::NT];
    int64_t qrow[2];
    bool qok[2];
    float lse2[2], delta[2];
#pragma unroll
    for (int nb = 0; nb < 2; ++nb) {
        const int64_t row = (int64_t)blockIdx.x * 64 * kWaves + 64 * wave + 32 * nb + qi;
        qok[nb] = row < a.N;
        qrow[nb] = qok[nb] ? row : 0;
        load_row_frags<C>(tp<T>(a.q) + b * a.qsb + h * a.qsh + qrow[nb] * a.qsn, qok[nb], g, qf[nb]);
        load_row_frags<C>(tp<T>(a.dog) + ((int64_t)bh * a.N + qrow[nb]) * D, qok[nb], g, df[nb]);
        lse2[nb] = qok[nb] ? a.lse_g[(int64_t)bh * a.N + qrow[nb]] * kLog2e : INFINITY;
        delta[nb] = qok[nb] ? a.dg[(int64_t)bh * a.N + qrow[nb]] : 0.f;
    }
    f32x16 acc[2][C::MB];
#pragma unroll
    for (int nb = 0; nb < 2; ++nb)
#pragma unroll
        for (int mb = 0; mb < C::MB; ++mb)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[nb][mb][r] = 0.f;

    zero_padding_rows<C>(lds + 2 * SK * C::KSTR, S::TGS, SK);
    zero_padding_rows<C>(lds + S::SIZE + 2 * SK * C::KSTR, S::TGS, SK);
    const DqDma<C, SK> dma;
    dma.copy(a, bg, 0, lds);

    // The wave's reference point m = the largest lse (log2 units) of its live
    // queries.  The score MFMAs start from -m (one 16-register accumulator
    // for both blocks), so 2^(s - m) <= 1, lse bounding every score of its
    // query, and P = 2^(s - m) c with c = 2^(m - lse) per query, which folds
    // into dP - Delta as one fma: dS = 2^(s - m) (c dP - c Delta), two VALU
    // operations and an exponential per score instead of three and one.
    // When a live query's lse lies more than 64 below m, terms that matter
    // could underflow, and the wave takes the per-query path instead.
    // Only 16-bit types up to head_dim 48 have the registers for both paths
    // (wider ones and fp32 keep the per-query path, which already fills them).
    constexpr bool kFast = sizeof(T) == 2 && D <= 48;
    float mw = 0.f, cq[2] = {0.f, 0.f}, cd[2] = {0.f, 0.f};
    bool fast = false;
    if constexpr (kFast) {
        mw = -INFINITY;
#pragma unroll
        for (int nb = 0; nb < 2; ++nb)
            if (qok[nb]) mw = fmaxf(mw, lse2[nb]);
        mw = wave_max(mw);
        if (mw == -INFINITY) mw = 0.f;  // no live query in the wave
        bool spread = false;
#pragma unroll
        for (int nb = 0; nb < 2; ++nb) spread |= qok[nb] && mw - lse2[nb] > 64.f;
        fast = __builtin_amdgcn_ballot_w64(spread) == 0;
#pragma unroll
        for (int nb = 0; nb < 2; ++nb) {
            cq[nb] = qok[nb] ? __builtin_amdgcn_exp2f(mw - lse2[nb]) : 0.f;
            cd[nb] = -cq[nb] * delta[nb];
        }
    }
    dma_wait();
    __syncthreads();

    // The stage loop, with dS formed as described above (FAST) or per query.
    auto sweep = [&](auto mode) __attribute__((always_inline)) {
        constexpr bool FAST = decltype(mode)::value;
        f32x16 minit;
#pragma unroll
        for (int r = 0; r < 16; ++r) minit[r] = -mw;
        int buf = 0;
        for (int base = 0; base < a.M; base += SK) {
            const int next = base + SK;
            // The other buffer held the previous stage, which every wave finished
            // before the last barrier.
            if (next < a.M) dma.copy(a, bg, next, lds + (buf ^ 1) * S::SIZE);
            const T* cur = lds + buf * S::SIZE;
#pragma unroll
            for (int tt = 0; tt < SK / 32; ++tt) {
                const int first = base + 32 * tt;
                if (first >= a.M) break;
                typename C::Frag kf[C::NT], vf[C::NT], tf[C::MB * C::KSTEPS];
                load_kfrags<C>(cur + (32 * tt + kperm<C::E, C::KS>(qi)) * C::KSTR + C::E * g, kf);
                load_kfrags<C>(cur + SK * C::KSTR + (32 * tt + kperm<C::E, C::KS>(qi)) * C::KSTR + C::E * g, vf);
                load_vfrags<C, true>(cur + 2 * SK * C::KSTR, S::TGS, 32 * tt, lane, tf);
#pragma unroll
                for (int nb = 0; nb < 2; ++nb) {
                    f32x16 s;
                    if constexpr (FAST)
                        s = score_tile<C>(kf, qf[nb], minit);
                    else
                        s = score_tile<C>(kf, qf[nb]);
                    const f32x16 dp = score_tile<C>(vf, df[nb]);
                    float ds[16];
#pragma unroll
                    for (int r = 0; r < 16; ++r) {
                        if constexpr (FAST)
                            ds[r] = __builtin_amdgcn_exp2f(s[r]) * fmaf(dp[r], cq[nb], cd[nb]);
                        else
                            ds[r] = __builtin_amdgcn_exp2f(s[r] - lse2[nb]) * (dp[r] - delta[nb]);
                    }
                    if (first + 32 > a.M) {  // the last tile: summaries past M contribute nothing
#pragma unroll
                        for (int r = 0; r < 16; ++r)
                            if (first + kperm<C::E, C::KS>(acc_row(r, g)) >= a.M) ds[r] = 0.f;
                    }
#pragma unroll
                    for (int ks = 0; ks < C::KSTEPS; ++ks) {
                        const typename C::Frag pf = frag_from_p<T>(ds, ks);
#pragma unroll
                        for (int mb = 0; mb < C::MB; ++mb)
                            acc[nb][mb] = C::M::mfma(tf[mb * C::KSTEPS + ks], pf, acc[nb][mb]);
                    }
                }
            }
            dma_wait();
            __syncthreads();
            buf ^= 1;
        }
    };
    if (kFast && fast) {
        if constexpr (kFast) sweep(std::true_type{});
    } else {
        sweep(std::false_type{});
    }
    // One summary: P = 1 and dS = 0 exactly (kernels.py:198-199), so dQ_G = 0.
    const float out_scale = a.M > 1 ? kLn2 : 0.f;
#pragma unroll
    for (int nb = 0; nb < 2; ++nb) {
        if (!qok[nb]) continue;
        float* dq = a.dq_g + ((int64_t)bh * a.N + qrow[nb]) * D;
#pragma unroll
        for (int mb = 0; mb < C::MB; ++mb)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int c = 32 * mb + acc_row(r, g);
                if (c < D) dq[c] = acc[nb][mb][r] * out_scale;
            }
    }
}

// Query stages of SK rows (64, or 32 when two stages of 64 would not fit in
// LDS) for the global dK/dV pass: q and dO_G rows (row stride KSTR), q and
// dO_G transposed (row stride SK + EP, zero padding rows), and -lse_G (log2
// units; -inf past the last query) and -Delta_G.  Each thread moves PI
// 16-byte pieces.
template <typename C, int SK, bool TDMA = false>
struct KvStage {
    typedef typename C::T_ T;
    static constexpr int EP = Piece<T>::N;
    static constexpr int PPR = C::D / EP;
    static constexpr int TGS = SK + EP;
    static constexpr int PIECES = SK * PPR;
    static constexpr int PI = (PIECES + 64 * kWaves - 1) / (64 * kWaves);
    static constexpr int ROWS = 2 * SK * C::KSTR;                 // q rows, dO rows
    static constexpr int TRANS = 2 * 32 * C::MB * TGS;            // q^T, dO^T
    static constexpr int SIZE = ROWS + TRANS + 2 * SK * (int)(sizeof(float) / sizeof(T));  // + lse, delta
    // 16-bit types: the transposed copies' 8-column groups are swizzled by row.
    static constexpr int MASK = sizeof(T) == 2 ? SK / 8 - 1 : 0;
    uint4 q[PI], d[PI];
    unsigned qb[PI], db[PI], lb;
    int qsn;
    float lse_raw = 0.f, delta_raw = 0.f;
    int lo = 0, hi = 0;

    // Row of piece i inside the stage (SK for a piece past the stage) and its column.
    static __device__ __forceinline__ int piece_row(int i) {
        const int p = threadIdx.x + i * 64 * kWaves;
        return p < PIECES ? p / PPR : SK;
    }
    static __device__ __forceinline__ int piece_col(int i) {
        const int p = threadIdx.x + i * 64 * kWaves;
        return (p - (p / PPR) * PPR) * EP;
    }

    // Byte offsets of the lane's pieces and of its lse / Delta entry inside a
    // stage, fixed for the kernel (32-bit: the host checks that SK rows of q
    // span less than 2^31 bytes).  Rows past max_row (only when the whole
    // query range is shorter than a stage) repeat row max_row.
    __device__ __forceinline__ void init(int64_t qsn_, int max_row) {
        qsn = (int)qsn_;
#pragma unroll
        for (int i = 0; i < PI; ++i) {
            const int r = min(piece_row(i), max_row);
            qb[i] = (unsigned)((r * (int)qsn + piece_col(i)) * (int)sizeof(T));
            db[i] = (unsigned)((r * C::D + piece_col(i)) * (int)sizeof(T));
        }
        lb = (unsigned)min((int)threadIdx.x, max_row) * 4u;
    }

    // Stage rows start at q (dO_G rows at dO, lse_G and Delta_G at ls, dl);
    // rows [lo, hi) of the stage are queries of this pass, the others repeat
    // queries and get lse = +inf in store(), so P = 0 and dS = 0 there.  The
    // loads use only scalar bases and the loop-invariant offsets: address
    // temporaries could be overwritten by the stage's MFMAs while the loads
    // are in flight, and arithmetic on the loaded values here would wait for
    // them, either of which stalls the compute behind this prefetch.
    __device__ __forceinline__ void load(const T* qs, const T* ds, const float* ls, const float* dl, int lo_,
                                         int hi_) {
        const uint32_t qbytes = (uint32_t)(((SK - 1) * qsn + C::D) * (int)sizeof(T));
        const __amdgpu_buffer_rsrc_t rq = buffer_rsrc(qs, qbytes);
        const __amdgpu_buffer_rsrc_t rd = buffer_rsrc(ds, SK * C::D * (uint32_t)sizeof(T));
#pragma unroll
        for (int i = 0; i < PI; ++i)
            if (PIECES % (64 * kWaves) == 0 || i + 1 < PI || piece_row(i) < SK) {
                q[i] = buffer_load16(rq, qb[i]);
                d[i] = buffer_load16(rd, db[i]);
            }
        if (threadIdx.x < SK) {
            lse_raw = buffer_load_f32(buffer_rsrc(ls, SK * 4), lb);
            delta_raw = buffer_load_f32(buffer_rsrc(dl, SK * 4), lb);
        }
        lo = lo_, hi = hi_;
    }

    __device__ __forceinline__ void store(T* stage) const {
        T* qt = stage + ROWS;
        T* dt = qt + 32 * C::MB * TGS;
#pragma unroll
        for (int i = 0; i < PI; ++i) {
            const int r = piece_row(i), c = piece_col(i);
            if (r < SK) {
                *reinterpret_cast<uint4*>(stage + r * C::KSTR + c) = q[i];
                *reinterpret_cast<uint4*>(stage + SK * C::KSTR + r * C::KSTR + c) = d[i];
                if constexpr (!TDMA) {
                    const T* qv = reinterpret_cast<const T*>(&q[i]);
                    const T* dv = reinterpret_cast<const T*>(&d[i]);
                    const int col = swz_col<MASK>(c, r);  // rows c .. c + EP - 1 share one group swizzle
#pragma unroll
                    for (int e = 0; e < EP; ++e) {
                        qt[(c + e) * TGS + col] = qv[e];
                        dt[(c + e) * TGS + col] = dv[e];
                    }
                }
            }
        }
        if (threadIdx.x < SK) {
            float* f = reinterpret_cast<float*>(stage + ROWS + TRANS);
            const bool live = (int)threadIdx.x >= lo && (int)threadIdx.x < hi;
            f[threadIdx.x] = live ? -lse_raw * kLog2e : -INFINITY;
            f[SK + threadIdx.x] = live ? -delta_raw : 0.f;
        }
    }
};

// The transposed query and dO_G regions of a dK/dV stage (16-bit types),
// copied by the LDS DMA from transposed copies in HBM ([B*H][D][N], one row
// of N queries per channel) instead of being written from the staged rows
// by 2-byte LDS stores.  A region row c (channel) holds the stage's SK
// queries in pieces of EP; physical piece P of row c holds logical query
// group P ^ swizzle(c) (the layout swz_col<MASK> gives the stores), piece
// SK / EP is padding (its lanes fetch group 0 again).  A copy writes 64
// consecutive pieces; the last copy of a region starts 64 pieces before the
// region's end.  Copies are split evenly over the waves (a wave with fewer
// repeats its last one).
template <typename C, int SK>
struct KvTransDma {
    typedef typename C::T_ T;
    typedef KvStage<C, SK, true> S;
    static constexpr int EP = Piece<T>::N;
    static constexpr int PR = S::TGS / EP;               // pieces per region row
    static constexpr int SLOTS = C::D * PR;
    static constexpr int CH = (SLOTS + 63) / 64;
    static constexpr int PER = (2 * CH + kWaves - 1) / kWaves;
    static_assert(S::TGS % EP == 0 && SLOTS >= 64 && sizeof(T) == 2, "transposed stage layout");
    uint32_t off[PER];  // byte offset of this lane's source piece from the stage's first query of channel 0
    int wave;

    __device__ __forceinline__ static int chunk(int w, int i) { return min(w * PER + i, 2 * CH - 1); }
    __device__ __forceinline__ static int first_slot(int c) { return min(64 * (c % CH), SLOTS - 64); }

    __device__ __forceinline__ KvTransDma(int n) {
        wave = __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6);
        const int lane = threadIdx.x & 63;
#pragma unroll
        for (int i = 0; i < PER; ++i) {
            const int slot = first_slot(chunk(wave, i)) + lane;
            const int row = slot / PR, pp = slot % PR;
            const int group = pp < SK / EP ? pp ^ ((row >> 3) & S::MASK) : 0;
            off[i] = (uint32_t)(row * n + group * EP) * sizeof(T);
        }
    }

    // Copy queries [bp, bp + SK) of head plane bh into the stage at `stage`.
    __device__ __forceinline__ void copy(const BwdDev& a, int64_t bh, int bp, T* stage) const {
        const int64_t e0 = bh * C::D * (int64_t)a.N + bp;
        const uint32_t lds0 = lds_address(stage + S::ROWS);
#pragma unroll
        for (int i = 0; i < PER; ++i) {
            const int c = chunk(wave, i), r = c / CH;
            const T* src = (r == 0 ? tp<T>(a.q_t) : tp<T>(a.dog_t)) + e0;
            dma_copy16(src, off[i], lds0 + (uint32_t)(r * 32 * C::MB * S::TGS) * sizeof(T) +
                                        (uint32_t)first_slot(c) * 16u);
        }
    }
};

// Global dK / dV of the summaries (kernels.py:209-237): lane = summary (a
// wave owns 32), queries streamed in stages of 64 over this split's range of
// every query head of the kv group.  S[q][key] = q . sk (log2 units) with the
// key fragments resident as the B operand; P = 2^(S - lse log2 e); dP = dO .
// sv; dS = P (dP - Delta); dK^T += q^T dS, dV^T += dO^T P (dS and P enter as
// B operands).  Writes fp32 partials [split][bg][m][D]; dK is in true units
// (divided by sqrt(d)), before the pooling's 1/count.
template <typename C, int SK>
using KvStageR = KvStage<C, SK>;

// Stand-in for KvTransDma where the transposed regions are staged from registers.
struct NoTransDma {
    __device__ __forceinline__ explicit NoTransDma(int) {}
};

// TDMA: the transposed regions come by LDS DMA from a.q_t / a.dog_t.
template <typename T, int D, bool TDMA>
__global__ __launch_bounds__(64 * kWaves, 2) void k_global_dkv(BwdDev a) {
    typedef Cfg<T, D> C;
    constexpr int SK = stage_rows<C, KvStageR>();
    typedef KvStage<C, SK, TDMA> S;
    extern __shared__ __align__(16) unsigned char smem[];
    T* lds = reinterpret_cast<T*>(smem);
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, g = lane >> 5, qi = lane & 31;
    const int split = blockIdx.y;
    const int64_t bg = blockIdx.z;
    const int b = (int)(bg / a.G), kvh = (int)(bg % a.G), rep = a.H / a.G;
    const int key = blockIdx.x * 32 * kWaves + 32 * wave + qi;
    const bool kok = key < a.M;

    typename C::Frag kf[C::NT], vf[C::NT];
    load_row_frags<C>(tp<T>(a.sk) + (bg * a.Mp + (kok ? key : 0)) * D, kok, g, kf);
    load_row_frags<C>(tp<T>(a.sv_rows) + (bg * a.Mp + (kok ? key : 0)) * D, kok, g, vf);
#pragma unroll
    for (int t = 0; t < C::NT; ++t) settle(kf[t]), settle(vf[t]);
    f32x16 acck[C::MB], accv[C::MB];
#pragma unroll
    for (int mb = 0; mb < C::MB; ++mb)
#pragma unroll
        for (int r = 0; r < 16; ++r) acck[mb][r] = accv[mb][r] = 0.f;

    // Queries per split, this split's range [q0, q1) and its stage count: block-
    // uniform values, kept in scalar registers (the divisions run on the VALU).
    const int per = __builtin_amdgcn_readfirstlane((int)cdiv(cdiv((int64_t)a.N, SK), a.splits) * SK);
    const int q0 = split * per, q1 = min(a.N, q0 + per);
    const int stages = __builtin_amdgcn_readfirstlane(q1 > q0 ? (q1 - q0 + SK - 1) / SK : 0);
    zero_padding_rows<C>(lds + S::ROWS, S::TGS, SK);
    zero_padding_rows<C>(lds + S::ROWS + 32 * C::MB * S::TGS, S::TGS, SK);
    zero_padding_rows<C>(lds + S::SIZE + S::ROWS, S::TGS, SK);
    zero_padding_rows<C>(lds + S::SIZE + S::ROWS + 32 * C::MB * S::TGS, S::TGS, SK);
    const int total = stages * rep;
    if (total > 0) {
        // Stage (h, qb): query head h of the group, queries [qb, min(qb + SK, q1)).
        // Its rows start at bp = min(qb, N - SK) (0 when N < SK), so every
        // stage reads SK existing rows at the same offsets; rows below qb - bp
        // belong to the stage before it and are masked.
        const int h0 = kvh * rep;
        const int64_t bh0 = (int64_t)b * a.H + h0;
        const T* q_head = tp<T>(a.q) + b * a.qsb + h0 * a.qsh;
        const T* do_head = tp<T>(a.dog) + bh0 * a.N * D;
        const float* ls_head = a.lse_g + bh0 * a.N;
        const float* dl_head = a.dg + bh0 * a.N;
        const int last = a.N >= SK ? a.N - SK : 0;
        auto load_stage = [&](S& regs, int qb) __attribute__((always_inline)) {
            const int bp = min(qb, last);
            regs.load(q_head + (int64_t)bp * a.qsn, do_head + (int64_t)bp * D, ls_head + bp, dl_head + bp, qb - bp,
                      min(SK, min(q1, a.N) - bp));
        };
        int nq = q0;
        int64_t tbh = bh0;  // head plane of the stage at nq, for the transposed copies
        S regs;
        regs.init(a.qsn, min(SK, a.N) - 1);
        load_stage(regs, nq);
        const std::conditional_t<TDMA, KvTransDma<C, SK>, NoTransDma> tdma(a.N);
        if constexpr (TDMA) tdma.copy(a, tbh, min(nq, last), lds);
        regs.store(lds);
        if constexpr (TDMA) dma_wait();
        __syncthreads();
        int buf = 0;
        for (int it = 0; it < total; ++it) {
            const bool more = it + 1 < total;
            nq += SK;
            if (nq >= q1) {
                nq = q0;
                q_head += a.qsh;
                do_head += (int64_t)a.N * D;
                ls_head += a.N;
                dl_head += a.N;
                ++tbh;
            }
            if (more) load_stage(regs, nq);
            // The other buffer held the previous stage, which every wave
            // finished before the last barrier.
            if constexpr (TDMA)
                if (more) tdma.copy(a, tbh, min(nq, last), lds + (buf ^ 1) * S::SIZE);
            const T* cur = lds + buf * S::SIZE;
            const float* nlse = reinterpret_cast<const float*>(cur + S::ROWS + S::TRANS);
            const float* ndlt = nlse + SK;
#pragma unroll
            for (int tt = 0; tt < SK / 32; ++tt) {
                typename C::Frag qa[C::NT], da[C::NT], qt[C::MB * C::KSTEPS], dt[C::MB * C::KSTEPS];
                load_kfrags<C>(cur + (32 * tt + kperm<C::E, C::KS>(qi)) * C::KSTR + C::E * g, qa);
                load_kfrags<C>(cur + SK * C::KSTR + (32 * tt + kperm<C::E, C::KS>(qi)) * C::KSTR + C::E * g, da);
                load_vfrags<C, true, S::MASK>(cur + S::ROWS, S::TGS, 32 * tt, lane, qt);
                load_vfrags<C, true, S::MASK>(cur + S::ROWS + 32 * C::MB * S::TGS, S::TGS, 32 * tt, lane, dt);
                // Register r of lane group g holds query kperm(acc_row(r, g)) of the tile.
                // The score accumulator starts at -lse (log2 units) and the dP one at -Delta.
                f32x16 init, dinit;
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const int qq = 32 * tt + kperm<C::E, C::KS>(acc_row(r, g));
                    init[r] = nlse[qq];
                    dinit[r] = ndlt[qq];
                }
                const f32x16 s = score_tile<C>(qa, kf, init);
                const f32x16 dpd = score_tile<C>(da, vf, dinit);  // dP - Delta
                float p[16], ds[16];
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    p[r] = __builtin_amdgcn_exp2f(s[r]);
                    ds[r] = p[r] * dpd[r];
                }
#pragma unroll
                for (int ks = 0; ks < C::KSTEPS; ++ks) {
                    const typename C::Frag dsf = frag_from_p<T>(ds, ks);
                    const typename C::Frag pf = frag_from_p<T>(p, ks);
#pragma unroll
                    for (int mb = 0; mb < C::MB; ++mb) {
                        acck[mb] = C::M::mfma(qt[mb * C::KSTEPS + ks], dsf, acck[mb]);
                        accv[mb] = C::M::mfma(dt[mb * C::KSTEPS + ks], pf, accv[mb]);
                    }
                }
            }
            if (more) regs.store(lds + (buf ^ 1) * S::SIZE);
            if constexpr (TDMA) dma_wait();
            __syncthreads();
            buf ^= 1;
        }
    }
    if (!kok) return;
    // One summary: dS = 0 exactly (kernels.py:230-233), so dK = 0.
    const float inv_sqrt_d = a.M > 1 ? 1.f / sqrtf((float)D) : 0.f;
    float* dk = a.dsk_part + (((int64_t)split * a.B * a.G + bg) * a.Mp + key) * D;
    float* dv = a.dsv_part + (((int64_t)split * a.B * a.G + bg) * a.Mp + key) * D;
#pragma unroll
    for (int mb = 0; mb < C::MB; ++mb)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const int c = 32 * mb + acc_row(r, g);
            if (c < D) {
                dk[c] = acck[mb][r] * inv_sqrt_d;
                dv[c] = accv[mb][r];
            }
        }
}

// ------------------------------------------------------------------ finish
// dQ = R^T round(round(dQ_L) + round(dQ_G)) and dK_L = R^T round(dK_L), each
// rounded to the storage type; one 16-byte output piece per thread.  Grid y
// walks the (batch, head) planes of dq and then those of dkl; grid x the
// pieces of a plane's rows.  The fp32 inputs are read 16 bytes at a time and
// the rotation's pair descriptors come from LDS.
template <typename T, int D>
__global__ __launch_bounds__(256) void k_finish_bwd(BwdDev a, RopeDev rope, int plane0, p3d_view dq, p3d_view dkl) {
    constexpr int EP = Piece<T>::N;
    constexpr int PPR = D / EP;  // pieces per row
    __shared__ int4 meta[D / 2];
    for (int j = threadIdx.x; j < D / 2; j += blockDim.x) meta[j] = pair_meta(rope.pairs, j);
    __syncthreads();
    // Plane p: (b, head) of dq for p < B*H, else (b, kv head) of dkl.  Rows
    // of a plane times its pieces fit in 31 bits (checked on the host).
    const int p = plane0 + (int)blockIdx.y;
    const int idx = (int)blockIdx.x * 256 + (int)threadIdx.x;
    if (idx >= a.N * PPR) return;
    const int n = idx / PPR, piece = idx - n * PPR;
    const bool isq = p < a.B * a.H;
    const int pp = isq ? p : p - a.B * a.H, heads = isq ? a.H : a.G;
    const int64_t off = (int64_t)pp * a.N * D + (int64_t)n * D + piece * EP;  // dense fp32 inputs
    float x[EP];
    if (isq) {
        const f32x4* l = reinterpret_cast<const f32x4*>(a.dq_l + off);
        const f32x4* g = reinterpret_cast<const f32x4*>(a.dq_g + off);
#pragma unroll
        for (int v = 0; v < EP / 4; ++v) {
            const f32x4 lv = l[v], gv = g[v];
#pragma unroll
            for (int i = 0; i < 4; ++i) x[4 * v + i] = round_to<T>(round_to<T>(lv[i]) + round_to<T>(gv[i]));
        }
    } else {
        const f32x4* l = reinterpret_cast<const f32x4*>(a.dk_l + off);
#pragma unroll
        for (int v = 0; v < EP / 4; ++v) {
            const f32x4 lv = l[v];
#pragma unroll
            for (int i = 0; i < 4; ++i) x[4 * v + i] = round_to<T>(lv[i]);
        }
    }
    int pos[3];
    rope_position32(rope, n, pos);
#pragma unroll
    for (int e = 0; e < EP; e += 2) {
        const int4 m = meta[(piece * EP + e) >> 1];
        const float2 cs = rope.table[m.x + m.y * pos[0] + m.z * pos[1] + m.w * pos[2]];
        rotate_pair(x[e], x[e + 1], cs.x, -cs.y);
    }
    const p3d_view& o = isq ? dq : dkl;
    const int b = pp / heads, h = pp - b * heads;
    store_piece<T>(reinterpret_cast<T*>(o.data) + b * o.sb + h * o.sh + (int64_t)n * o.sn + piece * EP, x);
}

// ------------------------------------------------------------ transpose
// dst[(b H + h) D + c][n] = src[b][h][n][c] for 16-bit rows (N a multiple
// of 8): a thread loads an 8-row x 8-channel block as eight 16-byte pieces,
// transposes it in registers and stores eight 16-byte pieces, one per
// channel.  Consecutive threads take consecutive channel pieces of a row
// group, so the loads are whole row spans.
struct TrDev {
    const uint16_t* src;
    int64_t sb, sh, sn;
    uint16_t* dst;
    int H, N, D;
};

__global__ __launch_bounds__(256) void k_transpose_rows(TrDev a) {
    const int cgs = a.D / 8;
    const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (idx >= (int64_t)(a.N / 8) * cgs) return;
    const int rg = (int)(idx / cgs), cg = (int)(idx - (int64_t)rg * cgs);
    const int bh = blockIdx.y, b = bh / a.H, h = bh - b * a.H;
    const uint16_t* src = a.src + b * a.sb + h * a.sh + (int64_t)(8 * rg) * a.sn + 8 * cg;
    uint16_t in[8][8];
#pragma unroll
    for (int r = 0; r < 8; ++r) *reinterpret_cast<uint4*>(in[r]) = *reinterpret_cast<const uint4*>(src + r * a.sn);
    uint16_t out[8][8];
#pragma unroll
    for (int c = 0; c < 8; ++c)
#pragma unroll
        for (int r = 0; r < 8; ++r) out[c][r] = in[r][c];
    uint16_t* dst = a.dst + ((int64_t)bh * a.D + 8 * cg) * a.N + 8 * rg;
#pragma unroll
    for (int c = 0; c < 8; ++c) *reinterpret_cast<uint4*>(dst + (int64_t)c * a.N) = *reinterpret_cast<const uint4*>(out[c]);
}

int fill_bwd(const p3d_bwd_args& x, BwdDev& d) {
    const int es = dtype_size(x.dtype);
    P3D_REQUIRE(x.dtype >= P3D_F32 && x.dtype <= P3D_BF16, "unknown dtype");
    P3D_REQUIRE(x.head_dim == 16 || x.head_dim == 32 || x.head_dim == 48 || x.head_dim == 64 || x.head_dim == 128,
                "head_dim must be 16, 32, 48, 64 or 128");
    P3D_REQUIRE(x.batch >= 1 && x.heads >= 1 && x.kv_heads >= 1 && x.heads % x.kv_heads == 0 && x.tokens >= 1,
                "bad batch/head/token counts");
    P3D_REQUIRE(x.summaries >= 1, "need at least one summary");
    P3D_REQUIRE(view_ok(x.q, es) && view_ok(x.kl, es) && view_ok(x.vl, es) && view_ok(x.dy, es),
                "q/k/v/dy rows must be 16-byte aligned");
    // The summary dK/dV stages address 64 query rows with 32-bit byte offsets.
    P3D_REQUIRE(x.q.sn >= 0 && x.q.sn < (int64_t)1 << 23, "q token stride must be below 2^23 elements");
    d = BwdDev{};
    d.B = x.batch, d.H = x.heads, d.G = x.kv_heads, d.N = x.tokens, d.M = x.summaries;
    d.Mp = (int)cdiv(x.summaries, 32) * 32;
    d.gate_dtype = x.gate_dtype, d.parts = x.parts, d.splits = x.splits;
    d.q = (const char*)x.q.data, d.qsb = x.q.sb, d.qsh = x.q.sh, d.qsn = x.q.sn;
    d.kl = (const char*)x.kl.data, d.ksb = x.kl.sb, d.ksh = x.kl.sh, d.ksn = x.kl.sn;
    d.vl = (const char*)x.vl.data, d.vsb = x.vl.sb, d.vsh = x.vl.sh, d.vsn = x.vl.sn;
    d.gate = (const char*)x.gate.data, d.gsb = x.gate.sb, d.gsh = x.gate.sh, d.gsn = x.gate.sn;
    d.sl = x.local_scale, d.sg = x.global_scale;
    d.sk = (const char*)x.sk, d.svt = (const char*)x.svt;
    d.key_scale = x.key_scale;
    d.o_l = (const char*)x.o_local, d.o_g = (const char*)x.o_global;
    d.lse_l = x.lse_local, d.lse_g = x.lse_global;
    d.dy = (const char*)x.dy.data, d.dsb = x.dy.sb, d.dsh = x.dy.sh, d.dsn = x.dy.sn;
    d.dol = (char*)x.dol, d.dog = (char*)x.dog;
    d.dl = x.delta_local, d.dg = x.delta_global;
    d.dgate = (char*)x.dgate;
    d.dsl_part = x.dsl_part, d.dsg_part = x.dsg_part;
    d.sv_rows = (char*)x.sv_rows, d.skt = (char*)x.skt;
    d.dq_l = x.dq_local, d.dq_g = x.dq_global, d.dk_l = x.dk_local;
    d.dv_l = (char*)x.dv_local.data, d.dvsb = x.dv_local.sb, d.dvsh = x.dv_local.sh, d.dvsn = x.dv_local.sn;
    d.dsk_part = x.dsk_part, d.dsv_part = x.dsv_part;
    d.q_t = (const char*)x.q_t, d.dog_t = (const char*)x.dog_t;
    return P3D_OK;
}

template <typename C>
size_t lds_dq() {
    return (size_t)2 * DqStage<C, stage_rows<C, DqStage>()>::SIZE * sizeof(typename C::T_);
}

template <typename C>
size_t lds_dkv() {
    return (size_t)2 * KvStage<C, stage_rows<C, KvStageR>()>::SIZE * sizeof(typename C::T_);
}

template <int D>
void launch_mix(const BwdDev& d, int dtype, hipStream_t s) {
    switch (dtype) {
        case P3D_F32: k_mix_bwd<float, D><<<d.parts, 64 * kWaves, 0, s>>>(d); break;
        case P3D_F16: k_mix_bwd<_Float16, D><<<d.parts, 64 * kWaves, 0, s>>>(d); break;
        default: k_mix_bwd<__bf16, D><<<d.parts, 64 * kWaves, 0, s>>>(d); break;
    }
}

template <int D>
void launch_dq(const BwdDev& d, int dtype, hipStream_t s) {
    const dim3 grid((unsigned)cdiv(d.N, 64 * kWaves), (unsigned)(d.B * d.H));
    switch (dtype) {
        case P3D_F32: k_global_dq<float, D><<<grid, 64 * kWaves, lds_dq<Cfg<float, D>>(), s>>>(d); break;
        case P3D_F16: k_global_dq<_Float16, D><<<grid, 64 * kWaves, lds_dq<Cfg<_Float16, D>>(), s>>>(d); break;
        default: k_global_dq<__bf16, D><<<grid, 64 * kWaves, lds_dq<Cfg<__bf16, D>>(), s>>>(d); break;
    }
}

template <int D>
void launch_dkv(const BwdDev& d, int dtype, hipStream_t s) {
    const dim3 grid((unsigned)cdiv(d.M, 32 * kWaves), (unsigned)d.splits, (unsigned)(d.B * d.G));
    // The transposed copies are used when given, for 16-bit types whose
    // stages are 64 queries that every stage's window holds (N >= 64, and N
    // a multiple of 8 so that every window starts on a 16-byte piece).
    const bool tdma = d.q_t && d.dog_t && dtype != P3D_F32 && d.N >= 64 && d.N % 8 == 0;
    switch (dtype) {
        case P3D_F32: k_global_dkv<float, D, false><<<grid, 64 * kWaves, lds_dkv<Cfg<float, D>>(), s>>>(d); break;
        case P3D_F16:
            if (tdma)
                k_global_dkv<_Float16, D, true><<<grid, 64 * kWaves, lds_dkv<Cfg<_Float16, D>>(), s>>>(d);
            else
                k_global_dkv<_Float16, D, false><<<grid, 64 * kWaves, lds_dkv<Cfg<_Float16, D>>(), s>>>(d);
            break;
        default:
            if (tdma)
                k_global_dkv<__bf16, D, true><<<grid, 64 * kWaves, lds_dkv<Cfg<__bf16, D>>(), s>>>(d);
            else
                k_global_dkv<__bf16, D, false><<<grid, 64 * kWaves, lds_dkv<Cfg<__bf16, D>>(), s>>>(d);
            break;
    }
}

#define P3D_BWD_DISPATCH(FN, D_, ...)                      \
    switch (D_) {                                          \
        case 16: FN<16>(__VA_ARGS__); break;               \
        case 32: FN<32>(__VA_ARGS__); break;               \
        case 48: FN<48>(__VA_ARGS__); break;               \
        case 64: FN<64>(__VA_ARGS__); break;               \
        default: FN<128>(__VA_ARGS__); break;              \
    }

}  // namespace
}  // namespace p3d

using namespace p3d;

extern "C" int p3d_mix_bwd(const p3d_bwd_args* args, void* stream) {
    P3D_REQUIRE(args, "null args");
    BwdDev d;
    if (int rc = fill_bwd(*args, d)) return rc;
    P3D_REQUIRE(args->parts >= 1, "parts must be positive");
    P3D_REQUIRE(args->o_local && args->o_global && args->gate.data && args->local_scale && args->global_scale &&
                    args->dol && args->dog && args->delta_local && args->delta_global && args->dgate &&
                    args->dsl_part && args->dsg_part,
                "null pointer argument");
    P3D_BWD_DISPATCH(launch_mix, args->head_dim, d, args->dtype, as_stream(stream));
    return check_launch("p3d_mix_bwd");
}


namespace {
int global_bwd_args(const p3d_bwd_args* args, BwdDev& d) {
    P3D_REQUIRE(args, "null args");
    if (int rc = fill_bwd(*args, d)) return rc;
    P3D_REQUIRE(args->splits >= 1, "splits must be positive");
    P3D_REQUIRE(args->sk && args->svt && args->sv_rows && args->skt && args->dog && args->lse_global &&
                    args->delta_global && args->dq_global && args->dsk_part && args->dsv_part,
                "null pointer argument");
    return P3D_OK;
}
}  // namespace

extern "C" int p3d_global_bwd_dq(const p3d_bwd_args* args, void* stream) {
    BwdDev d;
    if (int rc = global_bwd_args(args, d)) return rc;
    hipStream_t s = as_stream(stream);
    const int64_t te = (int64_t)d.B * d.G * d.Mp * args->head_dim;
    switch (args->dtype) {
        case P3D_F32: k_summary_transpose<float><<<(unsigned)cdiv(te, 256), 256, 0, s>>>(d, args->head_dim); break;
        case P3D_F16: k_summary_transpose<_Float16><<<(unsigned)cdiv(te, 256), 256, 0, s>>>(d, args->head_dim); break;
        default: k_summary_transpose<__bf16><<<(unsigned)cdiv(te, 256), 256, 0, s>>>(d, args->head_dim); break;
    }
    P3D_BWD_DISPATCH(launch_dq, args->head_dim, d, args->dtype, s);
    return check_launch("p3d_global_bwd_dq");
}

extern "C" int p3d_global_bwd_dkv(const p3d_bwd_args* args, void* stream) {
    BwdDev d;
    if (int rc = global_bwd_args(args, d)) return rc;
    P3D_BWD_DISPATCH(launch_dkv, args->head_dim, d, args->dtype, as_stream(stream));
    return check_launch("p3d_global_bwd_dkv");
}

extern "C" int p3d_global_bwd(const p3d_bwd_args* args, void* stream) {
    if (int rc = p3d_global_bwd_dq(args, stream)) return rc;
    return p3d_global_bwd_dkv(args, stream);
}

template <typename T, int D>
void launch_finish(const BwdDev& d, const RopeDev& r, const p3d_view& dq, const p3d_view& dkl, hipStream_t s) {
    constexpr int PPR = D / Piece<T>::N;
    const unsigned bx = (unsigned)cdiv((int64_t)d.N * PPR, 256);
    const int planes = d.B * (d.H + d.G);
    for (int p0 = 0; p0 < planes; p0 += 65535) {
        const unsigned by = (unsigned)(planes - p0 < 65535 ? planes - p0 : 65535);
        k_finish_bwd<T, D><<<dim3(bx, by), 256, 0, s>>>(d, r, p0, dq, dkl);
    }
}

template <typename T>
void dispatch_finish(const BwdDev& d, const RopeDev& r, int head_dim, const p3d_view& dq, const p3d_view& dkl,
                     hipStream_t s) {
    switch (head_dim) {
        case 16: launch_finish<T, 16>(d, r, dq, dkl, s); break;
        case 32: launch_finish<T, 32>(d, r, dq, dkl, s); break;
        case 48: launch_finish<T, 48>(d, r, dq, dkl, s); break;
        case 64: launch_finish<T, 64>(d, r, dq, dkl, s); break;
        default: launch_finish<T, 128>(d, r, dq, dkl, s); break;
    }
}

extern "C" int p3d_finish_bwd(const p3d_bwd_args* args, const p3d_rope* rope, p3d_view dq, p3d_view dkl,
                              void* stream) {
    P3D_REQUIRE(args && rope, "null argument");
    BwdDev d;
    if (int rc = fill_bwd(*args, d)) return rc;
    P3D_REQUIRE(args->dq_local && args->dq_global && args->dk_local, "null pointer argument");
    P3D_REQUIRE(rope->table && rope->pairs && (rope->packed || rope->coords), "bad rope arguments");
    const int ep = 16 / dtype_size(args->dtype);
    P3D_REQUIRE((int64_t)d.N * (args->head_dim / ep) < ((int64_t)1 << 31), "tokens * pieces per row must be below 2^31");
    P3D_REQUIRE(view_ok(dq, dtype_size(args->dtype)) && view_ok(dkl, dtype_size(args->dtype)),
                "dq / dkl rows must be 16-byte aligned");
    hipStream_t s = as_stream(stream);
    const RopeDev r = rope_dev(*rope);
    switch (args->dtype) {
        case P3D_F32: dispatch_finish<float>(d, r, args->head_dim, dq, dkl, s); break;
        case P3D_F16: dispatch_finish<_Float16>(d, r, args->head_dim, dq, dkl, s); break;
        default: dispatch_finish<__bf16>(d, r, args->head_dim, dq, dkl, s); break;
    }
    return check_launch("p3d_finish_bwd");
}

extern "C" int p3d_transpose_rows(p3d_view src, void* dst, int32_t batch, int32_t heads, int32_t tokens,
                                  int32_t head_dim, int32_t dtype, void* stream) {
    P3D_REQUIRE(src.data && dst, "null pointer argument");
    P3D_REQUIRE(dtype == P3D_F16 || dtype == P3D_BF16, "dtype must be fp16 or bf16");
    P3D_REQUIRE(batch >= 1 && heads >= 1 && tokens >= 8 && tokens % 8 == 0, "tokens must be a multiple of 8");
    P3D_REQUIRE(head_dim >= 8 && head_dim % 8 == 0, "head_dim must be a multiple of 8");
    P3D_REQUIRE(view_ok(src, 2), "src rows must be 16-byte aligned");
    P3D_REQUIRE(aligned16(dst), "dst must be 16-byte aligned");
    P3D_REQUIRE((int64_t)batch * heads <= 65535, "batch * heads exceeds the launch grid");
    TrDev d;
    d.src = (const uint16_t*)src.data, d.sb = src.sb, d.sh = src.sh, d.sn = src.sn;
    d.dst = (uint16_t*)dst, d.H = heads, d.N = tokens, d.D = head_dim;
    const int64_t items = (int64_t)(tokens / 8) * (head_dim / 8);
    k_transpose_rows<<<dim3((unsigned)cdiv(items, 256), (unsigned)(batch * heads)), 256, 0, as_stream(stream)>>>(d);
    return check_launch("p3d_transpose_rows");
}
