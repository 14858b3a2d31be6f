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
// for 64 packed rows per wave, with the local branch read from y (written by
// the indexed local kernel) or from an fp32 buffer.
#include "attn_common.hpp"

namespace p3d {
namespace {

constexpr int kWaves = 4;      // brick kernel: one 4 x 8 x 8 brick per workgroup
constexpr int kRowsWaves = 4;  // rows kernel: 256 query rows per workgroup (8 waves measured slower)
constexpr int kPlane = 12;                 // plane side for radius <= 2 and an 8 x 8 brick face
constexpr int kPlaneKeys = kPlane * kPlane;
// LDS bytes of the rotation window: (cos, sin) for 64 pairs x 12 positions, then 64 axis ids.
constexpr int kRopeWindowBytes = 64 * kPlane * 8 + 256;
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
    const float* sk_norm_max;
    RopeDev rope;
    const int32_t* map;
    const float* o_local_in;
    char* y;
    int64_t ysb, ysh, ysn;
    float *lse_l, *lse_g;
    char *o_l, *o_g;
    float scale_log2;  // log2(e) / sqrt(D)
    int kl_rotated;    // kl already rotated: the grid kernel rotates q only
};

template <typename T>
__device__ __forceinline__ const T* tp(const char* p) { return reinterpret_cast<const T*>(p); }

// Load and rotate this lane's query channels into score-MFMA B fragments;
// rot(j) returns (cos, sin) of rotary pair j for this query.
template <typename C, typename Rot>
__device__ __forceinline__ void load_q(const typename C::T_* row, bool valid, Rot rot, int g,
                                       typename C::Frag* qf) {
    typedef typename C::T_ T;
#pragma unroll
    for (int t = 0; t < C::NT; ++t) {
        if constexpr (C::E == 8) {
            float x[8];
            const int c0 = t * C::KS + 8 * g;
            if (valid) {
                load_piece<T>(row + c0, x);
#pragma unroll
                for (int e = 0; e < 8; e += 2) {
                    const float2 cs = rot((c0 + e) >> 1);
                    rotate_pair(x[e], x[e + 1], cs.x, cs.y);
                }
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
                const float2 cs = rot(c0 >> 1);
                rotate_pair(x[0], x[1], cs.x, cs.y);
            }
            qf[t] = x[g];
        }
    }
}

// ---------------------------------------------------------------- summaries
// Summary stages of 64 keys, copied by the LDS DMA (global_load_lds_dwordx4):
// the pieces go from L2 straight into LDS, with no registers to hold them and
// no LDS store instructions.  One copy writes 64 consecutive 16-byte pieces
// of LDS, lane i the piece at M0 + 16 i, from a global address of the lane's
// choosing.  A stage holds K rows (natural order, row stride KSTR) and V
// transposed (rows of VGS): one contiguous block of sk ([64][D]) and one of
// svt ([2][D][32]).  A copy spans whole padded rows, its lanes on padding
// slots fetch a piece of the same row (finite, never read), and the last copy
// of each region starts 64 pieces before the region's end, so it rewrites its
// predecessor's tail with the same data instead of running into the V^T
// padding rows (the ones row and zeros, written once).  Copies are split evenly over the waves; a wave with fewer
// repeats the last copy, so every wave issues the same instructions.
// Completion is tracked by the vector-memory counter (dma_wait).
template <typename C, int WG>
struct StageDma {
    typedef typename C::T_ T;
    static constexpr int EP = Piece<T>::N;
    static constexpr int VGS = 64 + EP;
    static constexpr int KROW = C::KSTR / EP, VROW = VGS / EP;  // pieces per padded row
    static constexpr int KPIECES = 64 * KROW, VPIECES = C::D * VROW;
    static constexpr int KCH = (KPIECES + 63) / 64, VCH = (VPIECES + 63) / 64;
    static constexpr int CH = KCH + VCH, WAVES = WG / 64, PER = (CH + WAVES - 1) / WAVES;
    static_assert(C::KSTR % EP == 0 && VGS % EP == 0 && KPIECES >= 64 && VPIECES >= 64, "stage layout");
    uint32_t off[PER];  // byte offset of this lane's source piece in the stage's sk / svt block
    int wave;

    __device__ __forceinline__ static int chunk(int w, int i) { return min(w * PER + i, CH - 1); }
    // First piece of copy c within its region (K rows, or the data rows of V^T).
    __device__ __forceinline__ static int first_piece(int c) {
        return c < KCH ? min(64 * c, KPIECES - 64) : min(64 * (c - KCH), VPIECES - 64);
    }

    __device__ __forceinline__ StageDma() {
        wave = __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6);
        const int lane = threadIdx.x & 63;
#pragma unroll
        for (int i = 0; i < PER; ++i) {
            const int c = chunk(wave, i), slot = first_piece(c) + lane;
            int e;
            if (c < KCH) {
                const int row = slot / KROW, p = slot % KROW;
                e = row * C::D + (p < C::D / EP ? p : 0) * EP;
            } else {
                const int ch = slot / VROW, p = slot % VROW, dp = p < 64 / EP ? p : 0;
                e = (dp / (32 / EP)) * C::D * 32 + ch * 32 + (dp % (32 / EP)) * EP;
            }
            off[i] = (uint32_t)e * sizeof(T);
        }
    }

    // Copy stage [base, base + 64) into `stage`.  Source offsets are clamped
    // into the rows present, so every lane reads this (b, g)'s summaries.
    __device__ __forceinline__ void copy(const AttnDev& a, int64_t bg, int base, T* stage) const {
        const uint32_t last = (uint32_t)(min(64, a.Mp - base) * C::D - EP) * sizeof(T);
        const T* sk = tp<T>(a.sk) + ((int64_t)bg * a.Mp + base) * C::D;
        const T* svt = tp<T>(a.svt) + ((int64_t)bg * a.Mp + base) * C::D;
        const uint32_t lds0 = lds_address(stage);
#pragma unroll
        for (int i = 0; i < PER; ++i) {
            const int c = chunk(wave, i);
            const uint32_t m0 = lds0 + (uint32_t)(c < KCH ? first_piece(c) : KPIECES + first_piece(c)) * 16u;
            const T* src = c < KCH ? sk : svt;
            dma_copy16(src, min(off[i], last), m0);
        }
    }
};

// One summary stage (two 32-key tiles) on this wave's two column blocks.
template <typename C, bool BOUND>
__device__ __forceinline__ void global_stage(const AttnDev& a, int base, const typename C::T_* Ks,
                                             const typename C::T_* Vs, int vstride,
                                             const typename C::Frag (*qf)[C::NT], Soft<C::MB>* st,
                                             const f32x16* negm, int lane) {
    typedef typename C::T_ T;
    const int g = lane >> 5, qi = lane & 31;
#pragma unroll
    for (int tt = 0; tt < 2; ++tt) {
        const int first = base + 32 * tt;
        if (first >= a.M) break;
        typename C::Frag kf[C::NT], vf[C::MB * C::KSTEPS];
        load_kfrags<C>(Ks + (32 * tt + kperm<C::E, C::KS>(qi)) * C::KSTR + C::E * g, kf);
        load_vfrags<C, true>(Vs, vstride, 32 * tt, lane, vf);
        f32x16 s[2];
#pragma unroll
        for (int nb = 0; nb < 2; ++nb) s[nb] = BOUND ? score_tile<C>(kf, qf[nb], negm[nb]) : score_tile<C>(kf, qf[nb]);
        if (first + 32 > a.M) {
#pragma unroll
            for (int nb = 0; nb < 2; ++nb)
#pragma unroll
                for (int r = 0; r < 16; ++r)
                    if (first + kperm<C::E, C::KS>(acc_row(r, g)) >= a.M) s[nb][r] = -INFINITY;
        }
#pragma unroll
        for (int nb = 0; nb < 2; ++nb) {
            float p[16];
            if constexpr (BOUND)
                soft_probs_bounded<C>(st[nb], s[nb], p);
            else
                soft_probs<C>(st[nb], s[nb], 1.f, p);  // summary keys carry the log2(e)/sqrt(d) scale
            soft_accumulate<C>(st[nb], p, vf);
        }
    }
}

// All M summaries streamed through a double-buffered LDS region at `lds`.
template <typename C, bool BOUND, int WG>
__device__ __forceinline__ void global_sweep(const AttnDev& a, int64_t bg, typename C::T_* lds,
                                             const typename C::Frag (*qf)[C::NT], Soft<C::MB>* st, int lane) {
    f32x16 negm[2];
#pragma unroll
    for (int nb = 0; nb < 2; ++nb)
#pragma unroll
        for (int r = 0; r < 16; ++r) negm[nb][r] = -st[nb].m;
    typedef typename C::T_ T;
    constexpr int EP = Piece<T>::N;
    constexpr int VGS = 64 + EP;
    constexpr int STAGE = 64 * C::KSTR + 32 * C::MB * VGS;
    init_v_padding<C>(lds + 64 * C::KSTR, VGS, 64);
    init_v_padding<C>(lds + STAGE + 64 * C::KSTR, VGS, 64);
    const StageDma<C, WG> dma;
    dma.copy(a, bg, 0, lds);
    dma_wait();
    __syncthreads();
    int buf = 0;
    for (int base = 0; base < a.M; base += 64) {
        const int next = base + 64;
        // The other buffer held the previous stage, which every wave finished
        // before the last barrier.
        if (next < a.M) dma.copy(a, bg, next, lds + (buf ^ 1) * STAGE);
        T* cur = lds + buf * STAGE;
        global_stage<C, BOUND>(a, base, cur, cur + 64 * C::KSTR, VGS, qf, st, negm, lane);
        dma_wait();
        __syncthreads();
        buf ^= 1;
    }
}

// The bounded sweep, software-pipelined across tiles so that every stretch
// of exponentials has independent MFMAs beside it.  With s0 / s1 the score
// tiles of the wave's two column blocks, tile t runs as two phases:
//   A(t): exponentials of s0(t)  |  MFMAs: scores s1(t), products of block 1 for t - 1
//   B(t): exponentials of s1(t)  |  MFMAs: scores s0(t + 1), products of block 0 for t
// so each phase holds 16 exponentials, 8 converts and 7 independent MFMAs
// (head_dim 48), which the SIMD co-issues.  Stages rotate through three LDS
// buffers: while stage s is consumed, stage s + 1 (already in LDS) feeds the
// look-ahead score tile and stage s + 2 is fetched, so one barrier per stage
// suffices.  Used for bf16 with head_dim <= 48 (fp16 takes the running max).
template <typename C>
constexpr bool kPiped = std::is_same<typename C::T_, __bf16>::value && C::D <= 48;

template <typename C>
__device__ __forceinline__ void probs_to_frags(const f32x16& s, typename C::Frag* pf, float& l) {
    float p[16];
#pragma unroll
    for (int r = 0; r < 16; ++r) p[r] = __builtin_amdgcn_exp2f(s[r]);
    if constexpr (!C::ONES) {
        float psum = 0.f;
#pragma unroll
        for (int r = 0; r < 16; ++r) psum += p[r];
        l += psum;
    }
#pragma unroll
    for (int ks = 0; ks < C::KSTEPS; ++ks) pf[ks] = frag_from_p<typename C::T_>(p, ks);
}

template <typename C>
__device__ __forceinline__ void accumulate_frags(Soft<C::MB>& st, const typename C::Frag* vf,
                                                 const typename C::Frag* pf) {
#pragma unroll
    for (int ks = 0; ks < C::KSTEPS; ++ks)
#pragma unroll
        for (int b = 0; b < C::MB; ++b) st.acc[b] = C::M::mfma(vf[b * C::KSTEPS + ks], pf[ks], st.acc[b]);
}

// Scores of keys at or beyond M (the partial last tile) -> -inf.
template <typename C>
__device__ __forceinline__ void mask_tail(const AttnDev& a, int first, f32x16& s, int g) {
    if (first + 32 > a.M) {
#pragma unroll
        for (int r = 0; r < 16; ++r)
            if (first + kperm<C::E, C::KS>(acc_row(r, g)) >= a.M) s[r] = -INFINITY;
    }
}

// One phase of the pipelined sweep: the exponentials of `sx` (column block
// X) -> pfx, beside the score MFMAs sq = negm + K Q_Y^T of the other column
// block Y and the products accY += V pfy of block Y's previous tile.  They
// are written interleaved, each MFMA followed by its share of the
// exponentials and converts, with scheduling barriers between the groups,
// so that every exponential has an independent MFMA in flight beside it.
// With LOADS, once the score MFMAs have read kf the next tile's keys are
// loaded into it (this lane's key row at knext), and once the products have
// read vf the values of the tile at vnext (a transposed stage buffer) are.
template <typename C, bool LOADS>
__device__ __forceinline__ void pipe_phase(const f32x16& sx, typename C::Frag* pfx, float& lx,
                                           const typename C::Frag* qy, const f32x16& negm, f32x16& sq,
                                           Soft<C::MB>& sty, const typename C::Frag* pfy, typename C::Frag* kf,
                                           const typename C::T_* knext, typename C::Frag* vf,
                                           const typename C::T_* vnext, int lane) {
    constexpr int NQ = C::NT, NM = C::NT + C::MB * C::KSTEPS;
    float p[16];
#pragma unroll
    for (int j = 0; j < NM; ++j) {
        if (j < NQ) {
            sq = C::M::mfma(kf[j], qy[j], j == 0 ? negm : sq);
        } else {
            const int i = j - NQ, ks = i / C::MB, b = i % C::MB;
            sty.acc[b] = C::M::mfma(vf[b * C::KSTEPS + ks], pfy[ks], sty.acc[b]);
        }
#pragma unroll
        for (int r = 16 * j / NM; r < 16 * (j + 1) / NM; ++r) {
            p[r] = __builtin_amdgcn_exp2f(sx[r]);
            if (r % 8 == 7) pfx[r / 8] = frag_from_p<typename C::T_>(p, r / 8);
        }
        if (LOADS && j == NQ - 1) load_kfrags<C>(knext, kf);
        if (LOADS && j == NM - 1) load_vfrags<C, true>(vnext, 64 + Piece<typename C::T_>::N, 0, lane, vf);
        __builtin_amdgcn_sched_barrier(0);
    }
    if constexpr (!C::ONES) {
        float psum = 0.f;
#pragma unroll
        for (int r = 0; r < 16; ++r) psum += p[r];
        lx += psum;
    }
}

// One tile t of the pipelined sweep: phases A(t) and B(t).  On entry s0
// holds the block-0 scores and kf the keys of tile t, pf1 / vf the block-1
// probabilities and the values of tile t - 1; on exit s0 and kf belong to
// tile t + 1 (keys at knext), pf1 / vf to tile t (values at vcur).  negm is
// the wave's common reference point.  MASK masks keys at or beyond M (the
// partial last tile).
template <typename C, bool MASK>
__device__ __forceinline__ void pipe_tile(const AttnDev& a, const typename C::T_* vcur, int first,
                                          const typename C::T_* knext, const typename C::Frag (*qf)[C::NT],
                                          Soft<C::MB>* st, const f32x16& negm, f32x16& s0,
                                          typename C::Frag* kf, typename C::Frag* pf1, typename C::Frag* vf,
                                          int lane) {
    const int g = lane >> 5;
    typename C::Frag pf0[C::KSTEPS];
    f32x16 s1;
    if constexpr (MASK) mask_tail<C>(a, first, s0, g);
    // A(t): exponentials of s0(t) | scores s1(t), block 1's products of t - 1;
    // then the keys of t + 1 and the values of t are loaded
    pipe_phase<C, true>(s0, pf0, st[0].l, qf[1], negm, s1, st[1], pf1, kf, knext, vf, vcur, lane);
    if constexpr (MASK) mask_tail<C>(a, first, s1, g);
    // B(t): exponentials of s1(t) | scores s0(t + 1), block 0's products of t
    pipe_phase<C, false>(s1, pf1, st[1].l, qf[0], negm, s0, st[0], pf0, kf, nullptr, vf, nullptr, lane);
}

template <typename C, int WG>
__device__ __forceinline__ void global_sweep_piped(const AttnDev& a, int64_t bg, typename C::T_* lds,
                                                   const typename C::Frag (*qf)[C::NT], Soft<C::MB>* st,
                                                   int lane) {
    typedef typename C::T_ T;
    typedef typename C::Frag Frag;
    const int g = lane >> 5, qi = lane & 31;
    f32x16 negm;
#pragma unroll
    for (int r = 0; r < 16; ++r) negm[r] = -st[0].m;
    constexpr int EP = Piece<T>::N;
    constexpr int VGS = 64 + EP;
    constexpr int STAGE = 64 * C::KSTR + 32 * C::MB * VGS;
#pragma unroll
    for (int b = 0; b < 3; ++b) init_v_padding<C>(lds + b * STAGE + 64 * C::KSTR, VGS, 64);
    const int stages = (a.M + 63) / 64, full = a.M / 64;
    const StageDma<C, WG> dma;
    dma.copy(a, bg, 0, lds);
    dma.copy(a, bg, 64 * min(1, stages - 1), lds + STAGE);
    dma_wait();
    __syncthreads();

    const int krow = kperm<C::E, C::KS>(qi) * C::KSTR + C::E * g;
    Frag kf[C::NT], vf[C::MB * C::KSTEPS], pf1[C::KSTEPS];
#pragma unroll
    for (int i = 0; i < C::MB * C::KSTEPS; ++i) vf[i] = frag_fill<T>(0.f);
#pragma unroll
    for (int i = 0; i < C::KSTEPS; ++i) pf1[i] = frag_fill<T>(0.f);
    load_kfrags<C>(lds + krow, kf);
    f32x16 s0 = score_tile<C>(kf, qf[0], negm);

    // Stages whose 64 keys are all present: no masks.
    int cur = 0;  // buffer of stage `stage`
    // The loop body is one basic block (a branch would let the compiler sink
    // a phase's exponentials away from their MFMAs): stage s + 2 is always
    // fetched, past the last stage as a repeat of it into the buffer no one
    // reads any more.
    for (int stage = 0; stage < full; ++stage) {
        const int nxt = cur == 2 ? 0 : cur + 1;
        // Buffer cur + 2 held stage - 1, which every wave finished reading
        // before the barrier that ended the previous iteration.
        dma.copy(a, bg, 64 * min(stage + 2, stages - 1), lds + (nxt == 2 ? 0 : nxt + 1) * STAGE);
        const T* Ks = lds + cur * STAGE;
        pipe_tile<C, false>(a, Ks + 64 * C::KSTR, 0, Ks + 32 * C::KSTR + krow, qf, st, negm, s0, kf, pf1, vf, lane);
        pipe_tile<C, false>(a, Ks + 64 * C::KSTR + 32, 0, lds + nxt * STAGE + krow, qf, st, negm, s0, kf, pf1, vf,
                            lane);
        dma_wait();
        __syncthreads();
        cur = nxt;
    }
    // The last, partial stage (its rows past M are zero in LDS).
    if (full < stages) {
        const T* Ks = lds + cur * STAGE;
        const int base = 64 * full;
        pipe_tile<C, true>(a, Ks + 64 * C::KSTR, base, Ks + 32 * C::KSTR + krow, qf, st, negm, s0, kf, pf1, vf,
                           lane);
        if (base + 32 < a.M)
            pipe_tile<C, true>(a, Ks + 64 * C::KSTR + 32, base + 32, Ks + krow, qf, st, negm, s0, kf, pf1, vf,
                               lane);
        __syncthreads();
    }
    accumulate_frags<C>(st[1], vf, pf1);
}

// The summary pathway for this workgroup.  Summary keys are stored scaled by
// log2(e)/sqrt(d), so scores are in the exp2 domain.  Every score of a query
// is bounded by |q| max_j |sk_j| (Cauchy-Schwarz); that bound is the fixed
// softmax reference point, fed to the score MFMA as its initial accumulator.
// If it is so loose that a query's denominator underflows, the workgroup
// redoes the sweep with the exact online softmax.
//
// The probabilities are rounded to the storage type before the PV product.
// bf16 keeps fp32's exponent range, so every probability above the
// underflow check keeps its 8 significant bits, however loose the bound.
// fp16 does not: below 2^-14 a probability is subnormal and keeps only a few
// bits, so a bound 14-24 log2 units above the true maximum would degrade
// every probability of the query.  fp16 therefore takes the running max,
// which keeps the largest probability of each query in [1, 2^8].
template <typename C, int WG>
__device__ __forceinline__ void global_pass(const AttnDev& a, int64_t bg, typename C::T_* lds,
                                            const typename C::Frag (*qf)[C::NT], Soft<C::MB>* st, int lane) {
    if constexpr (std::is_same<typename C::T_, _Float16>::value) {
#pragma unroll
        for (int nb = 0; nb < 2; ++nb) st[nb].reset();
        global_sweep<C, false, WG>(a, bg, lds, qf, st, lane);
        return;
    }
    const float kmax = wave_max(a.sk_norm_max[bg * 64 + lane]);
#pragma unroll
    for (int nb = 0; nb < 2; ++nb) {
        st[nb].reset();
        st[nb].m = q_norm<C>(qf[nb]) * kmax;
    }
    if constexpr (kPiped<C>) {
        // One reference point for the wave's 64 queries (their largest bound),
        // so both column blocks share one initial accumulator.
        const float m = wave_max(fmaxf(st[0].m, st[1].m));
        st[0].m = st[1].m = m;
        global_sweep_piped<C, WG>(a, bg, lds, qf, st, lane);
    } else
        global_sweep<C, true, WG>(a, bg, lds, qf, st, lane);
    bool weak = false;
#pragma unroll
    for (int nb = 0; nb < 2; ++nb) weak = weak || !(soft_denominator<C>(st[nb], lane >> 5) > 0x1p-60f);
    if (__syncthreads_or(weak)) {
#pragma unroll
        for (int nb = 0; nb < 2; ++nb) st[nb].reset();
        global_sweep<C, false, WG>(a, bg, lds, qf, st, lane);
    }
}

// Channels of accumulator register r in lane group g of block mb.
__device__ __forceinline__ int acc_channel(int mb, int r, int g) { return 32 * mb + acc_row(r, g); }

template <typename T>
__device__ __forceinline__ void store_quad(T* dst, const float* v) {
#pragma unroll
    for (int i = 0; i < 4; ++i) dst[i] = from_f32<T>(v[i]);
}

template <typename T>
__device__ __forceinline__ void load_quad(const T* src, float* v) {
#pragma unroll
    for (int i = 0; i < 4; ++i) v[i] = to_f32(src[i]);
}

// Finish the local state: sl * o_L (storage type; the epilogue adds the
// global branch) goes to y, or with a park buffer into LDS (slot
// 4 mb + q of this lane, quads of 4 channels, lane-fastest), optionally
// saving o_L and its log-sum-exp.
template <typename C>
__device__ __forceinline__ void finish_local(const AttnDev& a, int b, int h, int64_t row, bool valid, int g,
                                             const Soft<C::MB>& st, typename C::T_* park, int lane) {
    typedef typename C::T_ T;
    const float den = soft_denominator<C>(st, g);
    const float inv = den > 0.f ? 1.f / den : 0.f;  // an all-masked row gives 0
    const int64_t bh = (int64_t)b * a.H + h;
    T* y = reinterpret_cast<T*>(a.y) + b * a.ysb + h * a.ysh + row * a.ysn;
    T* ol = a.o_l && valid ? reinterpret_cast<T*>(a.o_l) + (bh * a.N + row) * C::D : nullptr;
#pragma unroll
    for (int mb = 0; mb < C::MB; ++mb)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            if (32 * mb + 8 * q >= C::D) continue;
            const int ch0 = acc_channel(mb, 4 * q, g);
            float o[4], yl[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                o[i] = st.acc[mb][4 * q + i] * inv;
                yl[i] = a.sl[ch0 + i] * o[i];
            }
            if (park)
                store_quad<T>(park + ((4 * mb + q) * 64 + lane) * 4, yl);
            else if (valid)
                store_quad<T>(y + ch0, yl);
            if (ol) store_quad<T>(ol + ch0, o);
        }
    if (a.lse_l && valid) a.lse_l[bh * a.N + row] = den > 0.f ? st.m * kLn2 + __logf(den) : -INFINITY;
}

// y = sl * o_L + gate * sg * o_G.  The local term comes from y itself
// (LOCAL_Y: written by finish_local, or by p3d_local_fwd_indexed before the
// rows kernel), from o_local_in (LOCAL_IN, rows kernel) or from the LDS
// park buffer finish_local filled (LOCAL_PARK, brick kernel).
enum LocalSource { LOCAL_Y, LOCAL_IN, LOCAL_PARK };

template <typename C, int SRC>
__device__ __forceinline__ void epilogue(const AttnDev& a, int b, int h, int64_t row, bool valid, int g,
                                         const Soft<C::MB>& st, const typename C::T_* park = nullptr,
                                         int lane = 0) {
    typedef typename C::T_ T;
    const float den = soft_denominator<C>(st, g);
    if (!valid) return;
    const float inv = 1.f / den;
    const int64_t bh = (int64_t)b * a.H + h;
    const float gate = load_any(a.gate, b * a.gsb + h * a.gsh + row * a.gsn, a.gate_dtype);
    T* y = reinterpret_cast<T*>(a.y) + b * a.ysb + h * a.ysh + row * a.ysn;
    T* og = a.o_g ? reinterpret_cast<T*>(a.o_g) + (bh * a.N + row) * C::D : nullptr;
    const float* oli = SRC == LOCAL_IN ? a.o_local_in + (bh * a.N + row) * C::D : nullptr;
#pragma unroll
    for (int mb = 0; mb < C::MB; ++mb)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            if (32 * mb + 8 * q >= C::D) continue;
            const int ch0 = acc_channel(mb, 4 * q, g);
            float yl[4], out[4], o[4];
            if constexpr (SRC == LOCAL_Y) {
                load_quad<T>(y + ch0, yl);
            } else if constexpr (SRC == LOCAL_PARK) {
                load_quad<T>(park + ((4 * mb + q) * 64 + lane) * 4, yl);
            } else {
#pragma unroll
                for (int i = 0; i < 4; ++i) yl[i] = a.sl[ch0 + i] * oli[ch0 + i];
            }
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                o[i] = st.acc[mb][4 * q + i] * inv;
                out[i] = yl[i] + gate * a.sg[ch0 + i] * o[i];
            }
            store_quad<T>(y + ch0, out);
            if (og) store_quad<T>(og + ch0, o);
        }
    if (a.lse_g) a.lse_g[bh * a.N + row] = st.m * kLn2 + __logf(den);
}

// ------------------------------------------------------------------- grid
// Rotations of the workgroup's coordinate window, staged once in LDS: for
// rotary pair j, entry j * kPlane + w holds (cos, sin) at coordinate
// origin[axis(j)] + w of the pair's axis, w < kPlane; axis(j) is kept too.
// The window origin is (Z0 - rz, Y0 - ry, X0 - rx), covering every query and
// halo key of the brick.  Packed positions (row indices) do not fit a window
// and use the global table.
struct RopeWindow {
    float2* cs;
    int* axis;
    __device__ __forceinline__ float2 at(int j, int wz, int wy, int wx) const {
        const int ax = axis[j];
        return cs[j * kPlane + (ax == 0 ? wz : (ax == 1 ? wy : wx))];
    }
};

__device__ __forceinline__ void build_rope_window(const AttnDev& a, int D, int oz, int oy, int ox, RopeWindow w) {
    const int pairs = D / 2;
    for (int i = threadIdx.x; i < pairs * kPlane; i += blockDim.x) {
        const int j = i / kPlane, k = i - j * kPlane;
        const int32_t* d = a.rope.pairs + 3 * j;
        const int ax = d[2];
        const int origin = ax == 0 ? oz : (ax == 1 ? oy : ox);
        const int extent = ax == 0 ? a.Z : (ax == 1 ? a.Y : a.X);
        const int c = origin + k;
        w.cs[i] = (c >= 0 && c < extent) ? a.rope.table[d[0] + (int64_t)d[1] * c] : float2{1.f, 0.f};
        if (k == 0) w.axis[j] = ax;
    }
}

// Workgroups are dispatched round-robin over the 8 XCDs.  Give each XCD a
// contiguous run of work items (heads of a brick, then bricks in raster
// order) so that the items an XCD runs together share rows in its L2.
__device__ __forceinline__ int xcd_brick(int id, int bricks) {
    const int q = bricks / 8, r = bricks % 8;
    const int xcd = id % 8, slot = id / 8;
    return xcd < r ? xcd * (q + 1) + slot : r * (q + 1) + (xcd - r) * q + slot;
}

// Local-pathway plane staging.  A task is one channel piece of 4 x-adjacent
// keys of a plane row, handled as two halves of 2 keys whose loads are issued
// before they are consumed; K is rotated on the way and V is written
// transposed with one 2-key store per channel.
template <typename C>
struct PlaneStager {
    typedef typename C::T_ T;
    static constexpr int EP = Piece<T>::N;
    static constexpr int PPR = C::D / EP;                       // pieces per key row
    static constexpr int TASKS = kPlane * (kPlane / 4) * PPR;   // 4-key groups x pieces
    static constexpr int ITERS = (TASKS + 64 * kWaves - 1) / (64 * kWaves);
    typedef __attribute__((ext_vector_type(2))) T T2;

    __device__ __forceinline__ void stage(const AttnDev& a, const T* KL, const T* VL, int hz, int gz, int Y0,
                                          int X0, const RopeWindow& win, T* Kp, T* Vp, int vps) const {
#pragma unroll
        for (int it = 0; it < ITERS; ++it) {
            const int task = threadIdx.x + it * 64 * kWaves;
            if (task >= TASKS) break;
            const int piece = task % PPR, grp = task / PPR;
            const int ky = grp / (kPlane / 4), kx0 = 4 * (grp % (kPlane / 4));
            const int gy = Y0 - a.ry + ky;
            const bool row_in = gz >= 0 && gz < a.Z && gy >= 0 && gy < a.Y && ky < 8 + 2 * a.ry;
            // Two halves of 2 keys: loads of a half are issued before it is consumed.
#pragma unroll
            for (int half = 0; half < 2; ++half) {
                uint4 kraw[2], vraw[2];
                float2 cs[2][EP / 2];
                bool in[2];
#pragma unroll
                for (int i = 0; i < 2; ++i) {
                    const int kx = kx0 + 2 * half + i, gx = X0 - a.rx + kx;
                    in[i] = row_in && gx >= 0 && gx < a.X && kx < 8 + 2 * a.rx;
                    kraw[i] = vraw[i] = uint4{0, 0, 0, 0};
                    if (in[i]) {
                        const int64_t raster = ((int64_t)gz * a.Y + gy) * a.X + gx;
                        const int64_t row = a.map ? (int64_t)a.map[raster] : raster;
                        kraw[i] = *reinterpret_cast<const uint4*>(KL + row * a.ksn + piece * EP);
                        vraw[i] = *reinterpret_cast<const uint4*>(VL + row * a.vsn + piece * EP);
                        if (a.kl_rotated) {
#pragma unroll
                            for (int e = 0; e < EP / 2; ++e) cs[i][e] = float2{1.f, 0.f};  // not applied
                        } else if (a.rope.packed) {
                            const int64_t pos[3] = {row, 0, 0};
#pragma unroll
                            for (int e = 0; e < EP / 2; ++e) cs[i][e] = rope_cs(a.rope, piece * EP / 2 + e, pos);
                        } else {
#pragma unroll
                            for (int e = 0; e < EP / 2; ++e) cs[i][e] = win.at(piece * EP / 2 + e, hz, ky, kx);
                        }
                    }
                }
#pragma unroll
                for (int i = 0; i < 2; ++i) {
                    const T* kv = reinterpret_cast<const T*>(&kraw[i]);
                    T kt[EP];
#pragma unroll
                    for (int e = 0; e < EP; e += 2) {
                        float x0 = to_f32(kv[e]), x1 = to_f32(kv[e + 1]);
                        if (in[i] && !a.kl_rotated) rotate_pair(x0, x1, cs[i][e / 2].x, cs[i][e / 2].y);
                        kt[e] = from_f32<T>(x0);
                        kt[e + 1] = from_f32<T>(x1);
                    }
                    *reinterpret_cast<uint4*>(Kp + (ky * kPlane + kx0 + 2 * half + i) * C::KSTR + piece * EP) =
                        *reinterpret_cast<const uint4*>(kt);
                }
#pragma unroll
                for (int e = 0; e < EP; ++e) {
                    T2 col;
#pragma unroll
                    for (int i = 0; i < 2; ++i) col[i] = reinterpret_cast<const T*>(&vraw[i])[e];
                    *reinterpret_cast<T2*>(Vp + (piece * EP + e) * vps + ky * kPlane + kx0 + 2 * half) = col;
                }
            }
        }
    }
};

// 16-bit mask of the valid keys of chunk c among this lane's 16 scores:
// the (2ry+1) x (2rx+1) stencil in y and x around query (qy, qx) of the wave
// footprint, clipped to the grid.  The z condition is applied per plane.
template <typename C>
__device__ __forceinline__ uint32_t stencil_mask(const AttnDev& a, int c, int g, int qy, int qx, int Yw, int Xw) {
    uint32_t m = 0;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
        const int kr = kperm<C::E, C::KS>(acc_row(r, g));
        const int ky = 4 * c + kr / 8, kx = kr % 8;  // within the wave footprint
        const int gy = Yw - a.ry + ky, gx = Xw - a.rx + kx;
        const bool ok = (unsigned)(ky - qy) <= (unsigned)(2 * a.ry) && (unsigned)(kx - qx) <= (unsigned)(2 * a.rx) &&
                        (unsigned)gy < (unsigned)a.Y && (unsigned)gx < (unsigned)a.X;
        m |= (ok ? 1u : 0u) << r;
    }
    return m;
}

// Local-pathway plane staging by the LDS DMA (16-bit types; head_dim <= 48
// on 12-wide planes, head_dim 64 on 10-wide planes, see below).  Each
// halo plane is copied into one of two plane buffers while the previous plane
// is scored, so no wave waits on global memory between planes.  A buffer holds
// K and V in the same key-major layout (key row stride KSTR: D / 8 data slots
// of 16 bytes and one spare, whose lanes fetch a piece of the same row).  K is
// rotated in place once its copy has landed; the value fragments are read
// with ds_read_b64_tr_b16, so V needs no transposing store.  The packed row
// of every halo key of the brick is looked up once into a table in LDS; keys
// outside the grid take the row of the nearest grid key (finite, and masked
// by the stencil).
//
// A plane holds PW keys per row (x) and 12 rows (y), key (ky, kx) at
// ky * PW + kx.  PW = 12 covers radius 2.  At head_dim 64 two buffers of
// 12-wide planes do not leave room for a second workgroup per CU, so that
// head_dim takes radius <= 1 on 10-wide planes: a wave's 8-key-wide footprint
// then reaches columns 10 and 11 of its rows, which fall on the first keys of
// the next row (or, past the last row, on 12 - PW spare keys that hold grid
// keys too): finite values that the stencil masks, as for the clamped keys.
template <typename C, int PW>
constexpr bool kPlaneDma = sizeof(typename C::T_) == 2 && (PW == 12 ? C::D <= 48 : PW == 10 && C::D == 64);

template <typename C, int PW>
struct PlaneDma {
    typedef typename C::T_ T;
    static constexpr int EP = Piece<T>::N;
    static constexpr int PH = 12;                        // plane rows
    static constexpr int KEYS = PH * PW + (12 - PW);     // keys of one plane, spares included
    static constexpr int KROW = C::KSTR / EP;           // 16-byte slots per key row
    static constexpr int SLOTS = KEYS * KROW;            // slots of K (or V) of one plane
    static constexpr int CH = (SLOTS + 63) / 64;         // copies per region
    static constexpr int PER = (2 * CH + kWaves - 1) / kWaves;
    static constexpr size_t REGION = (size_t)SLOTS * 16;
    static constexpr size_t BUF = 2 * REGION;            // one plane: K region, then V region
    static constexpr int kMaxPlanes = PW == 12 ? 8 : 6;  // 4 + 2 rz with rz <= 2 (or <= 1)
    static constexpr size_t ROWS = (size_t)kMaxPlanes * KEYS * sizeof(int);
    static constexpr size_t BYTES = 2 * BUF + ROWS;      // two plane buffers and the row table
    static_assert(C::KSTR % EP == 0 && C::KSTR > C::D, "key rows need a spare slot");

    // Packed rows of the halo keys of planes [0, planes) (z from Z0 - rz).
    __device__ __forceinline__ static void fill_rows(const AttnDev& a, int Z0, int Y0, int X0, int planes,
                                                     int* rows) {
        for (int i = threadIdx.x; i < planes * KEYS; i += blockDim.x) {
            const int hz = i / KEYS, k = i - hz * KEYS, ky = k / PW, kx = k - ky * PW;
            const int gz = min(max(Z0 - a.rz + hz, 0), a.Z - 1);
            const int gy = min(max(Y0 - a.ry + ky, 0), a.Y - 1);
            const int gx = min(max(X0 - a.rx + kx, 0), a.X - 1);
            const int64_t raster = ((int64_t)gz * a.Y + gy) * a.X + gx;
            rows[i] = a.map ? a.map[raster] : (int)raster;
        }
    }

    // Issue the copies of one plane (its rows at `rows`) into `buf`.
    __device__ __forceinline__ static void copy(const AttnDev& a, const T* KL, const T* VL, const int* rows,
                                                unsigned char* buf, int wave, int lane) {
        const uint32_t lds0 = lds_address(buf);
#pragma unroll
        for (int i = 0; i < PER; ++i) {
            const int c = min(wave * PER + i, 2 * CH - 1);  // wave-uniform
            const bool v = c >= CH;
            const int first = min(64 * (v ? c - CH : c), SLOTS - 64);
            const int slot = first + lane, key = slot / KROW, s = slot - key * KROW;
            const int64_t row = rows[key];
            const int e = (s < C::D / EP ? s : 0) * EP;
            const T* src = v ? VL + row * a.vsn + e : KL + row * a.ksn + e;
            const uint32_t m0 = lds0 + (v ? (uint32_t)REGION : 0u) + (uint32_t)first * 16u;
            dma_copy16(src, m0);
        }
    }

    // Rotate the K rows of plane hz in place (rows: that plane's row table).
    // The spare keys past the last row stay as loaded (masked, never used).
    __device__ __forceinline__ static void rotate(const AttnDev& a, T* K, const int* rows, int hz,
                                                  const RopeWindow& win) {
        constexpr int PPR = C::D / EP;
        for (int i = threadIdx.x; i < PH * PW * PPR; i += blockDim.x) {
            const int key = i / PPR, piece = i - key * PPR, ky = key / PW, kx = key - ky * PW;
            uint4* p = reinterpret_cast<uint4*>(K + key * C::KSTR + piece * EP);
            const uint4 raw = *p;
            const T* kv = reinterpret_cast<const T*>(&raw);
            T kt[EP];
#pragma unroll
            for (int e = 0; e < EP; e += 2) {
                const int j = piece * EP / 2 + e / 2;
                float2 cs;
                if (a.rope.packed) {
                    const int64_t pos[3] = {rows[key], 0, 0};
                    cs = rope_cs(a.rope, j, pos);
                } else {
                    cs = win.at(j, hz, ky, kx);
                }
                float x0 = to_f32(kv[e]), x1 = to_f32(kv[e + 1]);
                rotate_pair(x0, x1, cs.x, cs.y);
                kt[e] = from_f32<T>(x0);
                kt[e + 1] = from_f32<T>(x1);
            }
            *p = *reinterpret_cast<const uint4*>(kt);
        }
    }

    // Value fragment (A operand of O^T += V^T P^T) of block mb from the
    // key-major V rows: lane l holds channel 32 mb + l % 32 of the 8 keys
    // key0 .. key0 + 7 (plane key indices, consecutive in x), read with
    // ds_read_b64_tr_b16 (tr_frag).  Blocks of 16 channels past D read the
    // last 16 and are replaced by the padding rows of O^T (the ones row at
    // channel D, zeros).
    __device__ __forceinline__ static typename C::Frag vfrag(const T* V, int key0, int mb, int lane) {
        typename C::Frag f = tr_frag<T, typename C::Frag>(V, key0, C::KSTR, 32 * mb, C::D - 16, lane);
        if (32 * mb + 16 >= C::D && 32 * mb + 16 * ((lane >> 4) & 1) >= C::D)
            f = frag_fill<T>(C::ONES && 32 * mb + (lane & 31) == C::D ? 1.f : 0.f);
        return f;
    }
};

// LDS of the brick kernel: the rotation window, then the plane buffer or
// the summary stages (whichever is larger), then -- when it still leaves room
// for two workgroups per CU -- the park buffer of sl * o_L (4 waves x 2
// column blocks x D / 8 quads x 64 lanes x 4 values), which saves y a write
// and a re-read.
template <typename C>
constexpr size_t grid_main_bytes() {
    constexpr size_t ep = Piece<typename C::T_>::N;
    constexpr size_t plane = (size_t)kPlaneKeys * C::KSTR + (size_t)32 * C::MB * (kPlaneKeys + ep);
    constexpr size_t stages = (kPiped<C> ? 3 : 2) * ((size_t)64 * C::KSTR + (size_t)32 * C::MB * (64 + ep));
    return kRopeWindowBytes + (plane > stages ? plane : stages) * sizeof(typename C::T_);
}
template <typename C>
constexpr size_t grid_park_bytes() {
    return (size_t)kWaves * 2 * (C::D / 8) * 64 * 4 * sizeof(typename C::T_);
}
template <typename C, int PW>
constexpr bool kPark = kPlaneDma<C, PW> || grid_main_bytes<C>() + grid_park_bytes<C>() <= 80 * 1024;
// With the plane DMA the regions after the rotation window are used twice:
// in the local phase by the two plane buffers and the row table, in the
// summary phase by the park buffer (over plane buffer 0, which the last
// plane -- always of odd index -- does not use) and the summary stages.
template <typename C, int PW>
constexpr size_t grid_dma_bytes() {
    constexpr size_t ep = Piece<typename C::T_>::N;
    constexpr size_t stages =
        (kPiped<C> ? 3 : 2) * ((size_t)64 * C::KSTR + (size_t)32 * C::MB * (64 + ep)) * sizeof(typename C::T_);
    constexpr size_t summary = grid_park_bytes<C>() + stages;
    return kRopeWindowBytes + (PlaneDma<C, PW>::BYTES > summary ? PlaneDma<C, PW>::BYTES : summary);
}
template <typename C, int PW>
constexpr size_t grid_lds_bytes() {
    if constexpr (kPlaneDma<C, PW>) {
        static_assert(grid_dma_bytes<C, PW>() <= 80 * 1024, "two workgroups per CU");
        static_assert(grid_park_bytes<C>() <= PlaneDma<C, PW>::BUF, "park buffer within plane buffer 0");
        return grid_dma_bytes<C, PW>();
    } else {
        return grid_main_bytes<C>() + (kPark<C, PW> ? grid_park_bytes<C>() : 0);
    }
}

// Scores and products of one staged plane on this wave's two column blocks
// (the chunks of its 8 x 8 key footprint).  Kb holds the plane's rotated K
// rows, PW keys per plane row; vfrag(c, mb, ks) returns the value fragment
// of chunk c.
template <typename C, int PW, typename VFrag>
__device__ __forceinline__ void plane_chunks(const AttnDev& a, const typename C::T_* Kb, VFrag vfrag, int hz,
                                             int wy, int wx, int qi, int g, const uint32_t* kmask,
                                             const typename C::Frag (*qf)[C::NT], Soft<C::MB>* st) {
#pragma unroll
    for (int c = 0; c < 2; ++c) {
        if (4 * c >= 4 + 2 * a.ry) continue;
        const int kap = kperm<C::E, C::KS>(qi);
        typename C::Frag kf[C::NT], vf[C::MB * C::KSTEPS];
        load_kfrags<C>(Kb + ((4 * wy + 4 * c + kap / 8) * PW + 4 * wx + kap % 8) * C::KSTR + C::E * g, kf);
#pragma unroll
        for (int mb = 0; mb < C::MB; ++mb)
#pragma unroll
            for (int ks = 0; ks < C::KSTEPS; ++ks) vf[mb * C::KSTEPS + ks] = vfrag(c, mb, ks);
        f32x16 bias;
#pragma unroll
        for (int r = 0; r < 16; ++r) bias[r] = (kmask[c] >> r) & 1 ? 0.f : -INFINITY;
#pragma unroll
        for (int nb = 0; nb < 2; ++nb) {
            // Column block nb holds query planes 2nb and 2nb + 1.
            if (hz < 2 * nb || hz > 2 * nb + 1 + 2 * a.rz) continue;
            f32x16 s = score_tile<C>(kf, qf[nb], bias);
            if (hz == 2 * nb || hz == 2 * nb + 1 + 2 * a.rz) {  // only one of the two query planes reaches
                const int qz = 2 * nb + (qi >> 4);
                if ((unsigned)(hz - qz) > (unsigned)(2 * a.rz)) {
#pragma unroll
                    for (int r = 0; r < 16; ++r) s[r] = -INFINITY;
                }
            }
            float p[16];
            soft_probs<C>(st[nb], s, a.scale_log2, p);
            soft_accumulate<C>(st[nb], p, vf);
        }
    }
}

template <typename T, int D, int PW>
__global__ __launch_bounds__(64 * kWaves, 2) void k_attn_grid(AttnDev a) {
    typedef Cfg<T, D> C;
    constexpr int EP = Piece<T>::N;
    constexpr int VPS = kPlaneKeys + EP;  // plane V row stride (elements)
    extern __shared__ __align__(16) unsigned char smem[];
    RopeWindow win{reinterpret_cast<float2*>(smem), reinterpret_cast<int*>(smem + kRopeWindowBytes - 256)};
    T* Kp = reinterpret_cast<T*>(smem + kRopeWindowBytes);
    T* Vp = Kp + kPlaneKeys * C::KSTR;

    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, g = lane >> 5, qi = lane & 31;
    // Heads run fastest: the workgroups of one brick's heads follow each other
    // on one XCD, so the rows they share (every head's slice of a token's
    // projection row lies in the same cache lines) are fetched from HBM once.
    const int work = xcd_brick(blockIdx.x, gridDim.x);
    const int bh = work % (a.B * a.H), brick = work / (a.B * a.H);
    const int b = bh / a.H, h = bh % a.H, kvh = h / (a.H / a.G);
    const int64_t bg = (int64_t)b * a.G + kvh;
    const int Z0 = 4 * (brick / (a.bricks_y * a.bricks_x));
    const int Y0 = 8 * ((brick / a.bricks_x) % a.bricks_y);
    const int X0 = 8 * (brick % a.bricks_x);
    const int wy = wave >> 1, wx = wave & 1;
    const int qy = (qi >> 2) & 3, qx = qi & 3;  // within the wave footprint

    typedef PlaneDma<C, PW> PD;
    constexpr bool DMA = kPlaneDma<C, PW>;
    unsigned char* const planes_lds = smem + kRopeWindowBytes;  // plane DMA: two buffers, then the row table
    int* const rowtab = reinterpret_cast<int*>(planes_lds + 2 * PD::BUF);
    const int planes = 4 + 2 * a.rz;
    const T* KL = tp<T>(a.kl) + b * a.ksb + kvh * a.ksh;
    const T* VL = tp<T>(a.vl) + b * a.vsb + kvh * a.vsh;
    if (!a.rope.packed) build_rope_window(a, D, Z0 - a.rz, Y0 - a.ry, X0 - a.rx, win);
    if constexpr (DMA) PD::fill_rows(a, Z0, Y0, X0, planes, rowtab);
    __syncthreads();
    const int uwave = __builtin_amdgcn_readfirstlane(wave);
    if constexpr (DMA) {
        if ((unsigned)(Z0 - a.rz) < (unsigned)a.Z) PD::copy(a, KL, VL, rowtab, planes_lds, uwave, lane);
    }

    // ---- queries
    typename C::Frag qf[2][C::NT];
    int64_t qrow[2];
    bool qok[2];
#pragma unroll
    for (int nb = 0; nb < 2; ++nb) {
        const int qz = 2 * nb + (qi >> 4);
        const int gz = Z0 + qz, gy = Y0 + 4 * wy + qy, gx = X0 + 4 * wx + qx;
        qok[nb] = gz < a.Z && gy < a.Y && gx < a.X;
        const int64_t raster = ((int64_t)gz * a.Y + gy) * a.X + gx;
        qrow[nb] = qok[nb] ? (a.map ? (int64_t)a.map[raster] : raster) : 0;
        const T* row = tp<T>(a.q) + b * a.qsb + h * a.qsh + qrow[nb] * a.qsn;
        if (a.rope.packed) {
            const int64_t pos[3] = {qrow[nb], 0, 0};
            load_q<C>(row, qok[nb], [&](int j) { return rope_cs(a.rope, j, pos); }, g, qf[nb]);
        } else {
            const int wz = qz + a.rz, wy_ = 4 * wy + qy + a.ry, wx_ = 4 * wx + qx + a.rx;
            load_q<C>(row, qok[nb], [&](int j) { return win.at(j, wz, wy_, wx_); }, g, qf[nb]);
        }
    }

    Soft<C::MB> st[2];
    st[0].reset();
    st[1].reset();

    // ---- local pathway: halo planes z = Z0 - rz .. Z0 + 3 + rz
    const uint32_t kmask[2] = {stencil_mask<C>(a, 0, g, qy, qx, Y0 + 4 * wy, X0 + 4 * wx),
                               stencil_mask<C>(a, 1, g, qy, qx, Y0 + 4 * wy, X0 + 4 * wx)};
    if constexpr (DMA) {
        for (int hz = 0; hz < planes; ++hz) {
            const int gz = Z0 - a.rz + hz;
            unsigned char* const buf = planes_lds + (hz & 1) * PD::BUF;
            // Plane hz has landed, and every wave is done with plane hz - 1,
            // whose buffer takes the copy of plane hz + 1.
            dma_wait();
            __syncthreads();
            if (hz + 1 < planes && (unsigned)(gz + 1) < (unsigned)a.Z)
                PD::copy(a, KL, VL, rowtab + (hz + 1) * PD::KEYS, planes_lds + ((hz + 1) & 1) * PD::BUF, uwave,
                         lane);
            if ((unsigned)gz >= (unsigned)a.Z) continue;  // plane outside the grid: nothing to attend
            T* const Kb = reinterpret_cast<T*>(buf);
            const T* const Vb = reinterpret_cast<const T*>(buf + PD::REGION);
            if (!a.kl_rotated) {
                PD::rotate(a, Kb, rowtab + hz * PD::KEYS, hz, win);
                __syncthreads();
            }
            plane_chunks<C, PW>(a, Kb,
                            [&](int c, int mb, int ks) {
                                return PD::vfrag(Vb, (4 * wy + 4 * c + (ks * C::KS + C::E * g) / 8) * PW + 4 * wx,
                                                 mb, lane);
                            },
                            hz, wy, wx, qi, g, kmask, qf, st);
        }
    } else {
        init_v_padding<C>(Vp, VPS, kPlaneKeys);
        const PlaneStager<C> stager;
        for (int hz = 0; hz < planes; ++hz) {
            const int gz = Z0 - a.rz + hz;
            if (hz) __syncthreads();
            stager.stage(a, KL, VL, hz, gz, Y0, X0, win, Kp, Vp, VPS);
            __syncthreads();
            if ((unsigned)gz >= (unsigned)a.Z) continue;  // plane outside the grid: nothing to attend
            plane_chunks<C, kPlane>(a, Kp,
                            [&](int c, int mb, int ks) {
                                const int k0 = ks * C::KS + C::E * g;  // chunk key (4c + k0/8, k0 % 8) of the footprint
                                return frag_load8<T>(Vp + (32 * mb + qi) * VPS + (4 * wy + 4 * c + k0 / 8) * kPlane +
                                                     4 * wx + k0 % 8);
                            },
                            hz, wy, wx, qi, g, kmask, qf, st);
        }
    }
    T* park = DMA ? reinterpret_cast<T*>(planes_lds)
                  : (kPark<C, PW> ? reinterpret_cast<T*>(smem + grid_main_bytes<C>()) : nullptr);
#pragma unroll
    for (int nb = 0; nb < 2; ++nb) {
        finish_local<C>(a, b, h, qrow[nb], qok[nb], g, st[nb],
                        park ? park + (wave * 2 + nb) * (C::D / 8) * 64 * 4 : nullptr, lane);
        st[nb].reset();
    }
    __syncthreads();  // the summary stages reuse the plane buffer

    // ---- global pathway (the rotation window is no longer needed)
    global_pass<C, 64 * kWaves>(a, bg, DMA ? reinterpret_cast<T*>(planes_lds + grid_park_bytes<C>()) : Kp,
                                qf, st, lane);
#pragma unroll
    for (int nb = 0; nb < 2; ++nb) {
        if constexpr (kPark<C, PW>)
            epilogue<C, LOCAL_PARK>(a, b, h, qrow[nb], qok[nb], g, st[nb],
                                    park + (wave * 2 + nb) * (C::D / 8) * 64 * 4, lane);
        else
            epilogue<C, LOCAL_Y>(a, b, h, qrow[nb], qok[nb], g, st[nb]);
    }
}

template <typename T, int D>
__global__ __launch_bounds__(64 * kRowsWaves, 2) void k_attn_rows(AttnDev a) {
    typedef Cfg<T, D> C;
    extern __shared__ __align__(16) unsigned char smem[];
    T* lds = reinterpret_cast<T*>(smem);

    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, g = lane >> 5, qi = lane & 31;
    const int bh = blockIdx.y, b = bh / a.H, h = bh % a.H, kvh = h / (a.H / a.G);
    const int64_t bg = (int64_t)b * a.G + kvh;

    typename C::Frag qf[2][C::NT];
    int64_t qrow[2];
    bool qok[2];
#pragma unroll
    for (int nb = 0; nb < 2; ++nb) {
        const int64_t row = (int64_t)blockIdx.x * 64 * kRowsWaves + 64 * wave + 32 * nb + qi;
        qok[nb] = row < a.N;
        qrow[nb] = qok[nb] ? row : 0;
        int64_t pos[3];
        rope_position(a.rope, qrow[nb], pos);
        load_q<C>(tp<T>(a.q) + b * a.qsb + h * a.qsh + qrow[nb] * a.qsn, qok[nb],
                  [&](int j) { return rope_cs(a.rope, j, pos); }, g, qf[nb]);
    }
    Soft<C::MB> st[2];
    st[0].reset();
    st[1].reset();
    global_pass<C, 64 * kRowsWaves>(a, bg, lds, qf, st, lane);
    if (a.o_local_in) {
#pragma unroll
        for (int nb = 0; nb < 2; ++nb) epilogue<C, LOCAL_IN>(a, b, h, qrow[nb], qok[nb], g, st[nb]);
    } else {  // y already holds sl * o_L (p3d_local_fwd_indexed)
#pragma unroll
        for (int nb = 0; nb < 2; ++nb) epilogue<C, LOCAL_Y>(a, b, h, qrow[nb], qok[nb], g, st[nb]);
    }
}

int fill_dev(const p3d_attn_args& x, AttnDev& d) {
    const int es = dtype_size(x.dtype);
    P3D_REQUIRE(x.dtype >= P3D_F32 && x.dtype <= P3D_BF16, "unknown dtype");
    P3D_REQUIRE(x.batch >= 1 && x.heads >= 1 && x.kv_heads >= 1 && x.heads % x.kv_heads == 0 && x.tokens >= 1,
                "bad batch/head/token counts");
    P3D_REQUIRE(x.summaries >= 1, "need at least one summary");
    P3D_REQUIRE(view_ok(x.q, es) && view_ok(x.kl, es) && view_ok(x.vl, es) && view_ok(x.y, es),
                "q/k/v/y rows must be 16-byte aligned");
    P3D_REQUIRE(x.gate.data && x.local_scale && x.global_scale && x.sk && x.svt && x.sk_norm_max,
                "null pointer argument");
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
    d.sk_norm_max = x.sk_norm_max;
    d.rope = rope_dev(x.rope);
    d.map = x.raster_to_packed;
    d.o_local_in = x.o_local_in;
    d.y = (char*)x.y.data, d.ysb = x.y.sb, d.ysh = x.y.sh, d.ysn = x.y.sn;
    d.lse_l = x.lse_local, d.lse_g = x.lse_global;
    d.o_l = (char*)x.o_local, d.o_g = (char*)x.o_global;
    d.scale_log2 = kLog2e / sqrtf((float)x.head_dim);
    d.kl_rotated = x.kl_rotated != 0;
    return P3D_OK;
}

template <typename T, int D, int PW>
size_t lds_grid() {
    typedef Cfg<T, D> C;
    return grid_lds_bytes<C, PW>();
}

template <typename T, int D>
size_t lds_rows() {
    typedef Cfg<T, D> C;
    constexpr int ep = Piece<T>::N;
    return (kPiped<C> ? 3 : 2) * ((size_t)64 * C::KSTR + (size_t)32 * C::MB * (64 + ep)) * sizeof(T);
}

template <typename T, int D, int PW>
void launch_grid_t(const AttnDev& d, dim3 grid, hipStream_t s) {
    k_attn_grid<T, D, PW><<<grid, 64 * kWaves, lds_grid<T, D, PW>(), s>>>(d);
}

// Head_dim 64 in a 16-bit type with radius <= 1 stages its halo planes by the
// LDS DMA on 10-wide planes; everything else takes 12-wide planes.
template <int D>
int launch_grid(const AttnDev& d, int dtype, dim3 grid, hipStream_t s) {
    constexpr int NARROW = D == 64 ? 10 : 12;
    const bool narrow = NARROW != 12 && d.rz <= 1 && d.ry <= 1 && d.rx <= 1;
    switch (dtype) {
        case P3D_F32: launch_grid_t<float, D, 12>(d, grid, s); break;
        case P3D_F16:
            if (narrow)
                launch_grid_t<_Float16, D, NARROW>(d, grid, s);
            else
                launch_grid_t<_Float16, D, 12>(d, grid, s);
            break;
        default:
            if (narrow)
                launch_grid_t<__bf16, D, NARROW>(d, grid, s);
            else
                launch_grid_t<__bf16, D, 12>(d, grid, s);
            break;
    }
    return check_launch("p3d_attn_fwd_grid");
}

template <int D>
int launch_rows(const AttnDev& d, int dtype, dim3 grid, hipStream_t s) {
    switch (dtype) {
        case P3D_F32: k_attn_rows<float, D><<<grid, 64 * kRowsWaves, lds_rows<float, D>(), s>>>(d); break;
        case P3D_F16: k_attn_rows<_Float16, D><<<grid, 64 * kRowsWaves, lds_rows<_Float16, D>(), s>>>(d); break;
        default: k_attn_rows<__bf16, D><<<grid, 64 * kRowsWaves, lds_rows<__bf16, D>(), s>>>(d); break;
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
    P3D_REQUIRE(bricks * d.B * d.H < (1LL << 31), "launch grid too large");
    dim3 grid((unsigned)(bricks * d.B * d.H));
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
    P3D_REQUIRE((int64_t)d.B * d.H < 65536, "launch grid too large");
    dim3 grid((unsigned)cdiv(d.N, 64 * kRowsWaves), (unsigned)(d.B * d.H));
    hipStream_t s = as_stream(stream);
    switch (args->head_dim) {
#define CASE(DD) \
    case DD: return launch_rows<DD>(d, args->dtype, grid, s);
        P3D_HEAD_DIMS(CASE)
#undef CASE
        default: return fail(P3D_EUNSUPPORTED, "head_dim must be one of 16, 32, 48, 64, 128");
    }
}

