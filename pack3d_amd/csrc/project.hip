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
#include <type_traits>

#include "rope.hpp"

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

// The rows of a wave's 32 tokens for the LayerNorm below: lane l loads token
// l % 32's channels 16 ks + 8 (l / 32) .. +8 for every 16-channel k-step ks
// (row 0 in dead lanes).  Apart from the arithmetic, so that a kernel can
// issue these loads first and let their latency pass under its set-up.
template <typename T, int KS>
__device__ __forceinline__ void layer_norm_load(const ProjDev& a, int64_t tok, bool live, int g, u32x4 (&raw)[KS]) {
    constexpr int DIM = 16 * KS;
    const T* xr = reinterpret_cast<const T*>(a.x) + (live ? tok : 0) * DIM + 8 * g;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) raw[ks] = *reinterpret_cast<const u32x4*>(xr + 16 * ks);
}

// An empty asm that claims to rewrite the pieces, so values derived from them
// before it are derived again after it instead of being kept in registers.
template <int KS>
__device__ __forceinline__ void renew_pieces(const u32x4 (&raw)[KS]) {
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
        u32x4& r = const_cast<u32x4&>(raw[ks]);
        asm volatile("" : "+v"(r.x), "+v"(r.y), "+v"(r.z), "+v"(r.w));
    }
}

// LayerNorm of the half rows `raw` (layer_norm_load) into the B fragments of
// the projection GEMM: normalised in fp32 (statistics shared with lane l ^
// 32, which holds the other half of the row) and rounded to the storage type
// as torch's LayerNorm output is.  lw / lb: the affine parameters in LDS as
// fp32.
template <typename T, int KS>
__device__ __forceinline__ void layer_norm_math(const ProjDev& a, const float* lw, const float* lb, int g,
                                                const u32x4 (&raw)[KS], typename Mma<T>::Frag (&xf)[KS]) {
    constexpr int DIM = 16 * KS;
    float sum = 0.f;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
        const T* v = reinterpret_cast<const T*>(&raw[ks]);
#pragma unroll
        for (int j = 0; j < 8; ++j) sum += to_f32(v[j]);
    }
    const float mean = (sum + lane_xor32(sum)) / (float)DIM;
    // Past 256 channels the row's fp32 values from one pass are not kept
    // for the next (the compiler held all 256 of them besides the 128
    // registers of the row and spilled): each pass converts the pieces again.
    if constexpr (KS > 16) renew_pieces(raw);
    float sq = 0.f;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
        const T* v = reinterpret_cast<const T*>(&raw[ks]);
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const float c = to_f32(v[j]) - mean;
            sq = fmaf(c, c, sq);
        }
    }
    const float rstd = 1.f / sqrtf((sq + lane_xor32(sq)) / (float)DIM + a.eps);
    if constexpr (KS > 16) renew_pieces(raw);
    // Explicit fused multiply-adds: every kernel that normalises through here
    // rounds the same way, whatever the compiler contracts elsewhere.
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
        const T* v = reinterpret_cast<const T*>(&raw[ks]);
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const int c = 16 * ks + 8 * g + j;
            xf[ks][j] = from_f32<T>(fmaf((to_f32(v[j]) - mean) * rstd, lw[c], lb[c]));
        }
    }
}

// Waves per SIMD: 4 up to dim 128, 3 at dim 192 (the 168 registers that
// leaves hold the GEMM without spilling; at 4 it spilled 16), else 2.
// LIN: x holds tokens already normalised (no LayerNorm: the loaded half rows
// are the B fragments), and the gate block writes its logits x Wg^T + bias,
// rounded once, as [rows, 2 heads] instead of the pair softmax (one
// workgroup per CU either way at dim 192, so LIN takes the register budget of
// two waves per SIMD there).
template <typename T, int KS, bool LIN>
__global__ __launch_bounds__(64 * kProjWaves)
__attribute__((amdgpu_waves_per_eu(KS <= 8 ? 4 : (KS <= 12 && !LIN ? 3 : 2)))) void k_project(ProjDev a) {
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
    const int lane = threadIdx.x & 63, g = lane >> 5, t = lane & 31;
    const int64_t tok0 = ((int64_t)blockIdx.x * kProjWaves + (threadIdx.x >> 6)) * 32, tok = tok0 + t;
    const bool live = tok < a.rows;
    // The token rows first: their latency passes under the set-up below
    // (rows past 256 channels would hold too many registers through it).
    constexpr bool kEarlyRows = KS <= 16;
    u32x4 xraw[KS];
    if constexpr (kEarlyRows) layer_norm_load<T, KS>(a, tok, live, g, xraw);
    if constexpr (!LIN)
        for (int c = threadIdx.x; c < DIM; c += blockDim.x) {
            lw[c] = load_any(a.ln_w, c, a.ln_dtype);
            lb[c] = load_any(a.ln_b, c, a.ln_dtype);
        }
    const int gbase = a.q_out + a.kv_out, nout = gbase + 2 * a.heads;
    const int nblocks = (nout + 31) / 32;
    // Weight row o of the concatenation [Wq; Wkv; Wg].
    auto wrow = [&](int o) __attribute__((always_inline)) -> const T* {
        return o < a.q_out ? reinterpret_cast<const T*>(a.wq) + (int64_t)o * DIM
               : o < gbase ? reinterpret_cast<const T*>(a.wkv) + (int64_t)(o - a.q_out) * DIM
                           : reinterpret_cast<const T*>(a.wg) + (int64_t)(o - gbase) * DIM;
    };
    // Every lane loads every time, with no branch and no select on the value
    // (either would make the wave wait for the load there): rows past nout
    // repeat row nout - 1, whose outputs are never stored, and the pieces
    // past PIECES are loaded and not staged.
    u32x4 wreg[PPT];
    auto fetch = [&](int ob) __attribute__((always_inline)) {
#pragma unroll
        for (int i = 0; i < PPT; ++i) {
            const int pc = threadIdx.x + i * 64 * kProjWaves, pcc = min(pc, PIECES - 1);
            const int r = pcc / (DIM / 8), c = (pcc % (DIM / 8)) * 8, o = 32 * ob + r;
            wreg[i] = *reinterpret_cast<const u32x4*>(wrow(min(o, nout - 1)) + c);
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
    fetch(min(1, nblocks - 1));
    __syncthreads();

    T* tile = otile[threadIdx.x >> 6];

    // ---- LayerNorm of the lane's half row (channels 16 ks + 8 g + j)
    Frag xf[KS];
    if constexpr (!kEarlyRows) layer_norm_load<T, KS>(a, tok, live, g, xraw);
    if constexpr (LIN) {
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) xf[ks] = __builtin_bit_cast(Frag, xraw[ks]);
    } else {
        layer_norm_math<T, KS>(a, lw, lb, g, xraw, xf);
    }

    // ---- D = W X^T, 32 outputs at a time
    T* go = reinterpret_cast<T*>(a.gate) + tok * a.heads;
    const uint32_t qbytes = 32u * a.q_out * sizeof(T), kvbytes = 32u * a.kv_out * sizeof(T);
    const __amdgpu_buffer_rsrc_t qrsrc = buffer_rsrc(reinterpret_cast<T*>(a.q) + tok0 * a.q_out, qbytes);
    const __amdgpu_buffer_rsrc_t kvrsrc = buffer_rsrc(reinterpret_cast<T*>(a.kv) + tok0 * a.kv_out, kvbytes);
    settle_loads(wreg, xf);
    // The GEMM of block ob into one accumulator set.
    auto gemm = [&](int ob) __attribute__((always_inline)) -> f32x16 {
        const T* wb = &wbuf[ob & 1][t * WS + 8 * g];
        f32x16 d;
#pragma unroll
        for (int r = 0; r < 16; ++r) d[r] = 0.f;
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) d = M::mfma(*reinterpret_cast<const Frag*>(wb + 16 * ks), xf[ks], d);
        return d;
    };
    // The outputs of block ob from its accumulators.
    auto epilogue = [&](int ob, const f32x16& d) __attribute__((always_inline)) {
        {
            // q / kv outputs of the block through the tile: row t, columns
            // acc_row(4 qd, g) .. +3, then 16-byte pieces (token tt, outputs
            // 8 pp .. +7) with four consecutive lanes per token.  Every block
            // runs this (the gate's block stores nothing here), and each piece
            // is one masked store into q and one into kv (a block may straddle
            // them), so that every block issues the same stores.
#pragma unroll
            for (int qd = 0; qd < 4; ++qd) {
                const float v[4] = {d[4 * qd], d[4 * qd + 1], d[4 * qd + 2], d[4 * qd + 3]};
                store4<T>(tile + t * OS + acc_row(4 * qd, g), v);
            }
            wave_lds_sync();
#pragma unroll
            for (int i = 0; i < 2; ++i) {
                const int tt = 16 * i + (lane >> 2), pp = lane & 3, o0 = 32 * ob + 8 * pp;
                const bool ok = tok0 + tt < a.rows && o0 < gbase;
                const u32x4 piece = *reinterpret_cast<const u32x4*>(tile + tt * OS + 8 * pp);
                buffer_store16(qrsrc, qbytes, (uint32_t)(tt * a.q_out + o0) * sizeof(T), ok && o0 < a.q_out, piece);
                buffer_store16(kvrsrc, kvbytes, (uint32_t)(tt * a.kv_out + o0 - a.q_out) * sizeof(T),
                               ok && o0 >= a.q_out, piece);
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
                        if constexpr (LIN) {
                            T* gl = reinterpret_cast<T*>(a.gate) + tok * 2 * a.heads + j;
                            gl[0] = from_f32<T>(l0);
                            gl[1] = from_f32<T>(l1);
                        } else {
                            const float m = fmaxf(l0, l1);
                            const float e0 = expf(l0 - m), e1 = expf(l1 - m);
                            go[j / 2] = from_f32<T>(e1 / (e0 + e1));
                        }
                    }
                }
            }
        }
    };
    // Unconditional (a stage after the last block fills a buffer no block
    // reads), so that every block issues the same loads.
    auto advance = [&](int ob) __attribute__((always_inline)) {
        stage((ob + 1) & 1);
        fetch(min(ob + 2, nblocks - 1));
        __syncthreads();
    };
    if constexpr (KS != 12 && KS != 16) {
        // One block at a time (the second accumulator set below would spill
        // at these widths).
        for (int ob = 0; ob < nblocks; ++ob) {
            epilogue(ob, gemm(ob));
            advance(ob);
        }
        return;
    }
    // Software-pipelined by one block: block ob's MFMAs are issued before
    // block ob - 1's epilogue, which then runs under them.  The staged
    // weights of block ob + 1 go into the buffer block ob - 1 read, whose
    // readers all passed the barrier that ended the step before.
    f32x16 d0 = gemm(0), d1;
    advance(0);
    int ob = 1;
    for (; ob + 1 < nblocks; ob += 2) {
        d1 = gemm(ob);
        epilogue(ob - 1, d0);
        advance(ob);
        d0 = gemm(ob + 1);
        epilogue(ob, d1);
        advance(ob + 1);
    }
    if (ob < nblocks) {
        d1 = gemm(ob);
        epilogue(ob - 1, d0);
        epilogue(ob, d1);
    } else {
        epilogue(ob - 1, d0);
    }
}

// ---------------------------------------------------------------- pooled
// k_project with the summary pooling of compression.py:28-44 fused in, for
// the no-grad forward on layouts whose fine block f of a batch is rows
// [64 f, 64 f + 64) (the blocks of build_layout), pool_size 1 and 64 slots.
// The kg / vg columns of kv are not written: in that forward their only
// reader is the pooling, which happens here on the values in the kernel.
//
// The waves 2k and 2k + 1 of a workgroup hold the two halves of one fine
// block.  The output blocks run in the order q | kl | vl | kg | vg | gate:
//   q, kl, vl   written as in k_project;
//   kg          each key rounded to the storage type (the value kv would
//               hold), rotated and rounded again (the reference pools rotated
//               keys stored in that type), into the wave's LDS rows;
//   (after the last kg block) the slot logits (k . w) / tau + bias_s from
//               those rows, the slot softmax over the fine block's 64 tokens
//               with the maxima and then the sums exchanged between the two
//               waves through LDS at workgroup barriers, and the weighted kg
//               sums over the wave's 32 tokens on MFMA: weights split into
//               two storage-type rows hi = round(a), lo = round(a - hi), so
//               every product is exact in fp32, as in k_pool_fwd;
//   vg          each block rounded through the wave's output tile and summed
//               the same way;
//   gate        as in k_project.
// At the end the even wave adds its partner's sums and stores the summary
// (keys times key_scale), its transposed value column and the key-norm slot
// as k_pool_fwd stores them.
struct PoolFuseDev {
    int G, D, GD, Mp;
    int tokens;       // per batch, a multiple of 64
    int kg0;          // output row of kg's first channel: q_out + 2 G D
    float inv_tau, key_scale;
    const float* weight;  // pooling weight [D], fp32
    const float* bias;    // slot bias [64], fp32
    RopeDev rope;
    char *sk, *svt;
    float* norm;          // [B, G, 64] key-norm slots, zero on entry
    int rotate_kl;        // store kl rotated by `rope` (rounded, rotated, rounded)
};

constexpr int kPoolFuseMaxCh = 192;  // G * D: the kg rows of 8 waves fill most of the LDS

// Dynamic LDS of k_project_pool (bytes), with KGS = G D + 8:
//   rows  [waves][32][KGS] T   each wave's rotated, rounded kg rows; after
//                              the kg sums, its fp32 sums [2][G D] (kg, vg)
//                              and key squares [G D]
//   wts   [waves][G][2][32] T  slot weights hi, lo of the wave's tokens
//   xch   [waves][16] float    softmax maxima [8] and sums [8] per head
//   meta  [G D / 2] int4       rotary pair metadata of each pair of G heads' channels
//   lwp   [D] float, lbias [64] float
inline size_t pool_fuse_lds_bytes(int G, int D) {
    return (size_t)kProjWaves * 32 * (G * D + 8) * 2 + (size_t)kProjWaves * G * 64 * 2 + (size_t)kProjWaves * 16 * 4 +
           (size_t)(G * D / 2) * 16 + (size_t)D * 4 + 64 * 4;
}

// Static LDS of k_project / k_project_pool at model width DIM (bytes).
inline size_t project_static_lds_bytes(int dim) {
    return (size_t)2 * dim * 4 + (size_t)2 * 32 * (dim + 8) * 2 + (size_t)kProjWaves * 32 * 40 * 2;
}

// sum_t (hi_t + lo_t) X[t][c0 + l] over a wave's 32 tokens, in lanes l < 16:
// one 16x16x32 MFMA with A = the weight rows hi, lo (w: [2][32]) and B =
// 16 channels of the row-major rows X (token t at x + t * stride, channel c0
// at x), read with two ds_read_b64_tr_b16: within a 16-lane block, lane
// B + 4a + e receives element e of the 8-byte windows addressed by lanes
// B + a + 4j (j = 0..3), so lane L addresses token 8 (L / 16) + (L % 16) / 4
// (four tokens further for the second read) at channel 4 (L % 4).
template <typename T>
__device__ __forceinline__ float slot_sum(const T* w, const T* x, int stride, int lane) {
    typedef typename Mma<T>::Frag Frag;
    typedef short v4s __attribute__((ext_vector_type(4)));
    typedef short v8s __attribute__((ext_vector_type(8)));
    typedef __attribute__((address_space(3))) v4s* lds_v4s;
    const int r = lane & 15;
    u32x4 wv = u32x4{0u, 0u, 0u, 0u};
    if (r < 2) wv = *reinterpret_cast<const u32x4*>(w + 32 * r + 8 * (lane >> 4));
    const int tk = 8 * (lane >> 4) + (r >> 2);
    const unsigned char* base = reinterpret_cast<const unsigned char*>(x + 4 * (lane & 3));
    const v4s lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4s)(base + tk * stride * 2));
    const v4s hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4s)(base + (tk + 4) * stride * 2));
    const v8s b = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
    const f32x4 d = Mma<T>::mfma16(__builtin_bit_cast(Frag, wv), __builtin_bit_cast(Frag, b), f32x4{0.f, 0.f, 0.f, 0.f});
    return d[0] + d[1];
}

// v0 for x < c1, v1 for x < c2, v2 for x < c3, else v3 (c1 <= c2 <= c3), as
// selects of values.
__device__ __forceinline__ int pick4(int x, int c1, int c2, int c3, int v0, int v1, int v2, int v3) {
    const int lo = x < c1 ? v0 : v1, hi = x < c3 ? v2 : v3;
    return x < c2 ? lo : hi;
}

// Block kinds of k_project_pool.
constexpr int kQV = 0, kKG = 1, kKL = 2, kPost = 3;

template <typename T, int KS>
__global__ __launch_bounds__(64 * kProjWaves)
__attribute__((amdgpu_waves_per_eu(2))) void k_project_pool(ProjDev a, PoolFuseDev p) {
    typedef Mma<T> M;
    typedef typename M::Frag Frag;
    constexpr int DIM = 16 * KS;
    constexpr int WS = DIM + 8;
    constexpr int PIECES = 32 * DIM / 8;
    constexpr int PPT = (PIECES + 64 * kProjWaves - 1) / (64 * kProjWaves);
    constexpr int OS = 32 + 8;
    __shared__ __align__(16) float lw[DIM], lb[DIM];
    __shared__ __align__(16) T wbuf[2][32 * WS];
    __shared__ __align__(16) T otile[kProjWaves][32 * OS];
    extern __shared__ __align__(16) unsigned char pool_lds[];
    const int G = p.G, D = p.D, GD = p.GD, KGS = GD + 8;
    T* rows_all = reinterpret_cast<T*>(pool_lds);
    T* wts_all = rows_all + kProjWaves * 32 * KGS;
    float* xch_all = reinterpret_cast<float*>(wts_all + kProjWaves * G * 64);
    int4* meta = reinterpret_cast<int4*>(xch_all + kProjWaves * 16);
    float* lwp = reinterpret_cast<float*>(meta + GD / 2);
    float* lbias = lwp + D;
    // Wave-uniform quantities in scalar registers: the batch and token of the
    // wave's first row (rows < 2^31, and a wave's 32 rows never straddle a
    // batch since tokens is a multiple of 64).
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int lane = threadIdx.x & 63, g = lane >> 5, t = lane & 31;
    const int64_t tok0 = ((int64_t)blockIdx.x * kProjWaves + wave) * 32, tok = tok0 + t;
    const int bw = (int)tok0 / p.tokens, n0 = (int)tok0 - bw * p.tokens;
    // rows is a multiple of 64: a wave, and the pair that holds its fine block,
    // is wholly live or not.
    const bool live = tok0 < a.rows;
    // The token rows and their rotary coordinates first: their latency passes
    // under the set-up below.
    u32x4 xraw[KS];
    layer_norm_load<T, KS>(a, tok, live, g, xraw);
    int pos[3];
    {
        // rope_position32 without its branch (a branch here doubled the
        // kernel's registers): a packed rotation reads three words of the
        // pair table, always valid, and discards them.
        const int n = live ? n0 + t : 0;
        const int* c = p.rope.packed ? p.rope.pairs : reinterpret_cast<const int*>(p.rope.coords) + 6 * n;
        const int c0 = c[0], c1 = c[2], c2 = c[4];
        pos[0] = p.rope.packed ? n : c0;
        pos[1] = p.rope.packed ? 0 : c1;
        pos[2] = p.rope.packed ? 0 : c2;
    }
    for (int c = threadIdx.x; c < DIM; c += blockDim.x) {
        lw[c] = load_any(a.ln_w, c, a.ln_dtype);
        lb[c] = load_any(a.ln_b, c, a.ln_dtype);
    }
    for (int j = threadIdx.x; j < GD / 2; j += blockDim.x) meta[j] = pair_meta(p.rope.pairs, j % (D / 2));
    for (int c = threadIdx.x; c < D; c += blockDim.x) lwp[c] = p.weight[c];
    for (int c = threadIdx.x; c < 64; c += blockDim.x) lbias[c] = p.bias[c];
    const int kg0 = p.kg0, vg0 = kg0 + GD, gbase = a.q_out + a.kv_out, nout = gbase + 2 * a.heads;
    const int kl0 = a.q_out, vl0 = a.q_out + GD;
    // Blocks of 32 output rows, in this order: q [0, kl0) and vl [vl0, kg0)
    // in [0, c1); kg block k and kl block k alternately in [c1, c2) (the two
    // share the rotation of their channels); vg [vg0, gbase) in [c2, c3); the
    // gate logits [gbase, nout) after.
    const int nq = (a.q_out + 31) / 32, nk = (GD + 31) / 32;
    const int c1 = nq + nk, c2 = c1 + 2 * nk, c3 = c2 + nk;
    const int nblocks = c3 + (2 * a.heads + 31) / 32;
    // Values through selects (pick4), not conditionals over captured
    // variables, which the compiler turns into loads from the closure in
    // scratch memory.
    auto start_of = [=](int ob) __attribute__((always_inline)) -> int {
        const int j = ob - c1;
        return pick4(ob, c1, c2, c3, ob < nq ? 32 * ob : vl0 + 32 * (ob - nq), (j & 1 ? kl0 : kg0) + 32 * (j >> 1),
                     vg0 + 32 * (ob - c2), gbase + 32 * (ob - c3));
    };
    auto end_of = [=](int ob) __attribute__((always_inline)) -> int {
        return pick4(ob, c1, c2, c3, ob < nq ? kl0 : kg0, (ob - c1) & 1 ? vl0 : vg0, gbase, nout);
    };
    // Weight row o of the concatenation [Wq; Wkv; Wg].
    auto wrow = [&](int o) __attribute__((always_inline)) -> const T* {
        return o < a.q_out ? reinterpret_cast<const T*>(a.wq) + (int64_t)o * DIM
               : o < gbase ? reinterpret_cast<const T*>(a.wkv) + (int64_t)(o - a.q_out) * DIM
                           : reinterpret_cast<const T*>(a.wg) + (int64_t)(o - gbase) * DIM;
    };
    u32x4 wreg[PPT];
    auto fetch = [&](int ob) __attribute__((always_inline)) {
        // A block's rows are consecutive rows of one weight matrix.  Loads as
        // k_project's: rows past the block's end repeat its last row (their
        // outputs are never stored or summed).
        const int o0 = start_of(ob), n = end_of(ob) - o0;
        const T* wbase = wrow(o0);
#pragma unroll
        for (int i = 0; i < PPT; ++i) {
            const int pc = threadIdx.x + i * 64 * kProjWaves, pcc = min(pc, PIECES - 1);
            const int r = pcc / (DIM / 8), c = (pcc % (DIM / 8)) * 8;
            wreg[i] = *reinterpret_cast<const u32x4*>(wbase + (int64_t)min(r, n - 1) * DIM + c);
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
    fetch(min(1, nblocks - 1));
    __syncthreads();

    T* tile = otile[wave];
    T* krows = rows_all + wave * 32 * KGS;
    float* sums = reinterpret_cast<float*>(krows);  // after the kg sums: kg sums, vg sums, key squares
    T* wts = wts_all + wave * G * 64;
    float* xch = xch_all + wave * 16;
    const float* xch_pair = xch_all + (wave ^ 1) * 16;

    Frag xf[KS];  // the LayerNorm'd row, computed after the first table loads are issued

    T* go = reinterpret_cast<T*>(a.gate) + tok * a.heads;
    // (cos, sin) of the lane's rotary pairs in kg (and kl) block k (channels
    // c .. c + 3 for c = 32 k + 8 qd + 4 g, pairs of one head since 4 | D),
    // loaded a block ahead so that the table reads' latency hides behind a
    // block's GEMM.
    float2 csn[8];
    auto load_cs = [&](int k) __attribute__((always_inline)) {
#pragma unroll
        for (int qd = 0; qd < 4; ++qd) {
            const int c = min(32 * k + 8 * qd + 4 * g, GD - 4);
#pragma unroll
            for (int pp = 0; pp < 2; ++pp) {
                const int4 m = meta[(c >> 1) + pp];
                csn[2 * qd + pp] = p.rope.table[m.x + m.y * pos[0] + m.z * pos[1] + m.w * pos[2]];
            }
        }
    };
    // One output block: the GEMM, then the epilogue of its kind: kQV (q, vl)
    // and kKL (kl, rotated when rotate_kl) stored; kKG rotated and kept in
    // LDS for the pooling; kPost vg (weighted sums) and the gate logits.  The block loop runs in two
    // parts around the slot softmax, so no value of that phase is hoisted
    // into a loop and held across it.
    auto run_block = [&](int ob, auto kind_tag) __attribute__((always_inline)) {
        constexpr int K = decltype(kind_tag)::value;
        const int o_first = start_of(ob), o_end = end_of(ob);
        const T* wb = &wbuf[ob & 1][t * WS + 8 * g];
        // A kl block rotates with the (cos, sin) of its kg block, the one just
        // before it, and then loads those of the next kg block.
        float2 cs_kl[8];
        if constexpr (K == kKL) {
#pragma unroll
            for (int k = 0; k < 8; ++k) cs_kl[k] = csn[k];
            load_cs(min(((ob - c1) >> 1) + 1, nk - 1));  // unconditional: the same loads in every block
        }
        f32x16 d;
#pragma unroll
        for (int r = 0; r < 16; ++r) d[r] = 0.f;
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) d = M::mfma(*reinterpret_cast<const Frag*>(wb + 16 * ks), xf[ks], d);
        if constexpr (K == kQV || K == kKL) {
            // q / kl / vl through the tile as coalesced 16-byte row pieces (as k_project);
            // with rotate_kl the kl values are rounded, rotated and rounded again.
#pragma unroll
            for (int qd = 0; qd < 4; ++qd) {
                float v[4] = {d[4 * qd], d[4 * qd + 1], d[4 * qd + 2], d[4 * qd + 3]};
                if (K == kKL && p.rotate_kl) {
#pragma unroll
                    for (int i = 0; i < 4; ++i) v[i] = to_f32(from_f32<T>(v[i]));
#pragma unroll
                    for (int pp = 0; pp < 2; ++pp)
                        rotate_pair(v[2 * pp], v[2 * pp + 1], cs_kl[2 * qd + pp].x, cs_kl[2 * qd + pp].y);
                }
                store4<T>(tile + t * OS + acc_row(4 * qd, g), v);
            }
            wave_lds_sync();
            // The block's outputs lie wholly in q or wholly in kv: one
            // resource over the wave's 32 rows of that tensor.
            const bool in_q = o_first < a.q_out;
            const int ostride = in_q ? a.q_out : a.kv_out;
            T* obase = in_q ? reinterpret_cast<T*>(a.q) + tok0 * a.q_out + o_first
                            : reinterpret_cast<T*>(a.kv) + tok0 * a.kv_out + (o_first - a.q_out);
            const uint32_t obytes = 32u * ostride * sizeof(T);
            const __amdgpu_buffer_rsrc_t orsrc = buffer_rsrc(obase, obytes);
#pragma unroll
            for (int i = 0; i < 2; ++i) {
                const int tt = 16 * i + (lane >> 2), pp = lane & 3;
                const u32x4 piece = *reinterpret_cast<const u32x4*>(tile + tt * OS + 8 * pp);
                buffer_store16(orsrc, obytes, (uint32_t)(tt * ostride + 8 * pp) * sizeof(T),
                               live && o_first + 8 * pp < o_end, piece);
            }
            wave_lds_sync();  // the next block's tile writes follow these reads
        } else if constexpr (K == kKG) {
            // kg: lane (t, g) holds channels c .. c + 3 of token t for c =
            // o_first - kg0 + 8 qd + 4 g, two rotary pairs of one head (4 | D).
            float2 cs[8];
#pragma unroll
            for (int k = 0; k < 8; ++k) cs[k] = csn[k];
#pragma unroll
            for (int qd = 0; qd < 4; ++qd) {
                const int c = o_first - kg0 + 8 * qd + 4 * g;
                if (c < GD) {
                    float x[4];
#pragma unroll
                    for (int i = 0; i < 4; ++i) x[i] = to_f32(from_f32<T>(d[4 * qd + i]));
#pragma unroll
                    for (int pp = 0; pp < 2; ++pp) rotate_pair(x[2 * pp], x[2 * pp + 1], cs[2 * qd + pp].x, cs[2 * qd + pp].y);
                    store4<T>(krows + t * KGS + c, x);
                }
            }
        } else if (ob < c3) {
            // vg: the rounded block through the tile, then the weighted sums of
            // its 16-channel tiles over the wave's tokens.
#pragma unroll
            for (int qd = 0; qd < 4; ++qd) {
                const float v[4] = {d[4 * qd], d[4 * qd + 1], d[4 * qd + 2], d[4 * qd + 3]};
                store4<T>(tile + t * OS + acc_row(4 * qd, g), v);
            }
            wave_lds_sync();
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                const int c = o_first - vg0 + 16 * j;
                if (c < GD) {
                    const float s = slot_sum<T>(wts + (c / D) * 64, tile + 16 * j, OS, lane);
                    if (lane < 16) sums[GD + c + lane] = s;
                }
            }
            wave_lds_sync();  // the next block's tile writes follow these reads
        } else if (live && o_first + 32 > gbase) {
#pragma unroll
            for (int qd = 0; qd < 4; ++qd) {
                const int o0 = o_first + acc_row(4 * qd, g);  // outputs o0 .. o0 + 3
                float v[4] = {d[4 * qd], d[4 * qd + 1], d[4 * qd + 2], d[4 * qd + 3]};
                if (o0 >= gbase && o0 < nout) {
                    // Logit pairs (2h, 2h + 1) of heads h = (o0 - gbase) / 2 + {0, 1}.
#pragma unroll
                    for (int q2 = 0; q2 < 2; ++q2) {
                        const int j = o0 - gbase + 2 * q2;
                        if (j + 1 >= 2 * a.heads) break;
                        const float l0 =
                            to_f32(from_f32<T>(v[2 * q2] + load_any(a.gate_bias, j, a.gate_bias_dtype)));
                        const float l1 =
                            to_f32(from_f32<T>(v[2 * q2 + 1] + load_any(a.gate_bias, j + 1, a.gate_bias_dtype)));
                        const float m = fmaxf(l0, l1);
                        const float e0 = expf(l0 - m), e1 = expf(l1 - m);
                        go[j / 2] = from_f32<T>(e1 / (e0 + e1));
                    }
                }
            }
        }
        // Unconditional (a stage after the last block fills a buffer no
        // block reads), so that every block issues the same loads.
        stage((ob + 1) & 1);
        fetch(min(ob + 2, nblocks - 1));
        __syncthreads();
    };
    load_cs(0);
    layer_norm_math<T, KS>(a, lw, lb, g, xraw, xf);
    settle_loads(wreg, xf);  // the table loads stay in flight under the q / vl blocks
    for (int ob = 0; ob < c1; ++ob) run_block(ob, std::integral_constant<int, kQV>{});
    for (int ob = c1; ob < c2; ob += 2) {
        run_block(ob, std::integral_constant<int, kKG>{});
        run_block(ob + 1, std::integral_constant<int, kKL>{});
    }
    {
        // Slot logits of the wave's 32 tokens for every head: lane (t, g)
        // takes half g of each head's channels, lane t ^ 32 the other.
        const int slot = 32 * (wave & 1) + t;
        float logit[8];
#pragma unroll
        for (int h = 0; h < 8; ++h) {
            if (h >= G) break;
            const T* row = krows + t * KGS + h * D + g * (D / 2);
            float dot = 0.f;
            for (int i = 0; i < D / 2; i += 8) {
                const u32x4 piece = *reinterpret_cast<const u32x4*>(row + i);
                const T* v = reinterpret_cast<const T*>(&piece);
#pragma unroll
                for (int e = 0; e < 8; ++e) dot += to_f32(v[e]) * lwp[g * (D / 2) + i + e];
            }
            dot += lane_xor32(dot);
            logit[h] = dot * p.inv_tau + lbias[slot];
            const float mx = wave_max(logit[h]);
            if (lane == 0) xch[h] = mx;
        }
        __syncthreads();
#pragma unroll
        for (int h = 0; h < 8; ++h) {
            if (h >= G) break;
            logit[h] = expf(logit[h] - fmaxf(xch[h], xch_pair[h]));
            const float s = wave_sum(g ? 0.f : logit[h]);
            if (lane == 0) xch[8 + h] = s;
        }
        __syncthreads();
#pragma unroll
        for (int h = 0; h < 8; ++h) {
            if (h >= G) break;
            const float wgt = logit[h] / (xch[8 + h] + xch_pair[8 + h]);
            if (g == 0) {
                const T hi = from_f32<T>(wgt);
                wts[h * 64 + t] = hi;
                wts[h * 64 + 32 + t] = from_f32<T>(wgt - to_f32(hi));
            }
        }
        wave_lds_sync();
        // The kg sums, 16 channels per MFMA, parked in the wave's idle output
        // tile and then moved over the rows, which are no longer needed.
        float* park = reinterpret_cast<float*>(tile);
#pragma unroll 4
        for (int j = 0; 16 * j < GD; ++j) {
            const float s = slot_sum<T>(wts + (16 * j / D) * 64, krows + 16 * j, KGS, lane);
            if (lane < 16) park[16 * j + lane] = s;
        }
        wave_lds_sync();
        for (int c = lane; c < GD; c += 64) sums[c] = park[c];
        wave_lds_sync();  // the next block's tile writes follow these reads
    }
    for (int ob = c2; ob < nblocks; ++ob) run_block(ob, std::integral_constant<int, kPost>{});

    // The fine block's summaries: the even wave adds its partner's sums (the
    // last block's barrier orders them).
    if (!live || (wave & 1)) return;
    const int b = bw, m = n0 / 64;
    const float* pair = reinterpret_cast<const float*>(krows + 32 * KGS);
    float* nsq = sums + 2 * GD;
    for (int c = lane; c < GD; c += 64) {
        const int h = c / D, cc = c - h * D;
        const int64_t bg = (int64_t)b * G + h;
        const T kx = from_f32<T>((sums[c] + pair[c]) * p.key_scale);
        const T vx = from_f32<T>(sums[GD + c] + pair[GD + c]);
        reinterpret_cast<T*>(p.sk)[(bg * p.Mp + m) * D + cc] = kx;
        reinterpret_cast<T*>(p.svt)[((bg * (p.Mp / 32) + m / 32) * D + cc) * 32 + (m & 31)] = vx;
        nsq[c] = to_f32(kx) * to_f32(kx);
    }
    wave_lds_sync();
    if (lane < G) {
        float sq = 0.f;
        for (int c = 0; c < D; ++c) sq += nsq[lane * D + c];
        // Norm of the stored (rounded) summary key; non-negative floats order
        // like their bit patterns, so an integer max is an exact float max.
        const float norm = sqrtf(sq) * (1.f + 1e-6f);
        atomicMax(reinterpret_cast<int*>(p.norm) + ((int64_t)b * G + lane) * 64 + (m % 64), __float_as_int(norm));
    }
}

// Output projection with the residual (attention.py:89): out = x + y Wo^T
// for y [rows, K] (the core's output, heads concatenated), Wo [dim, K] and
// x, out [rows, dim]: the same tiling as k_project without the LayerNorm (y
// is the B operand as loaded), 32 outputs per block.  The block's fp32
// accumulators go through the wave's tile, and the store phase adds the
// residual piece and rounds once, as a GEMM with the residual as its C
// operand does.  With a residual and output R = float (autocast over an fp32
// input), the product is rounded to T and added to the unrounded residual in
// fp32, as the reference's ``residual + to_out(...)`` does there.
template <typename T, int KS, typename R>
__global__ __launch_bounds__(64 * kProjWaves) __attribute__((amdgpu_waves_per_eu(KS <= 12 ? 4 : 2)))
void k_out_residual(const T* __restrict__ y, const T* __restrict__ wo, const R* __restrict__ x, R* __restrict__ out,
                    int64_t rows, int dim) {
    constexpr int RP = (int)sizeof(R) / 2;  // 16-byte pieces per 8 outputs
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
    const int lane = threadIdx.x & 63, g = lane >> 5, t = lane & 31;
    const int64_t tok0 = ((int64_t)blockIdx.x * kProjWaves + (threadIdx.x >> 6)) * 32, tok = tok0 + t;
    const bool live = tok < rows;
    float* tile = otile[threadIdx.x >> 6];
    const uint32_t obytes = 32u * dim * sizeof(R);
    const __amdgpu_buffer_rsrc_t orsrc = buffer_rsrc(out + tok0 * dim, obytes);
    // The token rows and the first residual pieces first: their latency
    // passes under the first weight block's fetch and staging.
    const T* yr = y + (live ? tok : 0) * K + 8 * g;
    Frag yf[KS];
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) yf[ks] = __builtin_bit_cast(Frag, *reinterpret_cast<const u32x4*>(yr + 16 * ks));
    // Residual pieces: lane (tt = 16 i + lane / 4, pp = lane % 4) of block ob
    // adds x[tok0 + tt][32 ob + 8 pp .. + 8].
    auto load_res = [&](int ob, u32x4 (*r)[RP]) __attribute__((always_inline)) {
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const int64_t tk = min(tok0 + 16 * i + (lane >> 2), rows - 1);
#pragma unroll
            for (int h = 0; h < RP; ++h)
                r[i][h] = *reinterpret_cast<const u32x4*>(x + tk * dim + 32 * ob + 8 * (lane & 3) + h * (8 / RP));
        }
    };
    // Each block's residual pieces are loaded a block ahead, into the
    // registers the block before has just consumed (a copy between two sets
    // would wait for the loads in flight).  Per block the vector memory
    // operations go: stores, next residual, next weights; each wait then
    // falls on loads issued a block earlier.
    u32x4 resv[2][RP];
    load_res(0, resv);
    u32x4 wreg[PPT];
    auto fetch = [&](int ob) __attribute__((always_inline)) {
#pragma unroll
        for (int i = 0; i < PPT; ++i) {
            const int pc = threadIdx.x + i * 64 * kProjWaves, pcc = min(pc, PIECES - 1);
            const int r = pcc / (K / 8), c = (pcc % (K / 8)) * 8;
            wreg[i] = *reinterpret_cast<const u32x4*>(wo + (int64_t)(32 * ob + r) * K + c);
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
    fetch(min(1, nblocks - 1));
    __syncthreads();
    settle_loads(wreg, yf, resv);

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
            const f32x4 lo = *reinterpret_cast<const f32x4*>(tile + tt * OS + 8 * pp);
            const f32x4 hi = *reinterpret_cast<const f32x4*>(tile + tt * OS + 8 * pp + 4);
            const R* rv = reinterpret_cast<const R*>(&resv[i][0]);
            u32x4 o[RP];
            R* ov = reinterpret_cast<R*>(&o[0]);
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                if constexpr (std::is_same<R, float>::value) {
                    ov[e] = to_f32(from_f32<T>(lo[e])) + rv[e];
                    ov[4 + e] = to_f32(from_f32<T>(hi[e])) + rv[4 + e];
                } else {
                    ov[e] = from_f32<T>(lo[e] + to_f32(rv[e]));
                    ov[4 + e] = from_f32<T>(hi[e] + to_f32(rv[4 + e]));
                }
            }
            // Masked stores without a branch: the next block's wait for its
            // weights then counts past them.
#pragma unroll
            for (int h = 0; h < RP; ++h)
                buffer_store16(orsrc, obytes, (uint32_t)(tt * dim + o0 + h * (8 / RP)) * sizeof(R), tok0 + tt < rows,
                               o[h]);
        }
        load_res(min(ob + 1, nblocks - 1), resv);
        wave_lds_sync();
        // Unconditional (a stage after the last block fills a buffer no
        // block reads), so that every block issues the same loads.
        stage((ob + 1) & 1);
        fetch(min(ob + 2, nblocks - 1));
        __syncthreads();
    }
}

template <typename T, bool LIN>
int launch_project(const ProjDev& d, hipStream_t s) {
    const unsigned blocks = (unsigned)cdiv(cdiv(d.rows, 32), kProjWaves);
    switch (d.dim) {
#define CASE(DIM)                                                                     \
    case DIM:                                                                         \
        k_project<T, DIM / 16, LIN><<<blocks, 64 * kProjWaves, 0, s>>>(d);            \
        break;
        CASE(64) CASE(96) CASE(128) CASE(192) CASE(256) CASE(384) CASE(512)
#undef CASE
        default: return fail(P3D_EUNSUPPORTED, "dim must be one of 64, 96, 128, 192, 256, 384, 512");
    }
    return check_launch(LIN ? "p3d_project_linear" : "p3d_project");
}

template <typename T, typename R>
int launch_out_residual(const void* y, const void* wo, const void* x, void* out, int64_t rows, int k, int dim,
                        hipStream_t s) {
    const unsigned blocks = (unsigned)cdiv(cdiv(rows, 32), kProjWaves);
    switch (k) {
#define CASE(KK)                                                                                                  \
    case KK:                                                                                                      \
        k_out_residual<T, KK / 16, R><<<blocks, 64 * kProjWaves, 0, s>>>((const T*)y, (const T*)wo, (const R*)x, \
                                                                         (R*)out, rows, dim);                     \
        break;
        CASE(64) CASE(96) CASE(128) CASE(192) CASE(256) CASE(384) CASE(512)
#undef CASE
        default: return fail(P3D_EUNSUPPORTED, "heads * head_dim must be one of 64, 96, 128, 192, 256, 384, 512");
    }
    return check_launch("p3d_out_residual");
}

template <typename T>
int launch_project_pool(const ProjDev& d, const PoolFuseDev& p, hipStream_t s) {
    const unsigned blocks = (unsigned)cdiv(cdiv(d.rows, 32), kProjWaves);
    const size_t smem = pool_fuse_lds_bytes(p.G, p.D);
    switch (d.dim) {
#define CASE(DIM)                                                                     \
    case DIM:                                                                         \
        k_project_pool<T, DIM / 16><<<blocks, 64 * kProjWaves, smem, s>>>(d, p);      \
        break;
        CASE(64) CASE(96) CASE(128) CASE(192) CASE(256)
#undef CASE
        default: return fail(P3D_EUNSUPPORTED, "pooled projections: dim must be one of 64, 96, 128, 192, 256");
    }
    return check_launch("p3d_project_pool");
}

__global__ void k_zero_norm_slots(float* p, int n) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) p[i] = 0.f;
}

}  // namespace
}  // namespace p3d

using namespace p3d;

extern "C" int p3d_out_residual(const void* y, const void* wo, const void* x, void* out, int64_t rows, int32_t k,
                                int32_t dim, int32_t dtype, int32_t res_dtype, void* stream) {
    P3D_REQUIRE(y && wo && x && out, "null pointer argument");
    P3D_REQUIRE(dtype == P3D_F16 || dtype == P3D_BF16, "dtype must be fp16 or bf16");
    P3D_REQUIRE(res_dtype == dtype || res_dtype == P3D_F32, "the residual must be of dtype or fp32");
    P3D_REQUIRE(rows >= 1, "need at least one row");
    P3D_REQUIRE(dim >= 32 && dim % 32 == 0 && dim <= kProjMaxDim, "dim must be a multiple of 32, at most 512");
    P3D_REQUIRE(aligned16(y) && aligned16(wo) && aligned16(x) && aligned16(out), "pointers must be 16-byte aligned");
    P3D_REQUIRE(cdiv(rows, 32 * kProjWaves) < (1LL << 31), "too many rows");
    hipStream_t s = as_stream(stream);
    if (res_dtype == P3D_F32)
        return dtype == P3D_F16 ? launch_out_residual<_Float16, float>(y, wo, x, out, rows, k, dim, s)
                                : launch_out_residual<__bf16, float>(y, wo, x, out, rows, k, dim, s);
    return dtype == P3D_F16 ? launch_out_residual<_Float16, _Float16>(y, wo, x, out, rows, k, dim, s)
                            : launch_out_residual<__bf16, __bf16>(y, wo, x, out, rows, k, dim, s);
}

namespace {

// Validates the projection arguments and fills the kernels' argument block
// (linear: no LayerNorm, whose parameters are then not read).
int project_dev(const p3d_project_args& a, ProjDev& d, bool linear = false) {
    P3D_REQUIRE(a.dtype == P3D_F16 || a.dtype == P3D_BF16, "dtype must be fp16 or bf16");
    P3D_REQUIRE((linear || (a.ln_dtype >= P3D_F32 && a.ln_dtype <= P3D_BF16)) && a.gate_bias_dtype >= P3D_F32 &&
                    a.gate_bias_dtype <= P3D_BF16,
                "unknown parameter dtype");
    P3D_REQUIRE(a.x && (linear || (a.ln_weight && a.ln_bias)) && a.wq && a.wkv && a.wg && a.gate_bias && a.q &&
                    a.kv && a.gate,
                "null pointer argument");
    P3D_REQUIRE(a.rows >= 1 && a.heads >= 1, "empty projection problem");
    P3D_REQUIRE(a.dim >= 16 && a.dim <= kProjMaxDim && a.dim % 16 == 0, "dim must be a multiple of 16, at most 512");
    P3D_REQUIRE(a.q_out >= 16 && a.q_out % 16 == 0 && a.kv_out >= 16 && a.kv_out % 16 == 0,
                "q_out and kv_out must be positive multiples of 16");
    P3D_REQUIRE(aligned16(a.x) && aligned16(a.wq) && aligned16(a.wkv) && aligned16(a.wg),
                "x and the weights must be 16-byte aligned");
    P3D_REQUIRE(aligned16(a.q) && aligned16(a.kv), "q and kv must be 16-byte aligned");
    P3D_REQUIRE(cdiv(a.rows, 32 * kProjWaves) < (1LL << 31), "too many rows");
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
    return P3D_OK;
}

}  // namespace

extern "C" int p3d_project(const p3d_project_args* args, void* stream) {
    P3D_REQUIRE(args, "null args");
    ProjDev d;
    if (int rc = project_dev(*args, d)) return rc;
    hipStream_t s = as_stream(stream);
    return args->dtype == P3D_F16 ? launch_project<_Float16, false>(d, s) : launch_project<__bf16, false>(d, s);
}

extern "C" int p3d_project_linear(const p3d_project_args* args, void* stream) {
    P3D_REQUIRE(args, "null args");
    ProjDev d;
    if (int rc = project_dev(*args, d, true)) return rc;
    hipStream_t s = as_stream(stream);
    return args->dtype == P3D_F16 ? launch_project<_Float16, true>(d, s) : launch_project<__bf16, true>(d, s);
}

extern "C" int p3d_project_pool(const p3d_project_args* args, const p3d_pool_args* pool, int32_t rotate_kl,
                                void* stream) {
    P3D_REQUIRE(args && pool, "null args");
    ProjDev d;
    int rc = project_dev(*args, d);
    if (rc) return rc;
    const p3d_pool_args& q = *pool;
    P3D_REQUIRE(q.dtype == args->dtype, "pooling and projections disagree on the dtype");
    P3D_REQUIRE(q.weight && q.bias && q.sk && q.svt && q.sk_norm_max && q.rope.table && q.rope.pairs &&
                    (q.rope.packed || q.rope.coords),
                "null pointer argument");
    P3D_REQUIRE(q.temperature > 0.f, "temperature must be positive");
    P3D_REQUIRE(q.kv_heads >= 1 && q.head_dim >= 16 && args->kv_out == 4 * q.kv_heads * q.head_dim,
                "kv_out must be 4 * kv_heads * head_dim");
    P3D_REQUIRE(q.tokens >= 64 && (int64_t)q.batch * q.tokens == args->rows,
                "rows must be batch * tokens");
    // Shapes the fused kernel does not take (the caller runs p3d_project and
    // p3d_pool_fwd instead); nothing has been launched.
    if (!(q.head_dim == 16 || q.head_dim == 32 || q.head_dim == 48 || q.head_dim == 64) || q.kv_heads > 8 ||
        q.kv_heads * q.head_dim > kPoolFuseMaxCh || q.slots != 64 || q.pool_size != 1 || q.tokens % 64 ||
        q.fine_blocks != q.tokens / 64 || q.summaries != q.fine_blocks ||
        !(args->dim == 64 || args->dim == 96 || args->dim == 128 || args->dim == 192 || args->dim == 256) ||
        project_static_lds_bytes(args->dim) + pool_fuse_lds_bytes(q.kv_heads, q.head_dim) > 160 * 1024)
        return fail(P3D_EUNSUPPORTED,
                    "pooled projections need head_dim 16/32/48/64, kv_heads * head_dim <= 192, 64-slot fine "
                    "blocks of pool_size 1 over tokens a multiple of 64, and dim 64/96/128/192/256 within the LDS");
    // k_project_pool indexes tokens, batches and summaries in 32 bits.
    if (args->rows >= ((int64_t)1 << 31))
        return fail(P3D_EUNSUPPORTED, "pooled projections take fewer than 2^31 rows");
    PoolFuseDev p;
    p.G = q.kv_heads;
    p.D = q.head_dim;
    p.GD = q.kv_heads * q.head_dim;
    p.Mp = (int)cdiv(q.summaries, 32) * 32;
    p.tokens = q.tokens;
    p.kg0 = args->q_out + 2 * p.GD;
    p.inv_tau = 1.f / q.temperature;
    p.key_scale = q.key_scale;
    p.weight = q.weight;
    p.bias = q.bias;
    p.rope = rope_dev(q.rope);
    p.sk = (char*)q.sk;
    p.svt = (char*)q.svt;
    p.norm = q.sk_norm_max;
    p.rotate_kl = rotate_kl != 0;
    hipStream_t s = as_stream(stream);
    if (!q.norms_cleared) {
        const int n = q.batch * q.kv_heads * 64;
        k_zero_norm_slots<<<(unsigned)cdiv(n, 256), 256, 0, s>>>(q.sk_norm_max, n);
        rc = check_launch("p3d_project_pool (norm slots)");
        if (rc) return rc;
    }
    return args->dtype == P3D_F16 ? launch_project_pool<_Float16>(d, p, s) : launch_project_pool<__bf16>(d, p, s);
}
