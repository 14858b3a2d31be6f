// Summary pooling (compression.py:28-44 of amilworks/Pack3D) and the
// standalone rotation (rotary.py:10-45).
//
// One wave pools one coarse summary of one (batch, kv head).  For each of its
// fine blocks the wave issues every 16-byte load of the block's K and V rows
// at once (lane l holds pieces l, l + 64, ... of the 64 x D/EP piece grid)
// and writes them to LDS as rows with 16-byte stores.  Then one lane per
// slot reads its K row, rotates it, rounds it to the storage type (the
// reference pools rotated keys stored in that type), writes it back and
// forms the slot logit; the slot softmax is a wave reduction.  The forward
// takes the weighted sums over the slots on MFMA (k_pool_fwd); the backward
// forms its column sums with one lane per column dword (column_sums_w).  The
// coarse mean divides by the number of non-empty fine blocks.
#include <algorithm>
#include <type_traits>

#include "rope.hpp"

namespace p3d {
namespace {

// Summary-norm maxima are spread over this many slots per (batch, kv head) so
// that the atomics of different waves rarely meet on one address.
constexpr int kNormSlots = 64;

struct PoolDev {
    int B, G, N, F, V, P, M, Mp;
    int bps, gsz;  // fine blocks per 64-lane pooling step; lanes of a block's slot group (64 if bps is 1)
    float inv_tau, key_scale;
    const char *kg, *vg;
    int64_t ksb, ksh, ksn, vsb, vsh, vsn;
    const int32_t* blocks;
    const float* weight;
    const float* bias;
    RopeDev rope;
    int table_entries;  // rope table entries (float2); staged in LDS when it fits
    void* sk;
    void* svt;
    float* sk_norm_max;
};

// Row geometry of the K / V row buffers in LDS: 64 rows (one per slot) of
// row stride D + EP elements.  For the column sums lane (h, u) owns column
// dword u of the slots h, h + S, h + 2S, ...; the row stride is 4 dwords more
// than a row, so the S lane groups read disjoint banks when S rows fit in 64
// banks.
template <typename T, int D>
struct PoolCfg {
    static constexpr int EP = Piece<T>::N;        // elements per 16-byte piece
    static constexpr int PPR = D / EP;             // pieces per row (and per lane, per tensor)
    static constexpr int CPD = 4 / sizeof(T);      // channels per dword
    static constexpr int RD = (D + EP) / CPD;      // row stride in dwords
    static constexpr int DW = D / CPD;             // payload dwords per row
    static constexpr int LW = DW <= 8 ? 8 : (DW <= 16 ? 16 : (DW <= 32 ? 32 : 64));  // lanes per slot group
    static constexpr int S = 64 / LW;              // slot groups
    static constexpr int SJ = (DW + 63) / 64;      // column dwords per lane
};

// Store a tensor's pieces (lane l holds pieces l, l + 64, ... of the 64 x PPR
// grid) as rows of the LDS buffer.
template <typename C>
__device__ __forceinline__ void stage_rows(uint32_t* rows, const uint4 (&r)[C::PPR], int lane) {
#pragma unroll
    for (int i = 0; i < C::PPR; ++i) {
        const int q = i * 64 + lane, s = q / C::PPR, p = q - s * C::PPR;
        *reinterpret_cast<uint4*>(rows + s * C::RD + p * 4) = r[i];
    }
}

// Product of two non-negative values below 2^24, as one 24-bit multiply
// (v_mul_u32_u24; HIP's __mul24 is an out-of-line library call here).
__device__ __forceinline__ int mul_u24(int x, int y) {
    return (int)(((unsigned)x & 0xffffffu) * ((unsigned)y & 0xffffffu));
}

__device__ __forceinline__ float2 pair_cs(const int4& p, const float2* tab, const int pos[3]) {
    // Table indices are below 2^23 (checked on the host): 24-bit products.
    return tab[p.x + mul_u24(p.y, pos[0]) + mul_u24(p.z, pos[1]) + mul_u24(p.w, pos[2])];
}

// Rotate a run of EP channels starting at c0 with (cos, sin) from `tab`
// (the rope table, in LDS or in global memory); meta as built by pair_meta.
template <int EP>
__device__ __forceinline__ void rotate_piece(const int4* meta, const float2* tab, const int pos[3], int c0, float* x) {
#pragma unroll
    for (int e = 0; e < EP; e += 2) {
        const float2 cs = pair_cs(meta[(c0 + e) >> 1], tab, pos);
        rotate_pair(x[e], x[e + 1], cs.x, cs.y);
    }
}

// The inverse rotation R^T of rotate_piece (rotation by -theta).
template <int EP>
__device__ __forceinline__ void rotate_piece_inverse(const int4* meta, const float2* tab, const int pos[3], int c0,
                                                     float* x) {
#pragma unroll
    for (int e = 0; e < EP; e += 2) {
        const float2 cs = pair_cs(meta[(c0 + e) >> 1], tab, pos);
        rotate_pair(x[e], x[e + 1], cs.x, -cs.y);
    }
}

// column_sums with the slot weights read from LDS (w[s] for slot s).
template <typename C, typename T>
__device__ __forceinline__ void column_sums_w(const uint32_t* rows, const float* w, int lane,
                                              float (&out)[C::SJ][C::CPD]) {
    const int h = lane / C::LW, u0 = lane % C::LW;
    float part[C::SJ][C::CPD];
#pragma unroll
    for (int j = 0; j < C::SJ; ++j)
#pragma unroll
        for (int c = 0; c < C::CPD; ++c) part[j][c] = 0.f;
    for (int i = 0; i < 64 / C::S; ++i) {
        const int s = i * C::S + h;
        const float ws = w[s];
#pragma unroll
        for (int j = 0; j < C::SJ; ++j) {
            // Lanes past the last column re-read it (no divergent branch);
            // their sums are never stored.
            const uint32_t raw = rows[s * C::RD + min(u0 + 64 * j, C::DW - 1)];
            const T* x = reinterpret_cast<const T*>(&raw);
#pragma unroll
            for (int c = 0; c < C::CPD; ++c) part[j][c] += ws * to_f32(x[c]);
        }
    }
#pragma unroll
    for (int o = C::LW; o < 64; o <<= 1)
#pragma unroll
        for (int j = 0; j < C::SJ; ++j)
#pragma unroll
            for (int c = 0; c < C::CPD; ++c) part[j][c] += __shfl_xor(part[j][c], o);
#pragma unroll
    for (int j = 0; j < C::SJ; ++j)
#pragma unroll
        for (int c = 0; c < C::CPD; ++c) out[j][c] += part[j][c];
}

// Round the EP channels of a piece to T in place (x then holds the rounded
// values) and return them packed as one 16-byte piece.  bf16 pairs take one
// packed round-to-nearest-even conversion each.
template <typename T, int EP>
__device__ __forceinline__ uint4 round_piece(float (&x)[EP]) {
    uint4 raw;
    T* t = reinterpret_cast<T*>(&raw);
#pragma unroll
    for (int e = 0; e < EP; ++e) {
        t[e] = from_f32<T>(x[e]);
        x[e] = to_f32(t[e]);
    }
    return raw;
}

template <>
__device__ __forceinline__ uint4 round_piece<__bf16, 8>(float (&x)[8]) {
    typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
    uint32_t w[4];
#pragma unroll
    for (int t = 0; t < 4; ++t) {
        w[t] = __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2){x[2 * t], x[2 * t + 1]}, bf16x2));
        x[2 * t] = __uint_as_float(w[t] << 16);
        x[2 * t + 1] = __uint_as_float(w[t] & 0xffff0000u);
    }
    return uint4{w[0], w[1], w[2], w[3]};
}

template <>
__device__ __forceinline__ uint4 round_piece<_Float16, 8>(float (&x)[8]) {
    typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
    uint32_t w[4];
#pragma unroll
    for (int t = 0; t < 4; ++t) {
        const f16x2 r = __builtin_convertvector((f32x2){x[2 * t], x[2 * t + 1]}, f16x2);
        w[t] = __builtin_bit_cast(uint32_t, r);
        x[2 * t] = (float)r.x;
        x[2 * t + 1] = (float)r.y;
    }
    return uint4{w[0], w[1], w[2], w[3]};
}

// ------------------------------------------------------------------ forward
//
// One wave pools one (batch, kv head, summary) item at a time, one step
// after the other.  A step holds bps fine blocks: with V slots per block a
// power of two up to 32, bps = 64 / V and lane l holds slot l % V of block
// l / V of the step (pool_size 16 with 16-slot blocks takes 4 steps instead
// of 16); otherwise bps = 1 and lane l holds slot l.  The slot softmax runs
// over each block's lanes, and the weighted sums over all 64 lanes add the
// step's blocks together, as the coarse mean needs.
//
// The K and V rows of a step are loaded with 16 bytes per lane and
// consecutive lanes on consecutive pieces of a row, so one load instruction
// covers whole row spans, and are written to the wave's LDS buffer as rows.
// (Loading each lane's own K row instead, 64 rows per load instruction, was
// measured slower.)  The loads of the wave's next step are issued into the
// prefetch registers early in a step, so their HBM latency hides behind that
// step's arithmetic.  Each lane reads its own slot's K row back, rotates it,
// rounds it to the storage type (the reference pools rotated keys stored in
// that type), forms the slot logit, and the slot softmax is a wave
// reduction.
//
// 2-byte types: the rotated, rounded K row is written back over its staged
// row, and the weighted sums over the 64 slots, sum_s a_s k_s and
// sum_s a_s v_s, run on MFMA: D = W X with W = [hi(a); lo(a)] (the weights
// split into two storage-type parts, hi = round(a), lo = round(a - hi)) and X
// the staged [64 slots x (K | V)] rows.  Its B operand needs 8 consecutive
// slots of one channel per lane, read straight out of the row-major rows with
// ds_read_b64_tr_b16 (two per fragment).  Each product of two storage-type
// values is exact in fp32 and the sum carries a with 16 significant bits.
//
// fp32: each lane also reads its own V row, and the sums are taken across
// lanes by a reduce-scatter butterfly.

template <typename T, int D>
struct PoolRowCfg {
    static constexpr bool MF = sizeof(T) == 2;       // MFMA slot sums
    static constexpr int EP = Piece<T>::N;          // elements per 16-byte piece
    static constexpr int PPR = D / EP;               // pieces per row
    static constexpr int PFN = (PPR + 3) & ~3;       // run flags, padded to 16 bytes
    static constexpr int RB = D * (int)sizeof(T);    // row bytes
    static constexpr int ROWS_BYTES = 2 * 64 * RB;   // K rows, then V rows
    // MFMA path: the rows, then the weight rows hi and lo (64 slots each).
    static constexpr int WAVE_BYTES = MF ? ROWS_BYTES + 2 * 64 * 2 : ROWS_BYTES;
    static constexpr int MAX_WAVES = (159 * 1024) / WAVE_BYTES < 8 ? (159 * 1024) / WAVE_BYTES : 8;
    static constexpr int VOFF = 64 * RB;             // where the V rows are staged
    static constexpr int NT = 2 * D / 16;            // 16-channel MFMA tiles of [k; v]
    static constexpr int NCH = D / 16;               // 16-channel chunks of the butterfly
    static constexpr int PPC = 16 / EP;              // pieces per chunk
    static constexpr int NACC = MF ? NT : NCH;       // per-lane partial sums
    static constexpr size_t FIXED = (size_t)(D / 2) * 16 + PFN * 4 + D * 4 + 64 * 4;
};

// One halving step of the butterfly between lanes l and l ^ 32 (rows of 32
// lanes swapped): the lower half ends with a summed over the pair, the upper
// half with b summed over the pair.
__device__ __forceinline__ float halve32(float a, float b) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(a), __float_as_uint(b), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// The same between lanes l and l ^ 16 (odd and even 16-lane rows swapped).
__device__ __forceinline__ float halve16(float a, float b) {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(a), __float_as_uint(b), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// The same within a row through a DPP lane permutation CTRL that pairs lanes
// across one lane bit; `upper` is that bit of this lane.
template <int CTRL>
__device__ __forceinline__ float halve_dpp(float a, float b, bool upper) {
    const float keep = upper ? b : a, send = upper ? a : b;
    return keep + dpp_move<CTRL>(send);
}

// Sums k[0..15] and v[0..15] over the 64 lanes of the wave.  Lane l ends
// with the full sum of tensor (l bit 5: 0 = k, 1 = v) at channel
// 8 b4 + 4 b3 + 2 b2 + b1 (bits of l); lanes l and l ^ 1 hold the same value.
// The pairings are l ^ 32, l ^ 16, l ^ 8 (row_ror:8), l ^ 7 (row_half_mirror,
// splitting on bit 2), l ^ 2 and l ^ 1 (quad_perm); their XOR span is the
// whole wave, so every value is a sum over all 64 lanes.
__device__ __forceinline__ float butterfly_sum(const float (&k)[16], const float (&v)[16], int lane) {
    float u[16];
#pragma unroll
    for (int j = 0; j < 16; ++j) u[j] = halve32(k[j], v[j]);
    float w[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) w[j] = halve16(u[j], u[8 + j]);
    float x[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) x[j] = halve_dpp<0x128>(w[j], w[4 + j], lane & 8);
    float y[2];
#pragma unroll
    for (int j = 0; j < 2; ++j) y[j] = halve_dpp<0x141>(x[j], x[2 + j], lane & 4);
    const float z = halve_dpp<0x4E>(y[0], y[1], lane & 2);
    return z + dpp_move<0xB1>(z);
}

template <typename T, int EP>
__device__ __forceinline__ void unpack_piece(const u32x4& raw, float (&x)[EP]) {
    const T* t = reinterpret_cast<const T*>(&raw);
#pragma unroll
    for (int e = 0; e < EP; ++e) x[e] = to_f32(t[e]);
}

// Max / sum over aligned groups of gsz lanes (gsz a power of two): the first
// log2(gsz) steps of wave_max / wave_sum, which reduce within 2, 4, 8, 16
// and 32 lanes in turn.
__device__ __forceinline__ float group_max(float x, int gsz) {
    if (gsz >= 64) return wave_max(x);
    if (gsz >= 2) x = fmaxf(x, dpp_move<0xB1>(x));
    if (gsz >= 4) x = fmaxf(x, dpp_move<0x4E>(x));
    if (gsz >= 8) x = fmaxf(x, dpp_move<0x141>(x));
    if (gsz >= 16) x = fmaxf(x, dpp_move<0x140>(x));
    if (gsz >= 32) x = fmaxf(x, lane_xor16(x));
    return x;
}
__device__ __forceinline__ float group_sum(float x, int gsz) {
    if (gsz >= 64) return wave_sum(x);
    if (gsz >= 2) x += dpp_move<0xB1>(x);
    if (gsz >= 4) x += dpp_move<0x4E>(x);
    if (gsz >= 8) x += dpp_move<0x141>(x);
    if (gsz >= 16) x += dpp_move<0x140>(x);
    if (gsz >= 32) x += lane_xor16(x);
    return x;
}

// Fine blocks of a step with at least one slot token: groups of V lanes of
// the ballot `filled` (bps groups).
__device__ __forceinline__ int blocks_filled(uint64_t filled, int bps, int V) {
    if (bps == 1) return 1;
    const uint64_t group = V == 64 ? ~0ull : ((1ull << V) - 1);
    int n = 0;
    for (int b = 0; b < bps; ++b) n += ((filled >> (b * V)) & group) != 0;
    return n;
}

// Store the summary of (batch * kv head bg, summary m) from the lane's sums
// acc (over the fine blocks of the summary).  MFMA layout: lanes 0..15 hold
// channel 16 t + l of [k; v] in acc[t].  Butterfly layout: lane l holds
// channel 16 k + 8 b4 + 4 b3 + 2 b2 + b1 of tensor b5 in acc[k] (even lanes
// store).  The coarse stage divides the group sum by the count of non-empty
// fine blocks (compression.py:42-43); keys are stored times key_scale.
template <typename T, int D>
__device__ __forceinline__ void store_summary(const PoolDev& a, int bg, int m, int lane, int count,
                                              const float (&acc)[PoolRowCfg<T, D>::NACC]) {
    typedef PoolRowCfg<T, D> C;
    T* sk = reinterpret_cast<T*>(a.sk) + ((int64_t)bg * a.Mp + m) * D;
    T* svt = reinterpret_cast<T*>(a.svt) + (((int64_t)bg * (a.Mp / 32) + m / 32) * D) * 32 + (m & 31);
    float sq = 0.f;
#pragma unroll
    for (int k = 0; k < C::NACC; ++k) {
        int c;
        bool is_v, writer;
        if constexpr (C::MF) {
            const int cc = 16 * k + lane;
            is_v = cc >= D;
            c = is_v ? cc - D : cc;
            writer = lane < 16;
        } else {
            c = 16 * k + 8 * ((lane >> 4) & 1) + 4 * ((lane >> 3) & 1) + 2 * ((lane >> 2) & 1) + ((lane >> 1) & 1);
            is_v = lane & 32;
            writer = !(lane & 1);
        }
        // count is wave-uniform: one fine block (pool_size 1) takes no division.
        const float mean = count == 1 ? acc[k] : (count ? acc[k] / (float)count : 0.f);
        if (writer && !is_v) {
            const T x = from_f32<T>(mean * a.key_scale);
            sk[c] = x;
            sq += to_f32(x) * to_f32(x);
        } else if (writer) {
            svt[c * 32] = from_f32<T>(mean);
        }
    }
    // Norm of the stored (rounded) summary key; non-negative floats order
    // like their bit patterns, so an integer max is an exact float max.
    const float norm = sqrtf(wave_sum(sq)) * (1.f + 1e-6f);
    if (lane == 0 && m < a.M)
        atomicMax(reinterpret_cast<int*>(a.sk_norm_max) + (int64_t)bg * kNormSlots + (m % kNormSlots),
                  __float_as_int(norm));
}

// Load the lane's pieces of the K and V rows of item i's step with slot
// tokens idx: lane l holds pieces l, l + 64, ... of the 64 x PPR grid of
// (slot, piece).  Empty slots read row 0; their slot weight is exactly 0, so
// they add 0 * row 0 to the sums, as the reference's masked product does
// (compression.py:38-39).
template <typename T, int D>
__device__ __forceinline__ void pool_fetch(const PoolDev& a, unsigned i, int idx, int lane,
                                           u32x4 (&pk)[PoolRowCfg<T, D>::PPR], u32x4 (&pv)[PoolRowCfg<T, D>::PPR]) {
    constexpr int PPR = PoolRowCfg<T, D>::PPR, EP = PoolRowCfg<T, D>::EP;
    const int g = (int)(i % a.G), b = (int)(i / a.G / a.Mp);
    const T* K = reinterpret_cast<const T*>(a.kg) + b * a.ksb + g * a.ksh;
    const T* Vv = reinterpret_cast<const T*>(a.vg) + b * a.vsb + g * a.vsh;
#pragma unroll
    for (int r = 0; r < PPR; ++r) {
        const int q = r * 64 + lane, s = q / PPR, p = q - s * PPR;
        const int64_t tok = max(__shfl(idx, s), 0);
        pk[r] = *reinterpret_cast<const u32x4*>(K + tok * a.ksn + p * EP);
        pv[r] = *reinterpret_cast<const u32x4*>(Vv + tok * a.vsn + p * EP);
    }
}

// MFMA B operand (16x16x32) for k-step ks and 16-channel tile t of [K | V]
// (2-byte types): lane L holds channel 16 t + L % 16 for slots
// 32 ks + 8 (L / 16) .. + 8, read from the row-major staged rows by two
// ds_read_b64_tr_b16.  Within a 16-lane block, lane B + 4a + e receives
// element e of the 8-byte windows addressed by lanes B + a + 4j (j = 0..3),
// so lane L addresses slot 32 ks + 8 (L / 16) + (L % 16) / 4 (four slots
// further for the second read) at channel 16 t + 4 (L % 4) of K or, past D,
// of V.  D is a multiple of 16, so no tile straddles K and V.
template <typename T, int D>
__device__ __forceinline__ typename Mma<T>::Frag pool_frag_tr(const unsigned char* rows, int ks, int t, int lane) {
    typedef PoolRowCfg<T, D> C;
    typedef short v4s __attribute__((ext_vector_type(4)));
    typedef short v8s __attribute__((ext_vector_type(8)));
    typedef __attribute__((address_space(3))) v4s* lds_v4s;
    const int slot = 32 * ks + 8 * (lane >> 4) + ((lane & 15) >> 2);
    const int ch = 16 * t + 4 * (lane & 3);
    const unsigned char* base = 16 * t < D ? rows + ch * 2 : rows + C::VOFF + (ch - D) * 2;
    const v4s lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4s)(base + slot * C::RB));
    const v4s hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4s)(base + (slot + 4) * C::RB));
    const v8s v = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
    return __builtin_bit_cast(typename Mma<T>::Frag, v);
}


// Persistent: wave w of block k takes items k * waves + w, + waves * grid, ...
// Items run kv head fastest, so the waves of a block read the neighbouring
// head slices of the same token rows together and each row's kg / vg span is
// fetched from HBM once.  A step is one fine block of an item (a padding
// summary has one step with no block); the block-table row of the step after
// next and the coordinates of the next step's tokens are loaded with the next
// step's rows.
template <typename T, int D, bool TAB_LDS>
__global__ __launch_bounds__((64 * PoolRowCfg<T, D>::MAX_WAVES)) void k_pool_fwd(PoolDev a) {
    typedef PoolRowCfg<T, D> C;
    constexpr int EP = C::EP, PPR = C::PPR, RB = C::RB, NCH = C::NCH, PPC = C::PPC;
    extern __shared__ __align__(16) unsigned char smem_raw[];
    const int waves = blockDim.x >> 6;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
    int4* meta = reinterpret_cast<int4*>(smem_raw);
    int* prun = reinterpret_cast<int*>(meta + D / 2);
    float* lweight = reinterpret_cast<float*>(prun + C::PFN);
    float* lbias = lweight + D;
    float2* ltab = reinterpret_cast<float2*>(lbias + 64);
    const int tab_dw = TAB_LDS ? ((a.table_entries * 2 + 3) & ~3) : 0;
    unsigned char* rows = reinterpret_cast<unsigned char*>(reinterpret_cast<uint32_t*>(ltab) + tab_dw) +
                          (size_t)wave * C::WAVE_BYTES;
    T* wrows = reinterpret_cast<T*>(rows + C::ROWS_BYTES);  // MFMA path: weight rows hi, lo
    for (int j = threadIdx.x; j < D / 2; j += blockDim.x) meta[j] = pair_meta(a.rope.pairs, j);
    // Piece p is a table run when its pairs read consecutive entries with one
    // stride vector: entry(j0 + t) = entry(j0) + t for every position.
    for (int p = threadIdx.x; p < PPR; p += blockDim.x) {
        const int j0 = p * EP / 2;
        const int4 m0 = pair_meta(a.rope.pairs, j0);
        int run = 1;
        for (int t = 1; t < EP / 2; ++t) {
            const int4 mt = pair_meta(a.rope.pairs, j0 + t);
            run &= mt.x == m0.x + t && mt.y == m0.y && mt.z == m0.z && mt.w == m0.w;
        }
        prun[p] = run;
    }
    for (int c = threadIdx.x; c < D; c += blockDim.x) lweight[c] = a.weight[c];
    for (int c = threadIdx.x; c < 64; c += blockDim.x) lbias[c] = c < a.V ? a.bias[c] : 0.f;
    const float2* tab = a.rope.table;
    if (TAB_LDS) {
        for (int e = threadIdx.x; e < a.table_entries; e += blockDim.x) ltab[e] = a.rope.table[e];
        tab = ltab;
    }
    __syncthreads();

    // Item indices fit in 32 bits (checked on the host), so the wave-uniform
    // item arithmetic is 32-bit scalar code.
    const unsigned total = (unsigned)a.B * a.G * a.Mp;
    const unsigned stride = gridDim.x * waves;
    const unsigned it0 = blockIdx.x * waves + wave;
    if (it0 >= total) return;

    // Waves walk the items from the last one down (item = total - 1 - i for
    // the i-th of the walk): the projections that write kg / vg just before
    // this kernel finish with the last tokens, and those rows are the likeliest
    // to still be in the last-level cache.
    auto item_of = [&](unsigned i) __attribute__((always_inline)) -> unsigned { return total - 1u - i; };
    auto steps_of = [&](unsigned i) __attribute__((always_inline)) -> int {
        const int m = (int)((item_of(i) / a.G) % a.Mp);
        return m < a.M ? (min(a.F, (m + 1) * a.P) - m * a.P + a.bps - 1) / a.bps : 1;
    };
    // The lane's slot token of step (i, fl), or -1 (empty slot, padding summary).
    const int lane_block = lane / (a.bps == 1 ? 64 : a.V), lane_slot = lane - lane_block * a.V;
    auto row_of = [&](unsigned i, int fl) __attribute__((always_inline)) -> int {
        const int m = (int)((item_of(i) / a.G) % a.Mp);
        const int f = m * a.P + fl * a.bps + lane_block;
        return (m < a.M && lane < a.bps * a.V && f < min(a.F, (m + 1) * a.P)) ? a.blocks[(int64_t)f * a.V + lane_slot]
                                                                              : -1;
    };
    // Pair metadata of each piece's first pair and the table-run flags, as
    // wave-uniform values (scalar registers) for the whole loop.
    int4 pm[PPR];
    unsigned runs = 0;
#pragma unroll
    for (int p = 0; p < PPR; ++p) {
        const int4 m0 = meta[p * EP / 2];
        pm[p] = int4{__builtin_amdgcn_readfirstlane(m0.x), __builtin_amdgcn_readfirstlane(m0.y),
                     __builtin_amdgcn_readfirstlane(m0.z), __builtin_amdgcn_readfirstlane(m0.w)};
        runs |= (unsigned)(__builtin_amdgcn_readfirstlane(prun[p]) != 0) << p;
    }
    if constexpr (C::MF) wrows[lane] = from_f32<T>(0.f);  // weight rows before the first step's sync

    // For 2-byte types the loop is compiled twice: once for tables whose
    // pieces are all runs (every (cos, sin) entry of a piece at e0 + t, no
    // per-pair metadata and no branch, so all the table reads of a step issue
    // together), once for the general pair order.
    auto pool_loop = [&](auto all_runs_tag) __attribute__((always_inline)) {
        constexpr bool ALL_RUNS = decltype(all_runs_tag)::value;
        u32x4 pk[PPR], pv[PPR];
        unsigned it = it0;
        int fl = 0, ns = steps_of(it);
        int idx = row_of(it, 0);
        int pos[3];
        rope_position32(a.rope, max(idx, 0), pos);
        pool_fetch<T, D>(a, item_of(it), idx, lane, pk, pv);
        unsigned it1 = ns > 1 ? it : it + stride;
        int fl1 = ns > 1 ? 1 : 0;
        int idx1 = it1 < total ? row_of(it1, fl1) : -1;
        float acc[C::NACC];
#pragma unroll
        for (int k = 0; k < C::NACC; ++k) acc[k] = 0.f;
        int count = 0;
        // The summary of a finished item is stored in the next step, after that
        // step's rows are staged and before the loads of the step after it are
        // issued, so the wait for those loads never waits on the stores.
        bool pending = false;
        int pend_bg = 0, pend_m = 0, pend_count = 0;
        float pend[C::NACC];
        for (;;) {
            // Stage this step's pieces as rows (slot s at s * RB).
#pragma unroll
            for (int r = 0; r < PPR; ++r) {
                const int q = r * 64 + lane;
                *reinterpret_cast<u32x4*>(rows + q * 16) = pk[r];
                *reinterpret_cast<u32x4*>(rows + C::VOFF + q * 16) = pv[r];
            }
            wave_lds_sync();
            if (pending) {
                store_summary<T, D>(a, pend_bg, pend_m, lane, pend_count, pend);
                pending = false;
            }
            // The lane's own K row (and V row for the fp32 butterfly).
            u32x4 kr[PPR], vr[PPR];
#pragma unroll
            for (int p = 0; p < PPR; ++p) {
                kr[p] = *reinterpret_cast<const u32x4*>(rows + lane * RB + p * 16);
                if constexpr (!C::MF) vr[p] = *reinterpret_cast<const u32x4*>(rows + C::VOFF + lane * RB + p * 16);
            }
            // Next step's coordinates, the block-table row after it, then the
            // next step's rows.  The load counter completes in issue order, and
            // the coordinates and table row are carried into the next iteration
            // (a register copy that must wait for them): issued before the rows,
            // that wait leaves the row loads in flight under this step's
            // arithmetic instead of draining them at the end of the step.
            const bool more = it1 < total;
            int ns1 = 1, pos1[3] = {0, 0, 0}, idx2 = -1;
            unsigned it2 = total;
            int fl2 = 0;
            if (more) {
                ns1 = steps_of(it1);
                rope_position32(a.rope, max(idx1, 0), pos1);
                it2 = fl1 + 1 < ns1 ? it1 : it1 + stride;
                fl2 = fl1 + 1 < ns1 ? fl1 + 1 : 0;
                if (it2 < total) idx2 = row_of(it2, fl2);
                pool_fetch<T, D>(a, item_of(it1), idx1, lane, pk, pv);
            }

            const uint64_t filled = __ballot(idx >= 0);
            if (filled != 0) {  // empty fine blocks: no mass, no count
                count += blocks_filled(filled, a.bps, a.V);
                // Rotate the slot's key, round it to the storage type, and form
                // its logit (compression.py:31-35): (k . w) / tau + bias_s.
                // 2-byte types read every (cos, sin) entry of the step first (one
                // batch of LDS reads); fp32 rows, twice as many pieces, read them
                // piece by piece.
                float2 cs[C::MF ? PPR : 1][EP / 2];
                auto table_piece = [&](int p, float2(&c)[EP / 2]) __attribute__((always_inline)) {
                    const int e0 = pm[p].x + mul_u24(pm[p].y, pos[0]) + mul_u24(pm[p].z, pos[1]) +
                                   mul_u24(pm[p].w, pos[2]);
                    if (ALL_RUNS || (runs >> p & 1)) {
#pragma unroll
                        for (int t = 0; t < EP / 2; ++t) c[t] = tab[e0 + t];
                    } else {
#pragma unroll
                        for (int t = 0; t < EP / 2; ++t) c[t] = pair_cs(meta[p * EP / 2 + t], tab, pos);
                    }
                };
                if constexpr (C::MF) {
#pragma unroll
                    for (int p = 0; p < PPR; ++p) table_piece(p, cs[p]);
                }
                float dot = 0.f;
#pragma unroll
                for (int p = 0; p < PPR; ++p) {
                    float2(&c)[EP / 2] = cs[C::MF ? p : 0];
                    if constexpr (!C::MF) table_piece(p, c);
                    float kx[EP];
                    unpack_piece<T, EP>(kr[p], kx);
#pragma unroll
                    for (int t = 0; t < EP / 2; ++t) rotate_pair(kx[2 * t], kx[2 * t + 1], c[t].x, c[t].y);
                    kr[p] = __builtin_bit_cast(u32x4, round_piece<T, EP>(kx));
#pragma unroll
                    for (int e = 0; e < EP; ++e) dot += kx[e] * lweight[p * EP + e];
                }
                const float logit = idx >= 0 ? dot * a.inv_tau + lbias[lane & (a.gsz - 1)] : -INFINITY;
                const float mx = group_max(logit, a.gsz);
                const float ex = idx >= 0 ? expf(logit - mx) : 0.f;
                const float den = group_sum(ex, a.gsz);
                const float wgt = den > 0.f ? ex / den : 0.f;  // a block of the step with no slot: 0
                if constexpr (C::MF) {
                    typedef typename Mma<T>::Frag Frag;
                    // The rotated, rounded key over the lane's own staged row (only
                    // this lane has read it).
#pragma unroll
                    for (int p = 0; p < PPR; ++p) *reinterpret_cast<u32x4*>(rows + lane * RB + p * 16) = kr[p];
                    const T hi = from_f32<T>(wgt);
                    wrows[lane] = hi;
                    wrows[64 + lane] = from_f32<T>(wgt - to_f32(hi));
                    wave_lds_sync();
                    // D[w][c] = sum_s W[w][s] X[s][c] for the weight rows w = 0
                    // (hi), 1 (lo), over 32 slots per instruction: lane l holds
                    // slots 8 (l / 16) + j of channel l % 16 (B) and, for
                    // l % 16 < 2, of weight row l % 16 (A); rows 0 and 1 of D
                    // are registers 0 and 1 of lanes 0..15.
                    const int wr = lane & 15;
                    Frag wa[2];
#pragma unroll
                    for (int ks = 0; ks < 2; ++ks) {
                        const u32x4 w = *reinterpret_cast<const u32x4*>(wrows + 64 * (wr & 1) + 32 * ks + 8 * (lane >> 4));
                        wa[ks] = __builtin_bit_cast(Frag, wr < 2 ? w : u32x4{0u, 0u, 0u, 0u});
                    }
                    Frag xb[2][C::NT];
#pragma unroll
                    for (int ks = 0; ks < 2; ++ks)
#pragma unroll
                        for (int t = 0; t < C::NT; ++t) xb[ks][t] = pool_frag_tr<T, D>(rows, ks, t, lane);
#pragma unroll
                    for (int t = 0; t < C::NT; ++t) {
                        f32x4 d = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
                        for (int ks = 0; ks < 2; ++ks) d = Mma<T>::mfma16(wa[ks], xb[ks][t], d);
                        acc[t] += d[0] + d[1];
                    }
                } else {
#pragma unroll
                    for (int k = 0; k < NCH; ++k) {
                        float kv[16], vv[16];
#pragma unroll
                        for (int t = 0; t < PPC; ++t) {
                            float xk[EP], xv[EP];
                            unpack_piece<T, EP>(kr[k * PPC + t], xk);
                            unpack_piece<T, EP>(vr[k * PPC + t], xv);
#pragma unroll
                            for (int e = 0; e < EP; ++e) {
                                kv[t * EP + e] = wgt * xk[e];
                                vv[t * EP + e] = wgt * xv[e];
                            }
                        }
                        acc[k] += butterfly_sum(kv, vv, lane);
                    }
                }
            }
            if (fl + 1 == ns) {
                const unsigned bm = item_of(it) / a.G;
                pending = true;
                pend_bg = (int)(bm / a.Mp) * a.G + (int)(item_of(it) % a.G);
                pend_m = (int)(bm % a.Mp);
                pend_count = count;
#pragma unroll
                for (int k = 0; k < C::NACC; ++k) {
                    pend[k] = acc[k];
                    acc[k] = 0.f;
                }
                count = 0;
            }
            if (!more) break;
            wave_lds_sync();  // the next step's staging overwrites the rows
            it = it1, fl = fl1, ns = ns1, idx = idx1;
            pos[0] = pos1[0], pos[1] = pos1[1], pos[2] = pos1[2];
            it1 = it2, fl1 = fl2, idx1 = idx2;
        }
        if (pending) store_summary<T, D>(a, pend_bg, pend_m, lane, pend_count, pend);
    };
    if constexpr (C::MF) {
        if (runs == (1u << PPR) - 1u) {
            pool_loop(std::true_type{});
            return;
        }
    }
    pool_loop(std::false_type{});
}

// Pooling backward (the VJP of compression.py:28-44; kernels.py:240-270 of
// amilworks/Pack3D): for summary m with fine blocks f and c non-empty blocks,
// g_k = dsk_m / c and g_v = dsv_m / c (dsk, dsv summed over the query splits
// of the global pass), and per slot s of block f, with a the slot softmax:
//   da_s = g_k . k_s + g_v . v_s,   dl_s = a_s (da_s - sum_s' a_s' da_s'),
//   dk_s = a_s g_k + dl_s w / tau,  dv_s = a_s g_v,
//   dw += sum_s dl_s k_s / tau,      db_s += dl_s.
// k_s is the rotated key rounded to the storage type, as in the forward; dk_s
// is rounded to the storage type, rotated back (R^T) and rounded again, which
// is the gradient of the unrotated key.  Fine blocks partition the tokens, so
// every row of dkg / dvg is written exactly once.
struct PoolBwdDev {
    const float *dsk_part, *dsv_part;
    int splits;
    p3d_view dkg, dvg;  // [B, G, N, D] views, storage type, 16-byte aligned rows
    float *dw_part;    // [B * G * Mp, D]
    float *db_part;    // [B * G * Mp, V]
};

template <typename T, int D, bool TAB_LDS>
__global__ __launch_bounds__(256) void k_pool_bwd(PoolDev a, PoolBwdDev bd) {
    typedef PoolCfg<T, D> C;
    constexpr int EP = C::EP, PPR = C::PPR, CPD = C::CPD;
    constexpr int WAVE_DW = 2 * 64 * C::RD + 2 * D + 64;  // K rows, V rows, g_k, g_v, slot weights
    extern __shared__ __align__(16) unsigned char smem_raw[];
    const int waves = blockDim.x >> 6;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
    int4* meta = reinterpret_cast<int4*>(smem_raw);
    float* lweight = reinterpret_cast<float*>(meta + D / 2);
    float* lbias = lweight + D;
    float2* ltab = reinterpret_cast<float2*>(lbias + 64);
    const int tab_dw = TAB_LDS ? ((a.table_entries * 2 + 3) & ~3) : 0;
    uint32_t* krows = reinterpret_cast<uint32_t*>(ltab) + tab_dw + wave * WAVE_DW;
    uint32_t* vrows = krows + 64 * C::RD;
    float* gk = reinterpret_cast<float*>(vrows + 64 * C::RD);
    float* gv = gk + D;
    float* lw = gv + D;
    for (int j = threadIdx.x; j < D / 2; j += blockDim.x)
        meta[j] = pair_meta(a.rope.pairs, j);
    for (int c = threadIdx.x; c < D; c += blockDim.x) lweight[c] = a.weight[c];
    for (int c = threadIdx.x; c < 64; c += blockDim.x) lbias[c] = c < a.V ? a.bias[c] : 0.f;
    const float2* tab = a.rope.table;
    if (TAB_LDS) {
        for (int e = threadIdx.x; e < a.table_entries; e += blockDim.x) ltab[e] = a.rope.table[e];
        tab = ltab;
    }
    __syncthreads();

    const unsigned total = (unsigned)a.B * a.G * a.Mp;
    const unsigned stride = gridDim.x * waves;
    const int64_t slice = (int64_t)total * D;  // one split of the partials
    // Fine blocks packed into a 64-lane step as in the forward: lane l holds
    // slot l % V of block l / V of the step (bps = 64 / V blocks), or slot l.
    const int lane_block = lane / (a.bps == 1 ? 64 : a.V), lane_slot = lane - lane_block * a.V;
    auto slot_token = [&](int fs, int f_end) __attribute__((always_inline)) -> int {
        const int f = fs + lane_block;
        return (lane < a.bps * a.V && f < f_end) ? a.blocks[(int64_t)f * a.V + lane_slot] : -1;
    };
    for (unsigned item = blockIdx.x * waves + wave; item < total; item += stride) {
        const int g = (int)(item % a.G);
        const unsigned bm = item / a.G;
        const int m = (int)(bm % a.Mp), b = (int)(bm / a.Mp);
        const int64_t bg = (int64_t)b * a.G + g;
        const int f0 = m * a.P, f_end = m < a.M ? min(a.F, (m + 1) * a.P) : 0;
        int count = 0;
        for (int fs = f0; fs < f_end; fs += a.bps) {
            const uint64_t filled = __ballot(slot_token(fs, f_end) >= 0);
            if (filled) count += blocks_filled(filled, a.bps, a.V);
        }
        float dwacc[C::SJ][CPD];
#pragma unroll
        for (int j = 0; j < C::SJ; ++j)
#pragma unroll
            for (int c = 0; c < CPD; ++c) dwacc[j][c] = 0.f;
        float dbacc = 0.f;
        if (count > 0) {
            const float inv = 1.f / (float)count;
            for (int c = lane; c < D; c += 64) {
                // The split partials in groups of 8 loads issued together, then
                // added in split order (the same sums as one at a time, without
                // a memory round trip per split).
                const float* pk = bd.dsk_part + (bg * a.Mp + m) * D + c;
                const float* pv = bd.dsv_part + (bg * a.Mp + m) * D + c;
                float sk = 0.f, sv = 0.f;
                int sp = 0;
                for (; sp + 8 <= bd.splits; sp += 8) {
                    float k8[8], v8[8];
#pragma unroll
                    for (int i = 0; i < 8; ++i) {
                        k8[i] = pk[(sp + i) * slice];
                        v8[i] = pv[(sp + i) * slice];
                    }
#pragma unroll
                    for (int i = 0; i < 8; ++i) {
                        sk += k8[i];
                        sv += v8[i];
                    }
                }
                for (; sp < bd.splits; ++sp) {
                    sk += pk[sp * slice];
                    sv += pv[sp * slice];
                }
                gk[c] = sk * inv;
                gv[c] = sv * inv;
            }
        }
        const T* K = reinterpret_cast<const T*>(a.kg) + b * a.ksb + g * a.ksh;
        const T* Vv = reinterpret_cast<const T*>(a.vg) + b * a.vsb + g * a.vsh;
        T* DK = reinterpret_cast<T*>(bd.dkg.data) + b * bd.dkg.sb + g * bd.dkg.sh;
        T* DV = reinterpret_cast<T*>(bd.dvg.data) + b * bd.dvg.sb + g * bd.dvg.sh;
        for (int fs = f0; fs < f_end; fs += a.bps) {
            const int idx = slot_token(fs, f_end);
            if (__ballot(idx >= 0) == 0) continue;
            int pos[3];
            rope_position32(a.rope, max(idx, 0), pos);
            uint4 kr[PPR], vr[PPR];
            int tok[PPR];
#pragma unroll
            for (int i = 0; i < PPR; ++i) tok[i] = __shfl(idx, (i * 64 + lane) / PPR);
#pragma unroll
            for (int i = 0; i < PPR; ++i) {
                const int q = i * 64 + lane, p = q - (q / PPR) * PPR;
                const int t = max(tok[i], 0);
                kr[i] = *reinterpret_cast<const uint4*>(K + (int64_t)t * a.ksn + p * EP);
                vr[i] = *reinterpret_cast<const uint4*>(Vv + (int64_t)t * a.vsn + p * EP);
            }
#pragma unroll
            for (int i = 0; i < PPR; ++i)
                if (tok[i] < 0) kr[i] = vr[i] = uint4{0u, 0u, 0u, 0u};
            stage_rows<C>(krows, kr, lane);
            stage_rows<C>(vrows, vr, lane);
            wave_lds_sync();
            // Lane = slot: rotate and round the K row, its logit, and da_s.
            float logit = -INFINITY, da = 0.f;
            if (idx >= 0) {
                float dot = 0.f;
#pragma unroll 1
                for (int p = 0; p < PPR; ++p) {
                    uint4 raw = *reinterpret_cast<const uint4*>(krows + lane * C::RD + p * 4);
                    const uint4 vraw = *reinterpret_cast<const uint4*>(vrows + lane * C::RD + p * 4);
                    T* kt = reinterpret_cast<T*>(&raw);
                    const T* vt = reinterpret_cast<const T*>(&vraw);
                    float kx[EP];
#pragma unroll
                    for (int e = 0; e < EP; ++e) kx[e] = to_f32(kt[e]);
                    rotate_piece<EP>(meta, tab, pos, p * EP, kx);
#pragma unroll
                    for (int e = 0; e < EP; ++e) {
                        kt[e] = from_f32<T>(kx[e]);
                        const float k = to_f32(kt[e]);
                        dot += k * lweight[p * EP + e];
                        da += gk[p * EP + e] * k + gv[p * EP + e] * to_f32(vt[e]);
                    }
                    *reinterpret_cast<uint4*>(krows + lane * C::RD + p * 4) = raw;
                }
                logit = dot * a.inv_tau + lbias[lane & (a.gsz - 1)];
            }
            // Softmax and sum_s a_s da_s over each block's lanes.
            const float mx = group_max(logit, a.gsz);
            const float ex = idx >= 0 ? expf(logit - mx) : 0.f;
            const float den = group_sum(ex, a.gsz);
            const float w = den > 0.f ? ex / den : 0.f;
            const float sa = group_sum(w * da, a.gsz);
            const float dl = w * (da - sa);
            dbacc += dl;
            lw[lane] = dl * a.inv_tau;
            // dk_s, dv_s of this lane's slot, rotated back and stored.
            if (idx >= 0) {
#pragma unroll 1
                for (int p = 0; p < PPR; ++p) {
                    float dk[EP], dv[EP];
#pragma unroll
                    for (int e = 0; e < EP; ++e) {
                        const int c = p * EP + e;
                        dk[e] = to_f32(from_f32<T>(w * gk[c] + dl * lweight[c] * a.inv_tau));
                        dv[e] = w * gv[c];
                    }
                    rotate_piece_inverse<EP>(meta, tab, pos, p * EP, dk);
                    uint4 ko, vo;
                    T* kt = reinterpret_cast<T*>(&ko);
                    T* vt = reinterpret_cast<T*>(&vo);
#pragma unroll
                    for (int e = 0; e < EP; ++e) {
                        kt[e] = from_f32<T>(dk[e]);
                        vt[e] = from_f32<T>(dv[e]);
                    }
                    *reinterpret_cast<uint4*>(DK + (int64_t)idx * bd.dkg.sn + p * EP) = ko;
                    *reinterpret_cast<uint4*>(DV + (int64_t)idx * bd.dvg.sn + p * EP) = vo;
                }
            }
            wave_lds_sync();  // rotated rows and dl / tau are read across lanes below
            column_sums_w<C, T>(krows, lw, lane, dwacc);
            wave_lds_sync();  // the next fine block overwrites the rows
        }
        // Partials of this item: dw (column dwords of group 0) and db (one per slot).
        float* dwp = bd.dw_part + (int64_t)item * D;
#pragma unroll
        for (int j = 0; j < C::SJ; ++j) {
            const int u = lane + 64 * j;
            if (lane < C::LW && u < C::DW)
#pragma unroll
                for (int c = 0; c < CPD; ++c) dwp[u * CPD + c] = dwacc[j][c];
        }
        // Slot s's bias gradient sums the lanes holding slot s of any block.
        for (int o = a.gsz; o < 64; o <<= 1) dbacc += __shfl_xor(dbacc, o);
        if (lane < a.V) bd.db_part[(int64_t)item * a.V + lane] = dbacc;
    }
}

__global__ void k_zero_f32(float* p, int n) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) p[i] = 0.f;
}

struct RotDev {
    int B, H, N, D, inverse;
    const char* x;
    int64_t xsb, xsh, xsn;
    char* y;
    int64_t ysb, ysh, ysn;
    RopeDev rope;
};

// One 16-byte piece per thread.  Grid y walks the (batch, head) planes from
// plane0, grid x the pieces of a plane's rows (tokens * pieces per row below
// 2^31, checked on the host); the pair descriptors come from LDS.
template <typename T, int D>
__global__ __launch_bounds__(256) void k_rotate(RotDev a, int plane0) {
    constexpr int EP = Piece<T>::N;
    constexpr int PPR = D / EP;
    __shared__ int4 meta[D / 2];
    for (int j = threadIdx.x; j < D / 2; j += blockDim.x) meta[j] = pair_meta(a.rope.pairs, j);
    __syncthreads();
    const int p = plane0 + (int)blockIdx.y;
    const int idx = (int)blockIdx.x * 256 + (int)threadIdx.x;
    if (idx >= a.N * PPR) return;
    const int n = idx / PPR, piece = idx - n * PPR;
    const int b = p / a.H, h = p - b * a.H;
    float x[EP];
    load_piece<T>(reinterpret_cast<const T*>(a.x) + b * a.xsb + h * a.xsh + (int64_t)n * a.xsn + piece * EP, x);
    int pos[3];
    rope_position32(a.rope, n, pos);
    const float sgn = a.inverse ? -1.f : 1.f;
#pragma unroll
    for (int e = 0; e < EP; e += 2) {
        const int4 m = meta[(piece * EP + e) >> 1];
        const float2 cs = a.rope.table[m.x + m.y * pos[0] + m.z * pos[1] + m.w * pos[2]];
        rotate_pair(x[e], x[e + 1], cs.x, sgn * cs.y);
    }
    uint4 raw;
    T* v = reinterpret_cast<T*>(&raw);
#pragma unroll
    for (int e = 0; e < EP; ++e) v[e] = from_f32<T>(x[e]);
    *reinterpret_cast<uint4*>(reinterpret_cast<T*>(a.y) + b * a.ysb + h * a.ysh + (int64_t)n * a.ysn + piece * EP) =
        raw;
}

template <typename T, int D>
void launch_rotate(const RotDev& d, hipStream_t s) {
    constexpr int PPR = D / Piece<T>::N;
    const unsigned bx = (unsigned)cdiv((int64_t)d.N * PPR, 256);
    const int planes = d.B * d.H;
    for (int p0 = 0; p0 < planes; p0 += 65535) {
        const unsigned by = (unsigned)(planes - p0 < 65535 ? planes - p0 : 65535);
        k_rotate<T, D><<<dim3(bx, by), 256, 0, s>>>(d, p0);
    }
}

template <typename T>
void dispatch_rotate(const RotDev& d, hipStream_t s) {
    switch (d.D) {
        case 16: launch_rotate<T, 16>(d, s); break;
        case 32: launch_rotate<T, 32>(d, s); break;
        case 48: launch_rotate<T, 48>(d, s); break;
        case 64: launch_rotate<T, 64>(d, s); break;
        default: launch_rotate<T, 128>(d, s); break;
    }
}

// Rope tables up to this size are staged in LDS by every pool block.
constexpr int kTableLdsBytes = 32768;

// Waves per pool block: four (the four kv heads of a summary run together)
// when the block's LDS fits in the 160 KiB of a CU, else two, else one.
inline int pool_waves(size_t fixed, size_t per_wave) {
    for (int w = 4; w > 1; w >>= 1)
        if (fixed + per_wave * w <= 160 * 1024) return w;
    return 1;
}

template <typename T, int D>
void launch_pool_t(const PoolDev& d, hipStream_t s) {
    // As many waves per block as the LDS holds row buffers for (at most 12);
    // a persistent grid of as many blocks as stay resident, each striding
    // over the items.
    typedef PoolRowCfg<T, D> C;
    const bool tab_lds = d.table_entries * 8 <= kTableLdsBytes;
    const size_t tab_bytes = tab_lds ? (size_t)((d.table_entries * 2 + 3) & ~3) * 4 : 0;
    const size_t fixed = C::FIXED + tab_bytes;
    int dev = 0, cus = 0, per_cu = 0;
    (void)hipGetDevice(&dev);
    (void)hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
    const int64_t items = (int64_t)d.B * d.G * d.Mp;
    int waves = (int)std::min<size_t>(C::MAX_WAVES, (160 * 1024 - fixed) / C::WAVE_BYTES);
    // Few items (long summaries: pool_size 16 gives 16 fine blocks each):
    // fewer waves per block, so that the blocks reach every compute unit.
    while (waves > 1 && cdiv(items, waves) < cus) waves >>= 1;
    const size_t smem = fixed + (size_t)C::WAVE_BYTES * waves;
    if (tab_lds)
        (void)hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, k_pool_fwd<T, D, true>, 64 * waves, smem);
    else
        (void)hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, k_pool_fwd<T, D, false>, 64 * waves, smem);
    const int64_t resident = (int64_t)std::max(1, cus) * std::max(1, per_cu);
    const int64_t needed = cdiv(items, waves);
    // Equal shares: the fewest rounds that cover every item, spread evenly.
    const int64_t rounds = cdiv(needed, resident);
    const unsigned blocks = (unsigned)cdiv(needed, rounds);
    if (tab_lds)
        k_pool_fwd<T, D, true><<<blocks, 64 * waves, smem, s>>>(d);
    else
        k_pool_fwd<T, D, false><<<blocks, 64 * waves, smem, s>>>(d);
}

template <int D>
void launch_pool(const PoolDev& d, int dtype, hipStream_t s) {
    switch (dtype) {
        case P3D_F32: launch_pool_t<float, D>(d, s); break;
        case P3D_F16: launch_pool_t<_Float16, D>(d, s); break;
        default: launch_pool_t<__bf16, D>(d, s); break;
    }
}

}  // namespace
}  // namespace p3d

using namespace p3d;

namespace p3d {
namespace {

// Argument checks and device view shared by the pooling forward and backward.
int fill_pool(const p3d_pool_args* args, PoolDev& d) {
    P3D_REQUIRE(args, "null args");
    const p3d_pool_args& a = *args;
    const int es = dtype_size(a.dtype);
    P3D_REQUIRE(a.dtype >= P3D_F32 && a.dtype <= P3D_BF16, "unknown dtype");
    P3D_REQUIRE(a.head_dim == 16 || a.head_dim == 32 || a.head_dim == 48 || a.head_dim == 64 || a.head_dim == 128,
                "head_dim must be 16, 32, 48, 64 or 128");
    P3D_REQUIRE(a.batch >= 1 && a.kv_heads >= 1 && a.tokens >= 1 && a.fine_blocks >= 1, "empty pooling problem");
    P3D_REQUIRE(a.slots >= 1 && a.slots <= 64 && a.pool_size >= 1 && a.pool_size <= 32, "bad pooling shape");
    P3D_REQUIRE(a.summaries == (a.fine_blocks + a.pool_size - 1) / a.pool_size, "summaries != ceil(F/P)");
    P3D_REQUIRE(view_ok(a.kg, es) && view_ok(a.vg, es), "kg/vg rows must be 16-byte aligned");
    P3D_REQUIRE(a.sk && a.svt && a.sk_norm_max && a.blocks && a.weight && a.bias && a.rope.table && a.rope.pairs,
                "null pointer argument");
    P3D_REQUIRE(a.rope.packed || a.rope.coords, "rope needs coords unless packed");
    P3D_REQUIRE(a.rope.table_entries >= 1 && a.rope.table_entries < (1 << 23),
                "rope table_entries must be in [1, 2^23)");
    P3D_REQUIRE(a.temperature > 0.f, "temperature must be positive");
    P3D_REQUIRE(a.key_scale > 0.f, "key_scale must be positive");
    d = PoolDev{};
    d.B = a.batch;
    d.G = a.kv_heads;
    d.N = a.tokens;
    d.F = a.fine_blocks;
    d.V = a.slots;
    d.P = a.pool_size;
    d.bps = (a.slots <= 32 && (a.slots & (a.slots - 1)) == 0) ? 64 / a.slots : 1;
    d.gsz = d.bps == 1 ? 64 : a.slots;
    d.M = a.summaries;
    d.Mp = (int)cdiv(a.summaries, 32) * 32;
    P3D_REQUIRE((int64_t)a.batch * a.kv_heads * d.Mp < ((int64_t)1 << 31), "batch * kv_heads * summaries too large");
    d.inv_tau = 1.f / a.temperature;
    d.key_scale = a.key_scale;
    d.kg = (const char*)a.kg.data;
    d.vg = (const char*)a.vg.data;
    d.ksb = a.kg.sb, d.ksh = a.kg.sh, d.ksn = a.kg.sn;
    d.vsb = a.vg.sb, d.vsh = a.vg.sh, d.vsn = a.vg.sn;
    d.blocks = a.blocks;
    d.weight = a.weight;
    d.bias = a.bias;
    d.rope = rope_dev(a.rope);
    d.table_entries = a.rope.table_entries;
    d.sk = a.sk;
    d.svt = a.svt;
    d.sk_norm_max = a.sk_norm_max;
    return P3D_OK;
}

template <typename T, int D>
void launch_pool_bwd_t(const PoolDev& d, const PoolBwdDev& bd, int64_t items, hipStream_t s) {
    const bool tab_lds = d.table_entries * 8 <= kTableLdsBytes;
    const size_t tab_bytes = tab_lds ? (size_t)((d.table_entries * 2 + 3) & ~3) * 4 : 0;
    const size_t fixed = (size_t)(D / 2) * 16 + (size_t)D * 4 + 64 * 4;
    const size_t per_wave = (size_t)(2 * 64 * PoolCfg<T, D>::RD + 2 * D + 64) * 4;
    int dev = 0, cus = 0, per_cu = 0;
    (void)hipGetDevice(&dev);
    (void)hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
    int waves = pool_waves(fixed + tab_bytes, per_wave);
    while (waves > 1 && cdiv(items, waves) < cus) waves >>= 1;  // as in the forward
    const size_t smem = fixed + tab_bytes + per_wave * waves;
    if (tab_lds)
        (void)hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, k_pool_bwd<T, D, true>, 64 * waves, smem);
    else
        (void)hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, k_pool_bwd<T, D, false>, 64 * waves, smem);
    const int64_t resident = (int64_t)std::max(1, cus) * std::max(1, per_cu);
    const int64_t needed = cdiv(items, waves);
    const int64_t rounds = cdiv(needed, resident);
    const unsigned blocks = (unsigned)cdiv(needed, rounds);
    if (tab_lds)
        k_pool_bwd<T, D, true><<<blocks, 64 * waves, smem, s>>>(d, bd);
    else
        k_pool_bwd<T, D, false><<<blocks, 64 * waves, smem, s>>>(d, bd);
}

template <int D>
void launch_pool_bwd(const PoolDev& d, const PoolBwdDev& bd, int dtype, int64_t items, hipStream_t s) {
    switch (dtype) {
        case P3D_F32: launch_pool_bwd_t<float, D>(d, bd, items, s); break;
        case P3D_F16: launch_pool_bwd_t<_Float16, D>(d, bd, items, s); break;
        default: launch_pool_bwd_t<__bf16, D>(d, bd, items, s); break;
    }
}

}  // namespace
}  // namespace p3d

extern "C" int p3d_pool_fwd(const p3d_pool_args* args, void* stream) {
    PoolDev d;
    if (int rc = fill_pool(args, d)) return rc;
    const p3d_pool_args& a = *args;
    hipStream_t s = as_stream(stream);
    const int bgn = a.batch * a.kv_heads * kNormSlots;
    if (!a.norms_cleared) k_zero_f32<<<(unsigned)cdiv(bgn, 256), 256, 0, s>>>(a.sk_norm_max, bgn);
    switch (a.head_dim) {
        case 16: launch_pool<16>(d, a.dtype, s); break;
        case 32: launch_pool<32>(d, a.dtype, s); break;
        case 48: launch_pool<48>(d, a.dtype, s); break;
        case 64: launch_pool<64>(d, a.dtype, s); break;
        default: launch_pool<128>(d, a.dtype, s); break;
    }
    return check_launch("p3d_pool_fwd");
}

extern "C" int p3d_rotate(p3d_view x, p3d_view y, int32_t batch, int32_t heads, int32_t tokens,
                          int32_t head_dim, int32_t dtype, const p3d_rope* rope, int32_t inverse, void* stream) {
    P3D_REQUIRE(rope && rope->table && rope->pairs && (rope->packed || rope->coords), "bad rope");
    const int es = dtype_size(dtype);
    P3D_REQUIRE(dtype >= P3D_F32 && dtype <= P3D_BF16, "unknown dtype");
    P3D_REQUIRE(head_dim == 16 || head_dim == 32 || head_dim == 48 || head_dim == 64 || head_dim == 128,
                "head_dim must be 16, 32, 48, 64 or 128");
    P3D_REQUIRE(batch >= 1 && heads >= 1 && tokens >= 1, "empty rotation problem");
    P3D_REQUIRE((int64_t)tokens * (head_dim / (16 / es)) < ((int64_t)1 << 31),
                "tokens * pieces per row must be below 2^31");
    P3D_REQUIRE(view_ok(x, es) && view_ok(y, es), "rows must be 16-byte aligned");
    RotDev d{};
    d.B = batch, d.H = heads, d.N = tokens, d.D = head_dim, d.inverse = inverse;
    d.x = (const char*)x.data, d.xsb = x.sb, d.xsh = x.sh, d.xsn = x.sn;
    d.y = (char*)y.data, d.ysb = y.sb, d.ysh = y.sh, d.ysn = y.sn;
    d.rope = rope_dev(*rope);
    hipStream_t s = as_stream(stream);
    switch (dtype) {
        case P3D_F32: dispatch_rotate<float>(d, s); break;
        case P3D_F16: dispatch_rotate<_Float16>(d, s); break;
        default: dispatch_rotate<__bf16>(d, s); break;
    }
    return check_launch("p3d_rotate");
}

extern "C" int p3d_pool_bwd(const p3d_pool_args* args, const float* dsk_part, const float* dsv_part,
                            int32_t splits, p3d_view dkg, p3d_view dvg, float* dw_part, float* db_part,
                            void* stream) {
    PoolDev d;
    if (int rc = fill_pool(args, d)) return rc;
    P3D_REQUIRE(dsk_part && dsv_part && dw_part && db_part, "null pointer argument");
    P3D_REQUIRE(view_ok(dkg, dtype_size(args->dtype)) && view_ok(dvg, dtype_size(args->dtype)),
                "dkg / dvg rows must be 16-byte aligned");
    P3D_REQUIRE(splits >= 1, "splits must be positive");
    PoolBwdDev bd{dsk_part, dsv_part, splits, dkg, dvg, dw_part, db_part};
    const int64_t items = (int64_t)d.B * d.G * d.Mp;
    hipStream_t s = as_stream(stream);
    switch (args->head_dim) {
        case 16: launch_pool_bwd<16>(d, bd, args->dtype, items, s); break;
        case 32: launch_pool_bwd<32>(d, bd, args->dtype, items, s); break;
        case 48: launch_pool_bwd<48>(d, bd, args->dtype, items, s); break;
        case 64: launch_pool_bwd<64>(d, bd, args->dtype, items, s); break;
        default: launch_pool_bwd<128>(d, bd, args->dtype, items, s); break;
    }
    return check_launch("p3d_pool_bwd");
}
