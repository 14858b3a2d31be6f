// Shared machinery of the attention kernels.
//
// A wave owns 2 "column blocks" of 32 queries each.  For a tile of 32 keys
// it computes the transposed score tile S^T = K Q^T on 32x32 MFMAs (lane l
// then holds 16 scores of query l % 32), runs the online-softmax update in
// the log2 domain, and feeds the probabilities straight back as the B
// operand of O^T = V^T P^T, so P never leaves the registers.  Because every
// lane holds one query, the running max, the rescale and the normaliser are
// per-lane scalars.  When head_dim is not a multiple of 32 the padding rows
// of O^T include a row of ones, which makes the MFMA produce the softmax
// denominator as well.
#pragma once

#include "rope.hpp"

namespace p3d {

template <typename T, int D_>
struct Cfg {
    typedef T T_;
    typedef Mma<T> M;
    typedef typename M::Frag Frag;
    static constexpr int D = D_;
    static constexpr int E = M::E;
    static constexpr int KS = M::KS;
    static constexpr int NT = D / KS;                 // MFMAs per score tile
    static constexpr bool ONES = (D % 32) != 0;       // denominator row in the O^T padding
    static constexpr int MB = (D + (ONES ? 1 : 0) + 31) / 32;  // 32-row blocks of O^T
    static constexpr int KSTEPS = 32 / KS;            // PV MFMAs per tile and block
    static constexpr int ONES_MB = D / 32;
    static constexpr int ONES_G = ((D % 32) / 4) & 1;
    static constexpr int ONES_R = 4 * ((D % 32) / 8) + (D % 4);
    static constexpr int KSTR = D + 16 / (int)sizeof(T);  // LDS key-row stride (elements)
    static_assert(D % KS == 0, "head_dim must be a multiple of the MFMA contraction");
};

// ------------------------------------------------------------- fragments
template <typename T>
__device__ __forceinline__ typename Mma<T>::Frag frag_load16(const T* p);  // 16-byte aligned
template <>
__device__ __forceinline__ bf16x8 frag_load16<__bf16>(const __bf16* p) { return *reinterpret_cast<const bf16x8*>(p); }
template <>
__device__ __forceinline__ f16x8 frag_load16<_Float16>(const _Float16* p) { return *reinterpret_cast<const f16x8*>(p); }
template <>
__device__ __forceinline__ float frag_load16<float>(const float* p) { return *p; }

template <typename T>
__device__ __forceinline__ typename Mma<T>::Frag frag_load8(const T* p);  // 8-byte aligned
template <>
__device__ __forceinline__ bf16x8 frag_load8<__bf16>(const __bf16* p) {
    typedef __attribute__((ext_vector_type(4))) __bf16 b4;
    b4 lo = *reinterpret_cast<const b4*>(p), hi = *reinterpret_cast<const b4*>(p + 4);
    return __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
}
template <>
__device__ __forceinline__ f16x8 frag_load8<_Float16>(const _Float16* p) {
    typedef __attribute__((ext_vector_type(4))) _Float16 h4;
    h4 lo = *reinterpret_cast<const h4*>(p), hi = *reinterpret_cast<const h4*>(p + 4);
    return __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
}
template <>
__device__ __forceinline__ float frag_load8<float>(const float* p) { return *p; }

template <typename T>
__device__ __forceinline__ typename Mma<T>::Frag frag_fill(float v);
template <>
__device__ __forceinline__ bf16x8 frag_fill<__bf16>(float v) {
    __bf16 b = (__bf16)v;
    return bf16x8{b, b, b, b, b, b, b, b};
}
template <>
__device__ __forceinline__ f16x8 frag_fill<_Float16>(float v) {
    _Float16 h = (_Float16)v;
    return f16x8{h, h, h, h, h, h, h, h};
}
template <>
__device__ __forceinline__ float frag_fill<float>(float v) { return v; }

// Probabilities p[16] of one tile -> B operand of PV k-step ks.
template <typename T>
__device__ __forceinline__ typename Mma<T>::Frag frag_from_p(const float* p, int ks);
template <>
__device__ __forceinline__ bf16x8 frag_from_p<__bf16>(const float* p, int ks) {
    bf16x8 f;
#pragma unroll
    for (int j = 0; j < 8; ++j) f[j] = (__bf16)p[8 * ks + j];
    return f;
}
template <>
__device__ __forceinline__ f16x8 frag_from_p<_Float16>(const float* p, int ks) {
    f16x8 f;
#pragma unroll
    for (int j = 0; j < 8; ++j) f[j] = (_Float16)p[8 * ks + j];
    return f;
}
template <>
__device__ __forceinline__ float frag_from_p<float>(const float* p, int ks) { return p[ks]; }

// --------------------------------------------------------------- state
template <int MB>
struct Soft {
    f32x16 acc[MB];
    float m;  // running max of the scaled scores (log2 units)
    float l;  // partial denominator of this lane's keys (when no ones row)
    __device__ __forceinline__ void reset() {
#pragma unroll
        for (int b = 0; b < MB; ++b)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[b][r] = 0.f;
        m = -INFINITY;
        l = 0.f;
    }
};

// Score tile S^T[32 keys x 32 queries] = init + K Q^T from preloaded key
// fragments; init carries the mask (0 or -inf per score) when there is one.
template <typename C>
__device__ __forceinline__ f32x16 score_tile(const typename C::Frag* kf, const typename C::Frag* qf,
                                             f32x16 init) {
#pragma unroll
    for (int t = 0; t < C::NT; ++t) init = C::M::mfma(kf[t], qf[t], init);
    return init;
}

template <typename C>
__device__ __forceinline__ f32x16 score_tile(const typename C::Frag* kf, const typename C::Frag* qf) {
    f32x16 zero;
#pragma unroll
    for (int r = 0; r < 16; ++r) zero[r] = 0.f;
    return score_tile<C>(kf, qf, zero);
}

// Rows [D, 32 * MB) of a transposed V buffer: the ones row (channel D, when
// the O^T padding holds the denominator) and zero rows.  Written once; the
// staging only ever writes rows < D, so the fragments need no selects.
template <typename C>
__device__ __forceinline__ void init_v_padding(typename C::T_* V, int vstride, int cols) {
    typedef typename C::T_ T;
    const int rows = 32 * C::MB - C::D;
    for (int i = threadIdx.x; i < rows * cols; i += blockDim.x) {
        const int r = i / cols, c = i - r * cols;
        V[(C::D + r) * vstride + c] = from_f32<T>((C::ONES && r == 0) ? 1.f : 0.f);
    }
}

// Column of element (row, col) in a transposed buffer whose 8-column groups
// are XOR-swizzled by row: group ^= (row / 8) & MASK (MASK = 0: no swizzle).
// Rows 8 apart start in different bank ranges, so a 16-bit store of 6 channels x
// 11 consecutive columns per wave spreads over the banks, while a 16-byte read
// of 8 consecutive rows at one logical group stays conflict-free.
template <int MASK>
__device__ __forceinline__ int swz_col(int row, int col) {
    return MASK ? col ^ (((row >> 3) & MASK) << 3) : col;
}

// Value fragments of block mb / k-step ks for a tile whose key 0 sits at
// column `col` of a transposed V buffer with 32 * MB rows (8-column groups
// swizzled by swz_col<MASK>).
template <typename C, bool ALIGNED16, int MASK = 0>
__device__ __forceinline__ void load_vfrags(const typename C::T_* Vs, int vstride, int col, int lane,
                                            typename C::Frag* vf) {
    typedef typename C::T_ T;
    const int g = lane >> 5, qi = lane & 31;
#pragma unroll
    for (int mb = 0; mb < C::MB; ++mb)
#pragma unroll
        for (int ks = 0; ks < C::KSTEPS; ++ks) {
            const int row = 32 * mb + qi;
            const T* p = Vs + row * vstride + swz_col<MASK>(row, col + ks * C::KS + C::E * g);
            vf[mb * C::KSTEPS + ks] = ALIGNED16 ? frag_load16<T>(p) : frag_load8<T>(p);
        }
}

// Key fragments of one tile; krow points at this lane's key row (offset by E * g).
template <typename C>
__device__ __forceinline__ void load_kfrags(const typename C::T_* krow, typename C::Frag* kf) {
#pragma unroll
    for (int t = 0; t < C::NT; ++t) kf[t] = frag_load16<typename C::T_>(krow + t * C::KS);
}

// ------------------------------------------------------------- LDS DMA
// LDS byte address of a pointer into the workgroup's shared memory.
template <typename T>
__device__ __forceinline__ uint32_t lds_address(const T* p) {
    return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) T*)p;
}

// One LDS DMA copy (global_load_lds_dwordx4): lane i's 16 bytes from global
// memory go to LDS byte address m0 + 16 i, with no register in between.  m0
// is wave-uniform.  Completion counts on the vector-memory counter.
__device__ __forceinline__ void dma_copy16(const void* base, uint32_t offset, uint32_t m0) {
    asm volatile("global_load_lds_dwordx4 %0, %1" ::"v"(offset), "s"(base), "{m0}"(m0) : "memory");
}
__device__ __forceinline__ void dma_copy16(const void* src, uint32_t m0) {
    asm volatile("global_load_lds_dwordx4 %0, off" ::"v"(src), "{m0}"(m0) : "memory");
}

// Wait for this wave's LDS DMA copies and its LDS reads, before the barrier
// after which another wave's copy may overwrite what they read.
__device__ __forceinline__ void dma_wait() { asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)" ::: "memory"); }

// Transposed fragment of 16-bit rows for a 32x32x16 A operand: lane l holds
// column (channel) c0 + l % 32 of the 8 rows row0 .. row0 + 7 (row stride
// `stride` elements), from two ds_read_b64_tr_b16.  Within a 16-lane block,
// lane B + 4a + e receives element e of the 8-byte windows addressed by lanes
// B + a + 4j (j = 0..3), so lane l addresses row row0 + (l % 16) / 4 (four
// rows further for the second read) at column c0 + 16 ((l / 16) % 2) +
// 4 (l % 4).  cmax: the last 16-column block that may be read (blocks past it
// read that one instead; the caller replaces their values).
template <typename T, typename Frag>
__device__ __forceinline__ Frag tr_frag(const T* rows, int row0, int stride, int c0, int cmax, int lane) {
    typedef short v4s __attribute__((ext_vector_type(4)));
    typedef short v8s __attribute__((ext_vector_type(8)));
    typedef __attribute__((address_space(3))) v4s* lds_v4s;
    const int blk = min(c0 + 16 * ((lane >> 4) & 1), cmax);
    const T* p = rows + (row0 + ((lane & 15) >> 2)) * stride + blk + 4 * (lane & 3);
    const v4s lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4s)p);
    const v4s hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4s)(p + 4 * stride));
    const v8s v = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
    return __builtin_bit_cast(Frag, v);
}

// The running max only moves when a tile's max exceeds it by more than this
// many log2 units, so the accumulator is rarely rescaled; probabilities are
// then bounded by 2^kLazy, far inside the fp32 / bf16 / fp16 range.
constexpr float kLazy = 8.f;

// Online-softmax step for one tile of raw (masked) scores s: updates the
// running max (lazily), rescales the accumulator when it moved, and returns
// the unnormalised probabilities p = 2^(s * scale_log2 - m).
template <typename C>
__device__ __forceinline__ void soft_probs(Soft<C::MB>& st, const f32x16& s, float scale_log2, float* p) {
    float tmax = fmaxf(s[0], s[1]);
#pragma unroll
    for (int r = 2; r < 16; r += 2) tmax = fmaxf(tmax, fmaxf(s[r], s[r + 1]));
    tmax = fmaxf(tmax, swap_half(tmax)) * scale_log2;
    const bool move = tmax > st.m + kLazy || (st.m == -INFINITY && tmax > -INFINITY);
    if (__builtin_amdgcn_ballot_w64(move)) {
        const float m_new = move ? tmax : st.m;
        const float alpha = move ? __builtin_amdgcn_exp2f(st.m - m_new) : 1.f;
#pragma unroll
        for (int b = 0; b < C::MB; ++b)
#pragma unroll
            for (int r = 0; r < 16; ++r) st.acc[b][r] *= alpha;
        if constexpr (!C::ONES) st.l *= alpha;
        st.m = m_new;
    }
    const float base = st.m == -INFINITY ? 0.f : st.m;
    float psum = 0.f;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
        p[r] = __builtin_amdgcn_exp2f(fmaf(s[r], scale_log2, -base));
        if constexpr (!C::ONES) psum += p[r];
    }
    if constexpr (!C::ONES) st.l += psum;
}

// Softmax step against a fixed reference point st.m that bounds every score
// of the query (st.m >= scale_log2 * max score): p = 2^(s * scale_log2 - m)
// <= 1, with no running max, rescale or branch.  Exact as long as the bound
// is not so loose that every p underflows, which the caller checks.
// s already holds score * scale_log2 - m (the score MFMA starts from -m).
template <typename C>
__device__ __forceinline__ void soft_probs_bounded(Soft<C::MB>& st, const f32x16& s, float* p) {
    float psum = 0.f;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
        p[r] = __builtin_amdgcn_exp2f(s[r]);
        if constexpr (!C::ONES) psum += p[r];
    }
    if constexpr (!C::ONES) st.l += psum;
}

// Squared 2-norm of this lane's query (both lane groups hold half the channels).
template <typename C>
__device__ __forceinline__ float q_norm(const typename C::Frag* qf) {
    float sq = 0.f;
#pragma unroll
    for (int t = 0; t < C::NT; ++t) {
        if constexpr (C::E == 1) {
            sq += qf[t] * qf[t];
        } else {
#pragma unroll
            for (int j = 0; j < C::E; ++j) sq += to_f32(qf[t][j]) * to_f32(qf[t][j]);
        }
    }
    return sqrtf(sq + swap_half(sq));
}

// acc += V^T P^T with preloaded value fragments vf[mb * KSTEPS + ks].
template <typename C>
__device__ __forceinline__ void soft_accumulate(Soft<C::MB>& st, const float* p, const typename C::Frag* vf) {
#pragma unroll
    for (int ks = 0; ks < C::KSTEPS; ++ks) {
        const typename C::Frag pf = frag_from_p<typename C::T_>(p, ks);
#pragma unroll
        for (int b = 0; b < C::MB; ++b) st.acc[b] = C::M::mfma(vf[b * C::KSTEPS + ks], pf, st.acc[b]);
    }
}

// Total denominator of this lane's query.
template <typename C>
__device__ __forceinline__ float soft_denominator(const Soft<C::MB>& st, int g) {
    if constexpr (C::ONES) {
        const float v = st.acc[C::ONES_MB][C::ONES_R];
        const float other = swap_half(v);
        return g == C::ONES_G ? v : other;
    } else {
        return st.l + swap_half(st.l);
    }
}

}  // namespace p3d
