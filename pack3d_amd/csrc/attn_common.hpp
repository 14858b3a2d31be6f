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

// Score tile: S^T[32 keys x 32 queries].  krow points at this lane's key row
// (already offset by E * g).
template <typename C, typename T>
__device__ __forceinline__ f32x16 score_tile(const T* krow, const typename C::Frag* qf) {
    f32x16 s;
#pragma unroll
    for (int r = 0; r < 16; ++r) s[r] = 0.f;
#pragma unroll
    for (int t = 0; t < C::NT; ++t) s = C::M::mfma(frag_load16<T>(krow + t * C::KS), qf[t], s);
    return s;
}

// Online-softmax update with the tile's (masked) raw scores s, then
// acc += V^T P^T.  vload(mb, ks) returns the V fragment of block mb, k-step ks.
template <typename C, typename VLoad>
__device__ __forceinline__ void soft_update(Soft<C::MB>& st, const f32x16& s, float scale_log2, VLoad vload) {
    float tmax = s[0];
#pragma unroll
    for (int r = 1; r < 16; ++r) tmax = fmaxf(tmax, s[r]);
    tmax = fmaxf(tmax, swap_half(tmax));
    const float m_new = fmaxf(st.m, tmax * scale_log2);
    const float base = m_new == -INFINITY ? 0.f : m_new;
    const float alpha = __builtin_amdgcn_exp2f(st.m - base);
    float p[16];
    float psum = 0.f;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
        p[r] = __builtin_amdgcn_exp2f(fmaf(s[r], scale_log2, -base));
        if constexpr (!C::ONES) psum += p[r];
    }
    st.m = m_new;
    if constexpr (!C::ONES) st.l = fmaf(st.l, alpha, psum);
#pragma unroll
    for (int b = 0; b < C::MB; ++b)
#pragma unroll
        for (int r = 0; r < 16; ++r) st.acc[b][r] *= alpha;
#pragma unroll
    for (int ks = 0; ks < C::KSTEPS; ++ks) {
        const typename C::Frag pf = frag_from_p<typename C::T_>(p, ks);
#pragma unroll
        for (int b = 0; b < C::MB; ++b) st.acc[b] = C::M::mfma(vload(b, ks), pf, st.acc[b]);
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
