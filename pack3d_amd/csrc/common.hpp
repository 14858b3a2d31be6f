// Shared helpers for the gfx950 PACK3D kernels: status reporting, element
// conversion, MFMA operand traits and wavefront utilities.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <string>

#include "../../include/pack3d_hip.h"

namespace p3d {

// ---------------------------------------------------------------- status
void set_error(const std::string& msg);
int fail(int code, const std::string& msg);
int check_launch(const char* what);

#define P3D_REQUIRE(cond, msg)                          \
    do {                                                \
        if (!(cond)) return ::p3d::fail(P3D_EINVAL, msg); \
    } while (0)

inline hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

// ------------------------------------------------------------ elements
typedef __attribute__((ext_vector_type(8))) __bf16 bf16x8;
typedef __attribute__((ext_vector_type(8))) _Float16 f16x8;
typedef __attribute__((ext_vector_type(16))) float f32x16;
typedef __attribute__((ext_vector_type(4))) float f32x4;
typedef __attribute__((ext_vector_type(2))) float f32x2;
typedef __attribute__((ext_vector_type(4))) unsigned int u32x4;  // one 16-byte piece

__device__ __forceinline__ float to_f32(float x) { return x; }
__device__ __forceinline__ float to_f32(_Float16 x) { return (float)x; }
__device__ __forceinline__ float to_f32(__bf16 x) { return (float)x; }

template <typename T>
__device__ __forceinline__ T from_f32(float x);
template <>
__device__ __forceinline__ float from_f32<float>(float x) { return x; }
template <>
__device__ __forceinline__ _Float16 from_f32<_Float16>(float x) { return (_Float16)x; }
template <>
__device__ __forceinline__ __bf16 from_f32<__bf16>(float x) { return (__bf16)x; }

// Load a scalar of runtime dtype (used for the gate, whose dtype may differ).
__device__ __forceinline__ float load_any(const void* p, int64_t i, int dtype) {
    if (dtype == P3D_F32) return reinterpret_cast<const float*>(p)[i];
    if (dtype == P3D_F16) return (float)reinterpret_cast<const _Float16*>(p)[i];
    return (float)reinterpret_cast<const __bf16*>(p)[i];
}

// Product and difference without contraction, so the rotation rounds
// exactly as the separate fp32 multiply / subtract of rope.py:44, in every
// kernel alike.  HIP's __fmul_rn and __fsub_rn are a plain * and -, which the
// compiler may fuse into an fma (it contracts by default), and whether it
// does depends on the surrounding kernel; the pragma marks these operations
// as not contractible wherever they are inlined.
__device__ __forceinline__ float mul_rn(float a, float b) {
#pragma clang fp contract(off)
    return a * b;
}
__device__ __forceinline__ float sub_rn(float a, float b) {
#pragma clang fp contract(off)
    return a - b;
}
__device__ __forceinline__ float add_rn(float a, float b) {
#pragma clang fp contract(off)
    return a + b;
}

// Rotate one channel pair: (x0 c - x1 s, x0 s + x1 c); inverse uses -s.
__device__ __forceinline__ void rotate_pair(float& x0, float& x1, float c, float s) {
    float a = sub_rn(mul_rn(x0, c), mul_rn(x1, s));
    float b = add_rn(mul_rn(x0, s), mul_rn(x1, c));
    x0 = a;
    x1 = b;
}

// ---------------------------------------------------------------- MFMA
// v_mfma_f32_32x32x{16,16,2}: D[32x32] = A[32xK] B[Kx32] + C.
// Operand fragments: lane l holds A row (l % 32) / B column (l % 32) and the
// E contraction elements k = E * (l / 32) + j, j < E.
// Accumulator: lane l, register r holds D[row][l % 32] with
//   row = 8 * (r / 4) + 4 * (l / 32) + (r % 4).
template <typename T>
struct Mma;

template <>
struct Mma<__bf16> {
    static constexpr int E = 8;    // elements per lane per fragment
    static constexpr int KS = 16;  // contraction length per instruction
    typedef bf16x8 Frag;
    __device__ __forceinline__ static f32x16 mfma(Frag a, Frag b, f32x16 c) {
        return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
    }
    // v_mfma_f32_16x16x32: D[16x16] = A[16x32] B[32x16] + C; lane l holds A
    // row / B column l % 16 and k = 8 (l / 16) + j; register r of lane l
    // holds D[4 (l / 16) + r][l % 16].
    __device__ __forceinline__ static f32x4 mfma16(Frag a, Frag b, f32x4 c) {
        return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
    }
};

template <>
struct Mma<_Float16> {
    static constexpr int E = 8;
    static constexpr int KS = 16;
    typedef f16x8 Frag;
    __device__ __forceinline__ static f32x16 mfma(Frag a, Frag b, f32x16 c) {
        return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
    }
    __device__ __forceinline__ static f32x4 mfma16(Frag a, Frag b, f32x4 c) {
        return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
    }
};

template <>
struct Mma<float> {
    static constexpr int E = 1;
    static constexpr int KS = 2;
    typedef float Frag;
    __device__ __forceinline__ static f32x16 mfma(Frag a, Frag b, f32x16 c) {
        return __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, c, 0, 0, 0);
    }
};

// Row of the 32x32 accumulator held by register r in lane group g = l / 32.
__device__ __forceinline__ constexpr int acc_row(int r, int g) { return 8 * (r / 4) + 4 * g + (r % 4); }

// Key order inside a 32-key tile.  When the score tile S^T = K Q^T is used
// directly as the B operand of O^T = V^T P^T, register r of lane group g
// contributes contraction index kappa = (r / E) * KS + E * g + (r % E).  Loading
// K row rho from key kperm(rho) makes kappa the key index, so V can stay in
// natural key order.
template <int E, int KS>
__device__ __forceinline__ constexpr int kperm(int rho) {
    int g = (rho >> 2) & 1;
    int r = 4 * (rho >> 3) + (rho & 3);
    return (r / E) * KS + E * g + (r % E);
}

// Completes the loads of x at this point (an empty asm that reads it).  A
// value loaded before a loop and first used inside it would otherwise get its
// wait inside the loop, where the in-order load counter also makes that wait
// cover the loop's own prefetches on every iteration.
template <typename X>
__device__ __forceinline__ void settle(const X& x) {
    asm volatile("" ::"v"(x));
}

// settle() of every element of each argument (arrays, nested or not).
template <typename X>
__device__ __forceinline__ void settle_all(const X& x) {
    settle(x);
}
__device__ __forceinline__ void settle_all(const float2& x) {
    settle(x.x);
    settle(x.y);
}
template <typename X, size_t N>
__device__ __forceinline__ void settle_all(const X (&x)[N]) {
#pragma unroll
    for (size_t i = 0; i < N; ++i) settle_all(x[i]);
}
template <typename... A>
__device__ __forceinline__ void settle_loads(const A&... a) {
    (settle_all(a), ...);
}

// Raw buffer resource over [base, base + bytes) of global memory, for buffer
// loads with a scalar base and 32-bit per-lane byte offsets (offsets past
// `bytes` read zero).  base must be wave-uniform; it is moved to scalar
// registers here.  The loads need no per-lane address arithmetic, so no
// address temporaries stay live while they are in flight.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buffer_rsrc(const void* base, uint32_t bytes) {
    const uint64_t v = reinterpret_cast<uint64_t>(base);
    // readfirstlane returns a signed int: each half goes through uint32_t so
    // that widening it does not sign-extend the low word into the high one.
    const uint32_t lo = (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)v);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)(v >> 32));
    const uint64_t u = ((uint64_t)hi << 32) | (uint64_t)lo;
    // Word 3: 32-bit data format (the raw-buffer setting of gfx9 parts).
    return __builtin_amdgcn_make_buffer_rsrc(reinterpret_cast<void*>(u), (short)0, (int)bytes, 0x00020000);
}

__device__ __forceinline__ uint4 buffer_load16(__amdgpu_buffer_rsrc_t r, uint32_t offset) {
    typedef unsigned v4u __attribute__((ext_vector_type(4)));
    const v4u x = __builtin_amdgcn_raw_buffer_load_b128(r, offset, 0, 0);
    return uint4{x[0], x[1], x[2], x[3]};
}

__device__ __forceinline__ float buffer_load_f32(__amdgpu_buffer_rsrc_t r, uint32_t offset) {
    return __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(r, offset, 0, 0));
}

// 16-byte store at byte offset `offset` of the resource r over `bytes`
// bytes (a multiple of 16), made by the lanes with ok set: the others aim
// past the end, where the hardware's range check drops the store.  No
// branch surrounds it, so every wave issues the same number of vector
// memory operations on every path, and a later s_waitcnt vmcnt for a load
// issued before it can count past it instead of waiting for its write
// acknowledgement.
__device__ __forceinline__ void buffer_store16(__amdgpu_buffer_rsrc_t r, uint32_t bytes, uint32_t offset, bool ok,
                                               u32x4 v) {
    __builtin_amdgcn_raw_buffer_store_b128(v, r, ok ? offset : bytes, 0, 0);
}

// --------------------------------------------------------------- wave
// Value held by lane l ^ 32.
__device__ __forceinline__ float swap_half(float x) { return __shfl_xor(x, 32); }

// Orders this wave's LDS writes before its later LDS reads of other lanes'
// data (and the compiler's view of them): a wavefront-scope fence pair
// around a wave barrier.
__device__ __forceinline__ void wave_lds_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// x of the lane that the DPP control CTRL selects (a permutation within each
// 16-lane row: every source lane exists, so `old` is never taken).
template <int CTRL>
__device__ __forceinline__ float dpp_move(float x) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), CTRL, 0xf, 0xf, false));
}

// x of lane l ^ 16 and of lane l ^ 32, through the gfx950 row swaps (no LDS).
// permlane16_swap(a, b) exchanges the odd 16-lane rows of a with the even
// rows of b; with a = b = x, an even-row lane finds its partner's value in the
// second result and an odd-row lane in the first.  permlane32_swap does the
// same for the two 32-lane halves.
__device__ __forceinline__ float lane_xor16(float x) {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return __uint_as_float((__lane_id() & 16) ? r[0] : r[1]);
}
__device__ __forceinline__ float lane_xor32(float x) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return __uint_as_float((__lane_id() & 32) ? r[0] : r[1]);
}

// All-reduce over the 64 lanes without LDS: partners l ^ 1, l ^ 2 (quad_perm),
// l ^ 7 within 8 (row_half_mirror), l ^ 15 within 16 (row_mirror), l ^ 16 and
// l ^ 32.  Each step combines two disjoint groups of equal size, and the
// operations are commutative, so every lane ends with the same bits.
__device__ __forceinline__ float wave_max(float x) {
    x = fmaxf(x, dpp_move<0xB1>(x));
    x = fmaxf(x, dpp_move<0x4E>(x));
    x = fmaxf(x, dpp_move<0x141>(x));
    x = fmaxf(x, dpp_move<0x140>(x));
    x = fmaxf(x, lane_xor16(x));
    return fmaxf(x, lane_xor32(x));
}
__device__ __forceinline__ float wave_sum(float x) {
    x += dpp_move<0xB1>(x);
    x += dpp_move<0x4E>(x);
    x += dpp_move<0x141>(x);
    x += dpp_move<0x140>(x);
    x += lane_xor16(x);
    return x + lane_xor32(x);
}
__device__ __forceinline__ int wave_max_i(int x) {
    for (int o = 32; o >= 1; o >>= 1) x = max(x, __shfl_xor(x, o));
    return x;
}

template <typename T>
struct Piece {
    static constexpr int N = 16 / sizeof(T);  // elements per 16-byte piece
};

template <typename T>
__device__ __forceinline__ void load_piece(const T* src, float* out) {
    constexpr int N = Piece<T>::N;
    typedef __attribute__((ext_vector_type(4))) unsigned int u4;
    u4 raw = *reinterpret_cast<const u4*>(src);
    const T* v = reinterpret_cast<const T*>(&raw);
#pragma unroll
    for (int e = 0; e < N; ++e) out[e] = to_f32(v[e]);
}

__host__ __device__ inline int64_t cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }

inline int dtype_size(int dt) { return dt == P3D_F32 ? 4 : 2; }

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

// Rows of the view start on 16-byte boundaries.
inline bool view_ok(const p3d_view& v, int esize) {
    const int64_t step = 16 / esize;
    return v.data && aligned16(v.data) && v.sb % step == 0 && v.sh % step == 0 && v.sn % step == 0;
}

}  // namespace p3d
