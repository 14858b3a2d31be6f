// Axial rotary embedding applied on load (rope.py:15-48 of amilworks/Pack3D).
#pragma once

#include "common.hpp"

namespace p3d {

struct RopeDev {
    const float2* table;
    const int32_t* pairs;  // [D/2][3]: base, stride, axis
    const int64_t* coords;
    int packed;
};

inline RopeDev rope_dev(const p3d_rope& r) {
    return RopeDev{reinterpret_cast<const float2*>(r.table), r.pairs, r.coords, r.packed};
}

// Position of packed row n along each axis.
__device__ __forceinline__ void rope_position(const RopeDev& r, int64_t n, int64_t pos[3]) {
    if (r.packed) {
        pos[0] = n;
        pos[1] = 0;
        pos[2] = 0;
    } else {
        pos[0] = r.coords[3 * n + 0];
        pos[1] = r.coords[3 * n + 1];
        pos[2] = r.coords[3 * n + 2];
    }
}

// Coordinate along `axis` (selects, not an indexed array, so it stays in registers).
__device__ __forceinline__ int64_t pick_axis(const int64_t pos[3], int axis) {
    return axis == 0 ? pos[0] : (axis == 1 ? pos[1] : pos[2]);
}

// (cos, sin) of rotary pair j at position pos.
__device__ __forceinline__ float2 rope_cs(const RopeDev& r, int j, const int64_t pos[3]) {
    const int32_t* p = r.pairs + 3 * j;
    return r.table[p[0] + (int64_t)p[1] * pick_axis(pos, p[2])];
}

// Rotate a contiguous run of `count` channels starting at even channel c0.
__device__ __forceinline__ void rope_apply(const RopeDev& r, const int64_t pos[3], int c0, float* x, int count,
                                           bool inverse = false) {
    for (int e = 0; e < count; e += 2) {
        float2 cs = rope_cs(r, (c0 + e) >> 1, pos);
        rotate_pair(x[e], x[e + 1], cs.x, inverse ? -cs.y : cs.y);
    }
}

// Rotary metadata of pair j, for staging in LDS: {base, stride along axis 0,
// along axis 1, along axis 2}, where only the pair's own axis has a non-zero
// stride, so the table index is base + sum_a stride_a * pos[a] with no
// per-pair branch on the axis.
__device__ __forceinline__ int4 pair_meta(const int32_t* pairs, int j) {
    const int base = pairs[3 * j], stride = pairs[3 * j + 1], axis = pairs[3 * j + 2];
    return int4{base, axis == 0 ? stride : 0, axis == 1 ? stride : 0, axis == 2 ? stride : 0};
}

// 32-bit forms for kernels that keep positions of many rows in registers.
// Table indices are base + stride * coordinate < 2^31: coordinates are below
// the token count and the hosts validate rows * head_dim < 2^31.
__device__ __forceinline__ void rope_position32(const RopeDev& r, int n, int pos[3]) {
    if (r.packed) {
        pos[0] = n;
        pos[1] = 0;
        pos[2] = 0;
    } else {
        // Coordinates are non-negative and below 2^31: read the low words of
        // the int64 entries only (no dead high halves held by a load).
        const int32_t* c = reinterpret_cast<const int32_t*>(r.coords) + 6 * (int64_t)n;
        pos[0] = c[0];
        pos[1] = c[2];
        pos[2] = c[4];
    }
}

__device__ __forceinline__ void rope_apply32(const RopeDev& r, const int pos[3], int c0, float* x, int count) {
    for (int e = 0; e < count; e += 2) {
        const int32_t* p = r.pairs + 3 * ((c0 + e) >> 1);
        const int axis = p[2];
        const int coord = axis == 0 ? pos[0] : (axis == 1 ? pos[1] : pos[2]);
        const float2 cs = r.table[p[0] + p[1] * coord];
        rotate_pair(x[e], x[e + 1], cs.x, cs.y);
    }
}

}  // namespace p3d
