// Integer geometry kernels: layout construction, validation, reverse
// adjacency and repack transport.  Every output is bit-exact with the CPU
// construction of amilworks/Pack3D (src/pack3d/geometry.py).
#include <climits>

#include "common.hpp"

namespace p3d {
namespace {

constexpr int kThreads = 256;

inline unsigned grid1d(int64_t n) { return (unsigned)cdiv(n, kThreads); }

__global__ void k_fill_i32(int32_t* p, int64_t n, int32_t v) {
    int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) p[i] = v;
}

__global__ void k_fill_i64(int64_t* p, int64_t n, int64_t v) {
    int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) p[i] = v;
}

// Number of points q of the box [0,E0) x [0,E1) x [0,E2) whose Morton code
// is smaller than that of p.  Codes interleave bit b of axis a at bit 3b+a
// (geometry.py:118-126).  Scanning code bits from the top, every 1 bit of p
// contributes the points that agree with p above it, hold 0 there and are
// free below; per axis that set is an aligned power-of-two interval clipped
// to the box, so the count is a product of three clipped lengths.
__device__ int64_t morton_rank(const int64_t p[3], const int64_t E[3], int nbits) {
    int64_t rank = 0;
    for (int b = nbits - 1; b >= 0; --b) {
        for (int a = 2; a >= 0; --a) {
            if (!((p[a] >> b) & 1)) continue;
            int64_t count = 1;
            for (int c = 0; c < 3 && count; ++c) {
                int64_t prefix;
                int k;
                if (c == a) {
                    prefix = (p[a] >> (b + 1)) << 1;
                    k = b;
                } else if (c < a) {
                    prefix = p[c] >> (b + 1);
                    k = b + 1;
                } else {
                    prefix = p[c] >> b;
                    k = b;
                }
                int64_t room = E[c] - (prefix << k);
                int64_t span = (int64_t)1 << k;
                count = room <= 0 ? 0 : count * (room < span ? room : span);
            }
            rank += count;
        }
    }
    return rank;
}

struct LayoutDims {
    int64_t g[3], blk[3], r[3];
    int64_t n, volume;
    int morton, nbits;
};

// Per raster token t: packed row, order, coordinates and raster->packed map
// (geometry.py:241-252).  Morton keys block_code*(max_slot+1)+slot_code are
// ordered lexicographically by (block code, slot code) and every block holds
// every slot, so the packed row is rank(block) * volume + rank(slot).
__global__ void k_layout_map(LayoutDims d, int64_t* order, int64_t* coords, int32_t* map) {
    int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= d.n) return;
    int64_t x = t % d.g[2];
    int64_t y = (t / d.g[2]) % d.g[1];
    int64_t z = t / (d.g[2] * d.g[1]);
    int64_t packed = t;
    if (d.morton) {
        int64_t bc[3] = {z / d.blk[0], y / d.blk[1], x / d.blk[2]};
        int64_t sc[3] = {z % d.blk[0], y % d.blk[1], x % d.blk[2]};
        int64_t be[3] = {d.g[0] / d.blk[0], d.g[1] / d.blk[1], d.g[2] / d.blk[2]};
        packed = morton_rank(bc, be, d.nbits) * d.volume + morton_rank(sc, d.blk, d.nbits);
    }
    if (map) map[t] = (int32_t)packed;
    order[packed] = t;
    coords[3 * packed + 0] = z;
    coords[3 * packed + 1] = y;
    coords[3 * packed + 2] = x;
}

// Neighbour column k is offset ((dz+rz)(2ry+1)+(dy+ry))(2rx+1)+(dx+rx), the
// itertools.product order of geometry.py:254-259; absent neighbours are -1.
__global__ void k_layout_neighbors(LayoutDims d, int64_t width, const int64_t* coords,
                                   const int32_t* map, int32_t* nb) {
    int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (e >= d.n * width) return;
    int64_t i = e / width;
    int64_t k = e - i * width;
    int64_t wy = 2 * d.r[1] + 1, wx = 2 * d.r[2] + 1;
    int64_t off[3] = {k / (wy * wx) - d.r[0], (k / wx) % wy - d.r[1], k % wx - d.r[2]};
    int64_t raster = 0;
    bool inside = true;
    for (int a = 0; a < 3; ++a) {
        int64_t c = coords[3 * i + a] + off[a];
        inside = inside && c >= 0 && c < d.g[a];
        raster = raster * d.g[a] + c;
    }
    nb[e] = inside ? (map ? map[raster] : (int32_t)raster) : -1;
}

__global__ void k_iota_i32(int32_t* p, int64_t n) {
    int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) p[i] = (int32_t)i;
}

// ----------------------------------------------------------- validation
template <typename I>
__global__ void k_check_neighbors(const I* nb, int64_t count, int64_t n, int32_t* out,
                                  int32_t* degree, int32_t* flags) {
    int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (e >= count) return;
    int64_t v = (int64_t)nb[e];
    bool bad = v < -1 || v >= n;
    out[e] = bad ? -1 : (int32_t)v;
    if (bad) atomicAdd(&flags[0], 1);
    else if (v >= 0) atomicAdd(&degree[v], 1);
}

template <typename I>
__global__ void k_check_blocks(const I* blocks, int64_t count, int64_t n, int32_t* out,
                               int32_t* cover, int32_t* flags) {
    int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (e >= count) return;
    int64_t v = (int64_t)blocks[e];
    bool bad = v < -1 || v >= n;
    out[e] = bad ? -1 : (int32_t)v;
    if (bad) atomicAdd(&flags[1], 1);
    else if (v >= 0) atomicAdd(&cover[v], 1);
}

// Bitonic sort of up to 128 int32 values held by one wave: element e lives in
// lane e % 64, register e / 64.  Ascending.
__device__ void wave_sort128(int32_t& a0, int32_t& a1) {
    const int lane = threadIdx.x & 63;
    for (int k = 2; k <= 128; k <<= 1) {
        for (int j = k >> 1; j >= 1; j >>= 1) {
            if (j == 64) {
                int32_t lo = min(a0, a1), hi = max(a0, a1);
                a0 = lo;
                a1 = hi;  // k == 128: every pair ascends
                continue;
            }
            for (int r = 0; r < 2; ++r) {
                int32_t v = r ? a1 : a0;
                int32_t p = __shfl_xor(v, j);
                int e = r * 64 + lane;
                bool up = (e & k) == 0;
                bool lower = (e & j) == 0;
                int32_t keep = (lower == up) ? min(v, p) : max(v, p);
                if (r) a1 = keep; else a0 = keep;
            }
        }
    }
}

// One wave per row: sort the row and look for equal valid neighbours.
__global__ void k_check_duplicates(const int32_t* nb, int64_t n, int32_t width, int32_t* flags) {
    int64_t row = (int64_t)blockIdx.x * (blockDim.x / 64) + threadIdx.x / 64;
    if (row >= n) return;
    const int lane = threadIdx.x & 63;
    const int32_t* p = nb + row * width;
    int32_t a0 = lane < width ? p[lane] : INT_MAX;
    int32_t a1 = lane + 64 < width ? p[lane + 64] : INT_MAX;
    if (a0 < 0) a0 = INT_MAX;
    if (a1 < 0) a1 = INT_MAX;
    wave_sort128(a0, a1);
    // Element e = r*64+lane; compare with element e+1.
    int32_t next0 = __shfl_down(a0, 1);
    int32_t first1 = __shfl(a1, 0);
    if (lane == 63) next0 = first1;
    int32_t next1 = __shfl_down(a1, 1);
    bool dup = (a0 != INT_MAX && a0 == next0) || (lane < 63 && a1 != INT_MAX && a1 == next1);
    unsigned long long any = __ballot(dup);
    if (lane == 0 && any) atomicAdd(&flags[2], 1);
}

__global__ void k_check_cover(const int32_t* cover, const int32_t* degree, int64_t n, int32_t* flags) {
    int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= n) return;
    if (cover[t] != 1) atomicAdd(&flags[3], 1);
    atomicMax(&flags[5], degree[t]);
}

__global__ void k_check_groups(const int32_t* blocks, int64_t fine, int32_t slots, int32_t pool,
                               int64_t groups, int32_t* flags) {
    int64_t g = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (g >= groups) return;
    int64_t end = min(fine, (g + 1) * pool);
    bool any = false;
    for (int64_t f = g * pool; f < end && !any; ++f)
        for (int s = 0; s < slots; ++s) any = any || blocks[f * slots + s] >= 0;
    if (!any) atomicAdd(&flags[4], 1);
}

// ------------------------------------------------------ reverse adjacency
__global__ void k_reverse_scatter(const int32_t* nb, int64_t count, int32_t width, int32_t* cursor,
                                  int32_t* reverse, int32_t rwidth) {
    int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (e >= count) return;
    int32_t j = nb[e];
    if (j < 0) return;
    int32_t slot = atomicAdd(&cursor[j], 1);
    if (slot < rwidth) reverse[(int64_t)j * rwidth + slot] = (int32_t)(e / width);
}

// Rows were filled in arbitrary order; sorting restores the ascending source
// order that the stable argsort of geometry.py:90 produces.
__global__ void k_reverse_sort(int32_t* reverse, int64_t n, int32_t rwidth) {
    int64_t row = (int64_t)blockIdx.x * (blockDim.x / 64) + threadIdx.x / 64;
    if (row >= n) return;
    const int lane = threadIdx.x & 63;
    int32_t* p = reverse + row * rwidth;
    int32_t a0 = lane < rwidth ? p[lane] : INT_MAX;
    int32_t a1 = lane + 64 < rwidth ? p[lane + 64] : INT_MAX;
    if (a0 < 0) a0 = INT_MAX;
    if (a1 < 0) a1 = INT_MAX;
    wave_sort128(a0, a1);
    if (lane < rwidth) p[lane] = a0 == INT_MAX ? -1 : a0;
    if (lane + 64 < rwidth) p[lane + 64] = a1 == INT_MAX ? -1 : a1;
}

// ---------------------------------------------------------------- repack
__global__ void k_invert(const int64_t* perm, int64_t n, int64_t* inverse, int32_t* flags) {
    int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    int64_t v = perm[i];
    if (v < 0 || v >= n) {
        atomicAdd(&flags[0], 1);
        return;
    }
    unsigned long long prev = atomicCAS(reinterpret_cast<unsigned long long*>(inverse + v),
                                        (unsigned long long)(-1LL), (unsigned long long)i);
    if (prev != (unsigned long long)(-1LL)) atomicAdd(&flags[0], 1);
}

__device__ __forceinline__ int32_t relabel(int32_t old, const int64_t* inverse) {
    return old >= 0 ? (int32_t)inverse[old] : -1;
}

__global__ void k_repack_rows(const int64_t* perm, int64_t n, const int32_t* nb, int32_t width,
                              const int64_t* inverse, int32_t* nb_out) {
    int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (e >= n * width) return;
    int64_t i = e / width;
    int64_t src = perm[i];
    nb_out[e] = (src >= 0 && src < n) ? relabel(nb[src * width + (e - i * width)], inverse) : -1;
}

__global__ void k_repack_tokens(const int64_t* perm, int64_t n, const int64_t* order, const int64_t* coords,
                                const int32_t* map, const int64_t* inverse, int64_t* order_out,
                                int64_t* coords_out, int32_t* map_out) {
    int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    int64_t src = perm[i];
    bool ok = src >= 0 && src < n;
    order_out[i] = ok ? order[src] : -1;
    for (int a = 0; a < 3; ++a) coords_out[3 * i + a] = ok ? coords[3 * src + a] : -1;
    if (map_out) map_out[i] = (int32_t)inverse[map ? map[i] : i];
}

__global__ void k_relabel(const int32_t* in, int64_t count, const int64_t* inverse, int32_t* out) {
    int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (e < count) out[e] = relabel(in[e], inverse);
}

__global__ void k_check_layout(LayoutDims d, const int64_t* order, const int64_t* coords,
                               int32_t* seen, int32_t* flags) {
    int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= d.n) return;
    int64_t t = order[i];
    if (t < 0 || t >= d.n) {
        atomicAdd(&flags[0], 1);
        return;
    }
    if (atomicAdd(&seen[t], 1) != 0) atomicAdd(&flags[0], 1);
    int64_t x = t % d.g[2], y = (t / d.g[2]) % d.g[1], z = t / (d.g[2] * d.g[1]);
    if (coords[3 * i] != z || coords[3 * i + 1] != y || coords[3 * i + 2] != x) atomicAdd(&flags[0], 1);
}

// ------------------------------------------------------ stencil match
// raster index -> packed row from a layout's order (order[i] = raster index of
// row i; map starts at -1); entries outside [0, n) and raster indices that
// appear twice (order is then no permutation, and some raster index is left
// without a row) are counted in flags[0].
__global__ void k_scatter_order(const int64_t* order, int64_t n, int32_t* map, int32_t* flags) {
    int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    int64_t t = order[i];
    if (t < 0 || t >= n) {
        atomicAdd(&flags[0], 1);
        return;
    }
    if (atomicExch(&map[t], (int32_t)i) != -1) atomicAdd(&flags[0], 1);
}

// Counts in flags[1] the entries of nb [N, W] that differ from the complete
// product-order stencil of radius d.r on grid d.g, evaluated at each row's
// raster coordinate (the table build_layout makes, geometry.py:253-259).
__global__ void k_compare_stencil(LayoutDims d, int64_t width, const int64_t* order, const int32_t* map,
                                  const int32_t* nb, int32_t* flags) {
    int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (e >= d.n * width) return;
    int64_t i = e / width;
    int64_t k = e - i * width;
    int64_t t = order[i];
    if (t < 0 || t >= d.n) return;  // counted by k_scatter_order
    int64_t c[3] = {t / (d.g[2] * d.g[1]), (t / d.g[2]) % d.g[1], t % d.g[2]};
    int64_t wy = 2 * d.r[1] + 1, wx = 2 * d.r[2] + 1;
    int64_t off[3] = {k / (wy * wx) - d.r[0], (k / wx) % wy - d.r[1], k % wx - d.r[2]};
    int64_t raster = 0;
    bool inside = true;
    for (int a = 0; a < 3; ++a) {
        int64_t v = c[a] + off[a];
        inside = inside && v >= 0 && v < d.g[a];
        raster = raster * d.g[a] + (inside ? v : 0);
    }
    int32_t expect = inside ? map[raster] : -1;
    if (nb[e] != expect) atomicAdd(&flags[1], 1);
}

}  // namespace
}  // namespace p3d

using namespace p3d;

extern "C" int p3d_build_layout(const int64_t grid[3], const int64_t block[3], const int64_t radius[3],
                                int32_t morton, int64_t* order, int64_t* coords,
                                int32_t* raster_to_packed, int32_t* neighbors, int32_t* blocks,
                                void* stream) {
    LayoutDims d{};
    d.n = 1;
    d.volume = 1;
    int64_t width = 1;
    for (int a = 0; a < 3; ++a) {
        P3D_REQUIRE(grid[a] >= 1 && block[a] >= 1 && radius[a] >= 0, "invalid grid, block or radius");
        P3D_REQUIRE(grid[a] % block[a] == 0, "grid must be divisible by block_shape");
        d.g[a] = grid[a];
        d.blk[a] = block[a];
        d.r[a] = radius[a];
        d.n *= grid[a];
        d.volume *= block[a];
        width *= 2 * radius[a] + 1;
    }
    P3D_REQUIRE(d.volume <= 64 && width <= 128, "layout exceeds supported block or neighborhood width");
    P3D_REQUIRE(d.n * width < ((int64_t)1 << 31), "geometry exceeds the 32-bit kernel indexing limit");
    P3D_REQUIRE(order && coords && neighbors && blocks, "null output");
    P3D_REQUIRE(!morton || raster_to_packed, "morton layouts need the raster->packed map");
    d.morton = morton != 0;
    d.nbits = 21;
    hipStream_t s = as_stream(stream);
    k_layout_map<<<grid1d(d.n), kThreads, 0, s>>>(d, order, coords, raster_to_packed);
    k_layout_neighbors<<<grid1d(d.n * width), kThreads, 0, s>>>(d, width, coords,
                                                                 morton ? raster_to_packed : nullptr,
                                                                 neighbors);
    k_iota_i32<<<grid1d(d.n), kThreads, 0, s>>>(blocks, d.n);
    return check_launch("p3d_build_layout");
}

extern "C" int p3d_geometry_check(const void* neighbors, int32_t nb_is64, int64_t n, int32_t width,
                                  const void* blocks, int32_t blocks_is64, int64_t fine, int32_t slots,
                                  int32_t pool_size, int32_t* neighbors32, int32_t* blocks32,
                                  int32_t* degree, int32_t* cover, int32_t* flags, void* stream) {
    P3D_REQUIRE(n >= 1 && width >= 1 && width <= 128 && fine >= 1 && slots >= 1 && slots <= 64,
                "invalid geometry shape");
    P3D_REQUIRE(pool_size >= 1 && pool_size <= 32, "pool_size must be an integer in [1,32]");
    hipStream_t s = as_stream(stream);
    k_fill_i32<<<1, 64, 0, s>>>(flags, 8, 0);
    k_fill_i32<<<grid1d(n), kThreads, 0, s>>>(degree, n, 0);
    k_fill_i32<<<grid1d(n), kThreads, 0, s>>>(cover, n, 0);
    int64_t cnb = n * width, cbl = fine * slots;
    if (nb_is64)
        k_check_neighbors<<<grid1d(cnb), kThreads, 0, s>>>((const int64_t*)neighbors, cnb, n, neighbors32, degree, flags);
    else
        k_check_neighbors<<<grid1d(cnb), kThreads, 0, s>>>((const int32_t*)neighbors, cnb, n, neighbors32, degree, flags);
    if (blocks_is64)
        k_check_blocks<<<grid1d(cbl), kThreads, 0, s>>>((const int64_t*)blocks, cbl, n, blocks32, cover, flags);
    else
        k_check_blocks<<<grid1d(cbl), kThreads, 0, s>>>((const int32_t*)blocks, cbl, n, blocks32, cover, flags);
    k_check_duplicates<<<(unsigned)cdiv(n, 4), 256, 0, s>>>(neighbors32, n, width, flags);
    k_check_cover<<<grid1d(n), kThreads, 0, s>>>(cover, degree, n, flags);
    int64_t groups = cdiv(fine, pool_size);
    k_check_groups<<<grid1d(groups), kThreads, 0, s>>>(blocks32, fine, slots, pool_size, groups, flags);
    return check_launch("p3d_geometry_check");
}

extern "C" int p3d_reverse_adjacency(const int32_t* neighbors, int64_t n, int32_t width, int32_t* cursor,
                                     int32_t* reverse, int32_t rwidth, void* stream) {
    P3D_REQUIRE(n >= 1 && width >= 1 && rwidth >= 1 && rwidth <= 128, "invalid reverse adjacency shape");
    hipStream_t s = as_stream(stream);
    k_fill_i32<<<grid1d(n), kThreads, 0, s>>>(cursor, n, 0);
    k_fill_i32<<<grid1d(n * rwidth), kThreads, 0, s>>>(reverse, n * rwidth, -1);
    k_reverse_scatter<<<grid1d(n * width), kThreads, 0, s>>>(neighbors, n * width, width, cursor, reverse, rwidth);
    k_reverse_sort<<<(unsigned)cdiv(n, 4), 256, 0, s>>>(reverse, n, rwidth);
    return check_launch("p3d_reverse_adjacency");
}

extern "C" int p3d_repack(const int64_t* perm, int64_t n, const int32_t* neighbors, int32_t width,
                          const int32_t* blocks, int64_t fine, int32_t slots, const int64_t* order,
                          const int64_t* coords, const int32_t* raster_map, int64_t* inverse,
                          int32_t* neighbors_out, int32_t* blocks_out, int64_t* order_out,
                          int64_t* coords_out, int32_t* raster_map_out, int32_t* flags, void* stream) {
    P3D_REQUIRE(n >= 1 && width >= 1 && fine >= 1 && slots >= 1, "invalid repack shape");
    hipStream_t s = as_stream(stream);
    k_fill_i32<<<1, 64, 0, s>>>(flags, 8, 0);
    k_fill_i64<<<grid1d(n), kThreads, 0, s>>>(inverse, n, -1);
    k_invert<<<grid1d(n), kThreads, 0, s>>>(perm, n, inverse, flags);
    // A rejected permutation leaves some inverse entries at -1; clamp them so
    // the gathers below stay in bounds (the caller raises on flags[0]).
    k_repack_rows<<<grid1d(n * width), kThreads, 0, s>>>(perm, n, neighbors, width, inverse, neighbors_out);
    k_relabel<<<grid1d(fine * slots), kThreads, 0, s>>>(blocks, fine * slots, inverse, blocks_out);
    k_repack_tokens<<<grid1d(n), kThreads, 0, s>>>(perm, n, order, coords, raster_map, inverse, order_out,
                                                  coords_out, raster_map_out);
    return check_launch("p3d_repack");
}

extern "C" int p3d_check_layout(const int64_t grid[3], const int64_t* order, const int64_t* coords,
                                int32_t* scratch, int32_t* flags, void* stream) {
    LayoutDims d{};
    d.n = grid[0] * grid[1] * grid[2];
    for (int a = 0; a < 3; ++a) d.g[a] = grid[a];
    P3D_REQUIRE(d.n >= 1, "empty grid");
    hipStream_t s = as_stream(stream);
    k_fill_i32<<<1, 64, 0, s>>>(flags, 8, 0);
    k_fill_i32<<<grid1d(d.n), kThreads, 0, s>>>(scratch, d.n, 0);
    k_check_layout<<<grid1d(d.n), kThreads, 0, s>>>(d, order, coords, scratch, flags);
    return check_launch("p3d_check_layout");
}

extern "C" int p3d_stencil_match(const int64_t grid[3], const int64_t radius[3], const int64_t* order,
                                 const int32_t* neighbors, int32_t width, int32_t* raster_to_packed,
                                 int32_t* flags, void* stream) {
    LayoutDims d{};
    d.n = 1;
    int64_t w = 1;
    for (int a = 0; a < 3; ++a) {
        P3D_REQUIRE(grid[a] >= 1 && radius[a] >= 0, "invalid grid or radius");
        d.g[a] = grid[a];
        d.r[a] = radius[a];
        d.n *= grid[a];
        w *= 2 * radius[a] + 1;
    }
    P3D_REQUIRE(w == width, "neighbour width does not match the stencil radius");
    P3D_REQUIRE(d.n * w < ((int64_t)1 << 31), "geometry exceeds the 32-bit kernel indexing limit");
    P3D_REQUIRE(order && neighbors && raster_to_packed && flags, "null argument");
    hipStream_t s = as_stream(stream);
    k_fill_i32<<<1, 64, 0, s>>>(flags, 8, 0);
    k_fill_i32<<<grid1d(d.n), kThreads, 0, s>>>(raster_to_packed, d.n, -1);
    k_scatter_order<<<grid1d(d.n), kThreads, 0, s>>>(order, d.n, raster_to_packed, flags);
    k_compare_stencil<<<grid1d(d.n * w), kThreads, 0, s>>>(d, w, order, raster_to_packed, neighbors, flags);
    return check_launch("p3d_stencil_match");
}
