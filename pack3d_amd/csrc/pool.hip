// Summary pooling (compression.py:28-44 of amilworks/Pack3D) and the
// standalone rotation (rotary.py:10-45).
//
// One wave pools one coarse summary of one (batch, kv head): for each of its
// fine blocks the wave stages the member rows of K (rotated on load and
// rounded to the storage type, as the reference pools rotated keys stored
// in that type) and V in LDS with coalesced 16-byte loads, computes the slot
// logits, the slot softmax and the weighted sums, and accumulates the fine
// summaries; the coarse mean divides by the number of non-empty fine blocks.
#include <algorithm>

#include "rope.hpp"

namespace p3d {
namespace {

constexpr int kPoolWaves = 4;
// Summary-norm maxima are spread over this many slots per (batch, kv head) so
// that the atomics of different waves rarely meet on one address.
constexpr int kNormSlots = 64;

struct PoolDev {
    int B, G, N, D, F, V, P, M, Mp;
    float inv_tau, key_scale;
    const char *kg, *vg;
    int64_t ksb, ksh, ksn, vsb, vsh, vsn;
    const int32_t* blocks;
    const float* weight;
    const float* bias;
    RopeDev rope;
    void* sk;
    void* svt;
    float* sk_norm_max;
};

template <typename T>
__global__ __launch_bounds__(64 * kPoolWaves) void k_pool_fwd(PoolDev a) {
    const int waves = blockDim.x >> 6;
    constexpr int EP = Piece<T>::N;
    extern __shared__ __align__(16) unsigned char smem_raw[];
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int D = a.D;
    const int stride = D + EP;  // LDS row stride in elements (keeps 16-byte alignment)
    T* lk = reinterpret_cast<T*>(smem_raw) + (size_t)wave * 2 * 64 * stride;
    T* lv = lk + 64 * stride;
    float* la = reinterpret_cast<float*>(reinterpret_cast<T*>(smem_raw) + (size_t)waves * 2 * 64 * stride) +
                wave * 64;

    const int64_t total = (int64_t)a.B * a.G * a.Mp;
    const int64_t item = (int64_t)blockIdx.x * waves + wave;
    if (item >= total) return;  // whole wave leaves; waves never synchronise with each other
    const int m = (int)(item % a.Mp);
    const int64_t bg = item / a.Mp;
    const int b = (int)(bg / a.G), g = (int)(bg % a.G);

    float sumk[2] = {0.f, 0.f}, sumv[2] = {0.f, 0.f};
    int count = 0;
    if (m < a.M) {
        const T* K = reinterpret_cast<const T*>(a.kg) + b * a.ksb + g * a.ksh;
        const T* Vv = reinterpret_cast<const T*>(a.vg) + b * a.vsb + g * a.vsh;
        const int ppr = D / EP;  // pieces per row
        const int f_end = min(a.F, (m + 1) * a.P);
        for (int f = m * a.P; f < f_end; ++f) {
            const int idx = lane < a.V ? a.blocks[(int64_t)f * a.V + lane] : -1;
            if (__ballot(idx >= 0) == 0) continue;  // empty fine block: no mass, no count
            ++count;
            for (int q = lane; q < 64 * ppr; q += 64) {
                const int s = q / ppr, piece = q - s * ppr;
                const int t = __shfl(idx, s);
                float kx[EP], vx[EP];
                if (t >= 0) {
                    load_piece<T>(K + t * a.ksn + piece * EP, kx);
                    load_piece<T>(Vv + t * a.vsn + piece * EP, vx);
                    int64_t pos[3];
                    rope_position(a.rope, t, pos);
                    rope_apply(a.rope, pos, piece * EP, kx, EP);
                } else {
#pragma unroll
                    for (int e = 0; e < EP; ++e) kx[e] = vx[e] = 0.f;
                }
#pragma unroll
                for (int e = 0; e < EP; ++e) {
                    lk[s * stride + piece * EP + e] = from_f32<T>(kx[e]);
                    lv[s * stride + piece * EP + e] = from_f32<T>(vx[e]);
                }
            }
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
            __builtin_amdgcn_wave_barrier();
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
            // Slot logits (compression.py:31-35): (k . w) / tau + bias_s.
            float logit = -INFINITY;
            if (idx >= 0) {
                float dot = 0.f;
                for (int c = 0; c < D; ++c) dot += to_f32(lk[lane * stride + c]) * a.weight[c];
                logit = dot * a.inv_tau + a.bias[lane];
            }
            const float mx = wave_max(logit);
            const float e = idx >= 0 ? expf(logit - mx) : 0.f;
            const float den = wave_sum(e);
            la[lane] = e / den;
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
            __builtin_amdgcn_wave_barrier();
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                const int c = lane + 64 * h;
                if (c < D) {
                    float fk = 0.f, fv = 0.f;
                    for (int s = 0; s < a.V; ++s) {
                        const float w = la[s];
                        fk += w * to_f32(lk[s * stride + c]);
                        fv += w * to_f32(lv[s * stride + c]);
                    }
                    sumk[h] += fk;
                    sumv[h] += fv;
                }
            }
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
            __builtin_amdgcn_wave_barrier();
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        }
    }
    T* sk = reinterpret_cast<T*>(a.sk) + ((int64_t)bg * a.Mp + m) * D;
    T* svt = reinterpret_cast<T*>(a.svt) + (((int64_t)bg * (a.Mp / 32) + m / 32) * D) * 32 + (m & 31);
    float sq = 0.f;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        const int c = lane + 64 * h;
        if (c < D) {
            // The coarse stage divides the group sum by the count (compression.py:42-43).
            const T kq = from_f32<T>(count ? sumk[h] / (float)count * a.key_scale : 0.f);
            sk[c] = kq;
            svt[c * 32] = from_f32<T>(count ? sumv[h] / (float)count : 0.f);
            sq += to_f32(kq) * to_f32(kq);
        }
    }
    // Norm of the stored (rounded) summary key; non-negative floats order
    // like their bit patterns, so an integer max is an exact float max.
    const float norm = sqrtf(wave_sum(sq)) * (1.f + 1e-6f);
    if (lane == 0 && m < a.M)
        atomicMax(reinterpret_cast<int*>(a.sk_norm_max) + bg * kNormSlots + (m % kNormSlots), __float_as_int(norm));
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

template <typename T>
__global__ void k_rotate(RotDev a) {
    constexpr int EP = Piece<T>::N;
    const int ppr = a.D / EP;
    const int64_t total = (int64_t)a.B * a.H * a.N * ppr;
    const int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (e >= total) return;
    const int piece = (int)(e % ppr);
    const int64_t row = e / ppr;
    const int64_t n = row % a.N;
    const int64_t bh = row / a.N;
    const int64_t b = bh / a.H, h = bh % a.H;
    float x[EP];
    load_piece<T>(reinterpret_cast<const T*>(a.x) + b * a.xsb + h * a.xsh + n * a.xsn + piece * EP, x);
    int64_t pos[3];
    rope_position(a.rope, n, pos);
    rope_apply(a.rope, pos, piece * EP, x, EP, a.inverse != 0);
    T* y = reinterpret_cast<T*>(a.y) + b * a.ysb + h * a.ysh + n * a.ysn + piece * EP;
#pragma unroll
    for (int i = 0; i < EP; ++i) y[i] = from_f32<T>(x[i]);
}

}  // namespace
}  // namespace p3d

using namespace p3d;

extern "C" int p3d_pool_fwd(const p3d_pool_args* args, void* stream) {
    P3D_REQUIRE(args, "null args");
    const p3d_pool_args& a = *args;
    const int es = dtype_size(a.dtype);
    P3D_REQUIRE(a.dtype >= P3D_F32 && a.dtype <= P3D_BF16, "unknown dtype");
    P3D_REQUIRE(a.head_dim >= 2 && a.head_dim <= 128 && a.head_dim % (16 / es) == 0,
                "head_dim must be a multiple of the 16-byte piece and at most 128");
    P3D_REQUIRE(a.slots >= 1 && a.slots <= 64 && a.pool_size >= 1 && a.pool_size <= 32, "bad pooling shape");
    P3D_REQUIRE(a.summaries == (a.fine_blocks + a.pool_size - 1) / a.pool_size, "summaries != ceil(F/P)");
    P3D_REQUIRE(view_ok(a.kg, es) && view_ok(a.vg, es), "kg/vg rows must be 16-byte aligned");
    P3D_REQUIRE(a.sk && a.svt && a.sk_norm_max && a.blocks && a.weight && a.bias && a.rope.table && a.rope.pairs,
                "null pointer argument");
    P3D_REQUIRE(a.rope.packed || a.rope.coords, "rope needs coords unless packed");
    P3D_REQUIRE(a.temperature > 0.f, "temperature must be positive");
    P3D_REQUIRE(a.key_scale > 0.f, "key_scale must be positive");
    PoolDev d{};
    d.B = a.batch;
    d.G = a.kv_heads;
    d.N = a.tokens;
    d.D = a.head_dim;
    d.F = a.fine_blocks;
    d.V = a.slots;
    d.P = a.pool_size;
    d.M = a.summaries;
    d.Mp = (int)cdiv(a.summaries, 32) * 32;
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
    d.sk = a.sk;
    d.svt = a.svt;
    d.sk_norm_max = a.sk_norm_max;
    const int64_t items = (int64_t)d.B * d.G * d.Mp;
    const int ep = 16 / es;
    // Each wave stages 64 rows of K and V; keep a block within 64 KiB of LDS.
    const size_t per_wave = (size_t)2 * 64 * (d.D + ep) * es + 64 * sizeof(float);
    const int waves = (int)std::max<size_t>(1, std::min<size_t>(kPoolWaves, 65536 / per_wave));
    const size_t smem = per_wave * waves;
    const unsigned blocks = (unsigned)cdiv(items, waves);
    hipStream_t s = as_stream(stream);
    const int bgn = a.batch * a.kv_heads * kNormSlots;
    k_zero_f32<<<(unsigned)cdiv(bgn, 256), 256, 0, s>>>(a.sk_norm_max, bgn);
    switch (a.dtype) {
        case P3D_F32: k_pool_fwd<float><<<blocks, 64 * waves, smem, s>>>(d); break;
        case P3D_F16: k_pool_fwd<_Float16><<<blocks, 64 * waves, smem, s>>>(d); break;
        default: k_pool_fwd<__bf16><<<blocks, 64 * waves, smem, s>>>(d); break;
    }
    return check_launch("p3d_pool_fwd");
}

extern "C" int p3d_rotate(p3d_view x, p3d_view y, int32_t batch, int32_t heads, int32_t tokens,
                          int32_t head_dim, int32_t dtype, const p3d_rope* rope, int32_t inverse, void* stream) {
    P3D_REQUIRE(rope && rope->table && rope->pairs && (rope->packed || rope->coords), "bad rope");
    const int es = dtype_size(dtype);
    P3D_REQUIRE(head_dim % (16 / es) == 0 && head_dim % 2 == 0, "head_dim must be a multiple of 16 bytes");
    P3D_REQUIRE(view_ok(x, es) && view_ok(y, es), "rows must be 16-byte aligned");
    RotDev d{};
    d.B = batch, d.H = heads, d.N = tokens, d.D = head_dim, d.inverse = inverse;
    d.x = (const char*)x.data, d.xsb = x.sb, d.xsh = x.sh, d.xsn = x.sn;
    d.y = (char*)y.data, d.ysb = y.sb, d.ysh = y.sh, d.ysn = y.sn;
    d.rope = rope_dev(*rope);
    const int64_t total = (int64_t)batch * heads * tokens * (head_dim / (16 / es));
    const unsigned g = (unsigned)cdiv(total, 256);
    hipStream_t s = as_stream(stream);
    switch (dtype) {
        case P3D_F32: k_rotate<float><<<g, 256, 0, s>>>(d); break;
        case P3D_F16: k_rotate<_Float16><<<g, 256, 0, s>>>(d); break;
        default: k_rotate<__bf16><<<g, 256, 0, s>>>(d); break;
    }
    return check_launch("p3d_rotate");
}
