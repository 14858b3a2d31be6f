// Local pathway backward on MFMA for complete-grid layouts: the VJP of the
// neighbourhood softmax attention (reference.py:23-30 of amilworks/Pack3D;
// the reference GPU backward is kernels.py:130-181 and its stencil variant),
// tiled like the forward grid kernel.
//
// A workgroup owns a 4 x 8 x 8 (z, y, x) brick of one (batch, head) for dQ or
// of one (batch, kv head) for dK / dV.  Eight waves each own a column block
// of 32 brick positions (two z planes of a 4 x 4 y-x quarter).  The halo is
// streamed through LDS plane by plane; per 32-position chunk of a wave's
// 8 x 8 footprint the scores are recomputed on MFMA, P = 2^(s log2(e)/sqrt(d)
// - lse log2(e)) with the saved log-sum-exp, dP on MFMA, dS = P (dP - Delta).
//   dQ kernel (lane = query): planes hold K rows, V rows and K transposed;
//     dQ^T += K^T dS^T.
//   dK/dV kernel (lane = key): planes hold q rows, dO rows, q and dO
//     transposed, lse and Delta of the plane's queries; every query head of
//     the kv group is streamed; dK^T += q^T dS, dV^T += dO^T P.
// The stencil is symmetric on a complete grid, so the key kernel uses the
// same masks with the roles of queries and keys exchanged.  Inputs q and kl
// are already rotated.
#include "attn_common.hpp"

namespace p3d {
namespace {

constexpr int kWaves = 8;
constexpr int kPlane = 12;
constexpr int kPlaneKeys = kPlane * kPlane;
constexpr float kLog2e = 1.4426950408889634f;

struct LbDev {
    int B, H, G, N, Z, Y, X, rz, ry, rx, bricks_y, bricks_x;
    const char *q, *kl, *vl;
    int64_t qsb, qsh, qsn, ksb, ksh, ksn, vsb, vsh, vsn;
    const char* dol;          // [B,H,N,D] contiguous
    const float *lse, *delta;  // [B,H,N]
    const int32_t* map;        // raster -> packed row, or null
    float* dq;                 // [B,H,N,D] fp32
    float* dk;                 // [B,G,N,D] fp32
    char* dv;                  // [B,G,N,D] view, storage type
    int64_t dvsb, dvsh, dvsn;
    float scale_log2, scale;   // log2(e)/sqrt(D), 1/sqrt(D)
};

template <typename T>
__device__ __forceinline__ const T* tp(const char* p) { return reinterpret_cast<const T*>(p); }

__device__ __forceinline__ int64_t packed_row(const LbDev& a, int gz, int gy, int gx) {
    const int64_t raster = ((int64_t)gz * a.Y + gy) * a.X + gx;
    return a.map ? (int64_t)a.map[raster] : raster;
}

// Same brick order as the forward: a contiguous run of bricks per XCD.
__device__ __forceinline__ int xcd_brick(int id, int bricks) {
    const int q = bricks / 8, r = bricks % 8;
    const int xcd = id % 8, slot = id / 8;
    return xcd < r ? xcd * (q + 1) + slot : r * (q + 1) + (xcd - r) * q + slot;
}

// Valid pairs of chunk c among this lane's 16 scores: the (2ry+1) x (2rx+1)
// stencil around the lane's position (py, px) in the wave footprint, with the
// chunk's positions clipped to the grid.  The z condition is per plane.
template <typename C>
__device__ __forceinline__ uint32_t chunk_mask(const LbDev& a, int c, int g, int py, int px, int Yw, int Xw) {
    uint32_t m = 0;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
        const int kr = kperm<C::E, C::KS>(acc_row(r, g));
        const int ky = 4 * c + kr / 8, kx = kr % 8;
        const int gy = Yw - a.ry + ky, gx = Xw - a.rx + kx;
        const bool ok = (unsigned)(ky - py) <= (unsigned)(2 * a.ry) && (unsigned)(kx - px) <= (unsigned)(2 * a.rx) &&
                        (unsigned)gy < (unsigned)a.Y && (unsigned)gx < (unsigned)a.X;
        m |= (ok ? 1u : 0u) << r;
    }
    return m;
}

// Plane position of chunk c's tile row kappa (natural order) in a wave footprint.
__device__ __forceinline__ int chunk_pos(int wy, int wx, int c, int kappa) {
    return (4 * wy + 4 * c + kappa / 8) * kPlane + 4 * wx + kappa % 8;
}

// fp16 score gradients can exceed the type's range (65504) while dQ and dK
// stay finite, e.g. tiny q, k against large v and dO.  In fp16 the dS of a
// query (dQ kernel) or key (dK kernel) enters the MFMA as dS * 2^-shift, with
// shift >= 0 raised, lazily and per lane column, until the largest |dS| seen
// fits below 2^15; the accumulator is rescaled when the shift grows and the
// result multiplied back by 2^shift.  The lane pair (l, l + 32) holds the
// same column, so both take the larger of their maxima.  Other types keep
// shift 0 (bf16 and fp32 have fp32's exponent range).
template <typename C>
__device__ __forceinline__ void fit_fp16(float* ds, int& shift, f32x16* acc) {
    if constexpr (std::is_same<typename C::T_, _Float16>::value) {
        float tmax = 0.f;
#pragma unroll
        for (int r = 0; r < 16; ++r) tmax = fmaxf(tmax, fabsf(ds[r]));
        tmax = fmaxf(tmax, swap_half(tmax));
        int e;
        frexpf(tmax, &e);  // tmax < 2^e
        const int need = e > 15 ? e - 15 : 0;
        if (__builtin_amdgcn_ballot_w64(need > shift)) {
            if (need > shift) {
                const float f = ldexpf(1.f, shift - need);
#pragma unroll
                for (int mb = 0; mb < C::MB; ++mb)
#pragma unroll
                    for (int r = 0; r < 16; ++r) acc[mb][r] *= f;
                shift = need;
            }
        }
        if (shift) {
            const float f = ldexpf(1.f, -shift);
#pragma unroll
            for (int r = 0; r < 16; ++r) ds[r] *= f;
        }
    }
}

// Stage one halo plane of two row tensors: rows (stride KSTR) of both and the
// transposes (stride TPS) of the tensors selected by TRANS_A / TRANS_B.
// Positions outside the grid or the halo are zero.
template <typename C, bool TRANS_A, bool TRANS_B>
__device__ __forceinline__ void stage_plane(const LbDev& a, const typename C::T_* A, int64_t asn,
                                            const typename C::T_* Bt, int64_t bsn, int gz, int Y0, int X0,
                                            typename C::T_* Ar, typename C::T_* Br, typename C::T_* At,
                                            typename C::T_* Btr, int tps) {
    typedef typename C::T_ T;
    constexpr int EP = Piece<T>::N, PPR = C::D / EP;
    constexpr int TASKS = kPlaneKeys * PPR;
    for (int task = threadIdx.x; task < TASKS; task += 64 * kWaves) {
        const int piece = task % PPR, pos = task / PPR;
        const int ky = pos / kPlane, kx = pos - ky * kPlane;
        const int gy = Y0 - a.ry + ky, gx = X0 - a.rx + kx;
        const bool in = (unsigned)gz < (unsigned)a.Z && (unsigned)gy < (unsigned)a.Y && (unsigned)gx < (unsigned)a.X &&
                        ky < 8 + 2 * a.ry && kx < 8 + 2 * a.rx;
        uint4 ra = uint4{0, 0, 0, 0}, rb = uint4{0, 0, 0, 0};
        if (in) {
            const int64_t row = packed_row(a, gz, gy, gx);
            ra = *reinterpret_cast<const uint4*>(A + row * asn + piece * EP);
            rb = *reinterpret_cast<const uint4*>(Bt + row * bsn + piece * EP);
        }
        *reinterpret_cast<uint4*>(Ar + pos * C::KSTR + piece * EP) = ra;
        *reinterpret_cast<uint4*>(Br + pos * C::KSTR + piece * EP) = rb;
        const T* va = reinterpret_cast<const T*>(&ra);
        const T* vb = reinterpret_cast<const T*>(&rb);
#pragma unroll
        for (int e = 0; e < EP; ++e) {
            if (TRANS_A) At[(piece * EP + e) * tps + pos] = va[e];
            if (TRANS_B) Btr[(piece * EP + e) * tps + pos] = vb[e];
        }
    }
}

// Zero rows [D, 32 * MB) of a transposed plane buffer.
template <typename C>
__device__ __forceinline__ void zero_pad_rows(typename C::T_* buf, int tps) {
    const int rows = 32 * C::MB - C::D;
    for (int i = threadIdx.x; i < rows * kPlaneKeys; i += blockDim.x) {
        const int r = i / kPlaneKeys, c = i - r * kPlaneKeys;
        buf[(C::D + r) * tps + c] = from_f32<typename C::T_>(0.f);
    }
}

// Fragments of a row (query or key) for the score MFMAs, no rotation.
template <typename C>
__device__ __forceinline__ void row_frags(const typename C::T_* row, bool valid, int g, typename C::Frag* f) {
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

// A-operand fragments of a transposed plane buffer for chunk c: row 32 mb + qi
// (channel), contraction index ks * KS + E * g + j = chunk position (natural).
template <typename C>
__device__ __forceinline__ void trans_frags(const typename C::T_* Tb, int tps, int wy, int wx, int c, int lane,
                                            typename C::Frag* f) {
    const int g = lane >> 5, qi = lane & 31;
#pragma unroll
    for (int mb = 0; mb < C::MB; ++mb)
#pragma unroll
        for (int ks = 0; ks < C::KSTEPS; ++ks) {
            const int k0 = ks * C::KS + C::E * g;
            f[mb * C::KSTEPS + ks] =
                frag_load8<typename C::T_>(Tb + (32 * mb + qi) * tps + chunk_pos(wy, wx, c, k0));
        }
}

// dQ^T += K^T dS^T for chunk c of one plane: kf / vf are the chunk's K and V
// row fragments (lane = key of the tile), tf the K^T fragments (A operand).
template <typename C>
__device__ __forceinline__ void dq_chunk(const typename C::Frag* kf, const typename C::Frag* vf,
                                         const typename C::Frag* tf, const typename C::Frag* qf,
                                         const typename C::Frag* df, bool zok, uint32_t kmask, float scale_log2,
                                         float lse2, float delta, int& shift, f32x16* acc) {
    typedef typename C::T_ T;
    const f32x16 s = score_tile<C>(kf, qf);
    const f32x16 dp = score_tile<C>(vf, df);
    float ds[16];
#pragma unroll
    for (int r = 0; r < 16; ++r) {
        const bool ok = zok && ((kmask >> r) & 1);
        ds[r] = ok ? __builtin_amdgcn_exp2f(fmaf(s[r], scale_log2, -lse2)) * (dp[r] - delta) : 0.f;
    }
    fit_fp16<C>(ds, shift, acc);
#pragma unroll
    for (int ks = 0; ks < C::KSTEPS; ++ks) {
        const typename C::Frag pf = frag_from_p<T>(ds, ks);
#pragma unroll
        for (int mb = 0; mb < C::MB; ++mb) acc[mb] = C::M::mfma(tf[mb * C::KSTEPS + ks], pf, acc[mb]);
    }
}

// dK^T += q^T dS and dV^T += dO^T P for chunk c of one plane: qa / da are the
// chunk's q and dO row fragments (lane = query of the tile), qt / dt the
// transposed fragments (A operands); lse2s / dlts hold the plane's lse (log2
// units, +inf where a position has no gradient) and Delta.
template <typename C>
__device__ __forceinline__ void dkv_chunk(const typename C::Frag* qa, const typename C::Frag* da,
                                          const typename C::Frag* qt, const typename C::Frag* dt,
                                          const typename C::Frag* kf, const typename C::Frag* vf, bool zok,
                                          uint32_t qmask, float scale_log2, const float* lse2s, const float* dlts,
                                          int wy, int wx, int c, int g, int& shift, f32x16* acck, f32x16* accv) {
    typedef typename C::T_ T;
    const f32x16 s = score_tile<C>(qa, kf);
    const f32x16 dp = score_tile<C>(da, vf);
    float p[16], ds[16];
#pragma unroll
    for (int r = 0; r < 16; ++r) {
        const int pos = chunk_pos(wy, wx, c, kperm<C::E, C::KS>(acc_row(r, g)));
        const bool ok = zok && ((qmask >> r) & 1);
        p[r] = ok ? __builtin_amdgcn_exp2f(fmaf(s[r], scale_log2, -lse2s[pos])) : 0.f;
        ds[r] = p[r] * (dp[r] - dlts[pos]);
    }
    fit_fp16<C>(ds, shift, acck);
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

// Halo planes by the LDS DMA (16-bit types, head_dim <= 64).  Each plane's
// rows of two tensors (K and V for dQ, q and dO for dK / dV) are copied into
// one of two plane buffers while the previous plane is processed, in the
// row-major layout of the register-staged kernels (row stride KSTR: D / 8
// 16-byte slots and one spare, whose lanes fetch piece 0 of the same row
// again).  The transposed A operands are read from those rows with
// ds_read_b64_tr_b16, so nothing is staged transposed.  The packed row of
// every halo position of the brick is looked up once into a table in LDS;
// positions outside the grid take the row of the nearest grid position
// (finite values, excluded by the stencil masks).  SIDE: each buffer also
// holds the plane's lse (log2 units) and Delta, written from registers.
template <typename C>
constexpr bool kBwdPlaneDma = sizeof(typename C::T_) == 2 && C::D <= 64;

template <typename C, bool SIDE>
struct BwdPlaneDma {
    typedef typename C::T_ T;
    typedef typename C::Frag Frag;
    static constexpr int EP = Piece<T>::N;
    static constexpr int KROW = C::KSTR / EP;            // 16-byte slots per row
    static constexpr int SLOTS = kPlaneKeys * KROW;      // slots of one tensor's plane
    static constexpr int CH = (SLOTS + 63) / 64;         // copies per tensor
    static constexpr int PER = (2 * CH + kWaves - 1) / kWaves;
    static constexpr size_t REGION = (size_t)SLOTS * 16;
    static constexpr size_t BUF = 2 * REGION + (SIDE ? 2 * kPlaneKeys * sizeof(float) : 0);
    static constexpr int kMaxPlanes = 8;                 // 4 + 2 rz with rz <= 2
    static constexpr size_t BYTES = 2 * BUF + (size_t)kMaxPlanes * kPlaneKeys * sizeof(int);
    static_assert(C::KSTR % EP == 0 && C::KSTR > C::D, "rows need a spare slot");
    // The copies address LDS through M0; the buffers stay inside the first
    // 128 KB of the workgroup's allocation.
    static_assert(2 * BUF <= 128 * 1024, "copy destinations below 128 KB");

    // Packed rows of the halo positions of planes [0, planes) (z from Z0 - rz).
    __device__ __forceinline__ static void fill_rows(const LbDev& a, int Z0, int Y0, int X0, int planes, int* rows) {
        for (int i = threadIdx.x; i < planes * kPlaneKeys; i += blockDim.x) {
            const int hz = i / kPlaneKeys, k = i - hz * kPlaneKeys, ky = k / kPlane, kx = k - ky * kPlane;
            const int gz = min(max(Z0 - a.rz + hz, 0), a.Z - 1);
            const int gy = min(max(Y0 - a.ry + ky, 0), a.Y - 1);
            const int gx = min(max(X0 - a.rx + kx, 0), a.X - 1);
            rows[i] = (int)packed_row(a, gz, gy, gx);
        }
    }

    // Issue the copies of one plane (its rows at `rows`): rows of A into the
    // first region of `buf`, rows of B into the second.
    __device__ __forceinline__ static void copy(const T* A, int64_t asn, const T* B, int64_t bsn, const int* rows,
                                                unsigned char* buf, int wave, int lane) {
        const uint32_t lds0 = lds_address(buf);
#pragma unroll
        for (int i = 0; i < PER; ++i) {
            const int c = min(wave * PER + i, 2 * CH - 1);  // wave-uniform
            const bool second = c >= CH;
            const int first = min(64 * (second ? c - CH : c), SLOTS - 64);
            const int slot = first + lane, key = slot / KROW, sl = slot - key * KROW;
            const int64_t row = rows[key];
            const int e = (sl < C::D / EP ? sl : 0) * EP;
            const T* src = second ? B + row * bsn + e : A + row * asn + e;
            dma_copy16(src, lds0 + (second ? (uint32_t)REGION : 0u) + (uint32_t)first * 16u);
        }
    }

    // A-operand fragment of block mb / k-step of a chunk from plane rows:
    // lane l holds channel 32 mb + l % 32 of the rows row0 .. row0 + 7
    // (consecutive in x); channels past D are zero.
    __device__ __forceinline__ static Frag tfrag(const T* rows, int row0, int mb, int lane) {
        Frag f = tr_frag<T, Frag>(rows, row0, C::KSTR, 32 * mb, C::D - 16, lane);
        if (32 * mb + 16 >= C::D && 32 * mb + 16 * ((lane >> 4) & 1) >= C::D) f = frag_fill<T>(0.f);
        return f;
    }

    __device__ __forceinline__ static void tfrags(const T* rows, int wy, int wx, int c, int lane, Frag* f) {
        const int g = lane >> 5;
#pragma unroll
        for (int mb = 0; mb < C::MB; ++mb)
#pragma unroll
            for (int ks = 0; ks < C::KSTEPS; ++ks)
                f[mb * C::KSTEPS + ks] = tfrag(rows, chunk_pos(wy, wx, c, ks * C::KS + C::E * g), mb, lane);
    }
};

template <typename T, int D>
__global__ __launch_bounds__(64 * kWaves) void k_local_dq_grid(LbDev a) {
    typedef Cfg<T, D> C;
    constexpr int EP = Piece<T>::N;
    constexpr int TPS = kPlaneKeys + EP;
    extern __shared__ __align__(16) unsigned char smem[];
    T* Kr = reinterpret_cast<T*>(smem);
    T* Vr = Kr + kPlaneKeys * C::KSTR;
    T* Kt = Vr + kPlaneKeys * C::KSTR;

    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, g = lane >> 5, qi = lane & 31;
    const int bh = blockIdx.y, b = bh / a.H, h = bh % a.H, kvh = h / (a.H / a.G);
    const int brick = xcd_brick(blockIdx.x, gridDim.x);
    const int Z0 = 4 * (brick / (a.bricks_y * a.bricks_x));
    const int Y0 = 8 * ((brick / a.bricks_x) % a.bricks_y);
    const int X0 = 8 * (brick % a.bricks_x);
    const int nb = wave >> 2, wy = (wave >> 1) & 1, wx = wave & 1;
    const int qy = (qi >> 2) & 3, qx = qi & 3;
    const int qz = 2 * nb + (qi >> 4);

    const int gz = Z0 + qz, gy = Y0 + 4 * wy + qy, gx = X0 + 4 * wx + qx;
    const bool qok = gz < a.Z && gy < a.Y && gx < a.X;
    const int64_t qrow = qok ? packed_row(a, gz, gy, gx) : 0;
    const int64_t qidx = (int64_t)bh * a.N + qrow;
    typename C::Frag qf[C::NT], df[C::NT];
    row_frags<C>(tp<T>(a.q) + b * a.qsb + h * a.qsh + qrow * a.qsn, qok, g, qf);
    row_frags<C>(tp<T>(a.dol) + qidx * D, qok, g, df);
    const float lse = qok ? a.lse[qidx] : -INFINITY;
    const bool live = lse != -INFINITY;  // an all-masked row has no local gradient
    const float lse2 = live ? lse * kLog2e : 0.f;
    const float delta = qok ? a.delta[qidx] : 0.f;
    f32x16 acc[C::MB];
#pragma unroll
    for (int mb = 0; mb < C::MB; ++mb)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[mb][r] = 0.f;
    int shift = 0;

    const T* KL = tp<T>(a.kl) + b * a.ksb + kvh * a.ksh;
    const T* VL = tp<T>(a.vl) + b * a.vsb + kvh * a.vsh;
    const uint32_t kmask[2] = {chunk_mask<C>(a, 0, g, qy, qx, Y0 + 4 * wy, X0 + 4 * wx),
                               chunk_mask<C>(a, 1, g, qy, qx, Y0 + 4 * wy, X0 + 4 * wx)};
    zero_pad_rows<C>(Kt, TPS);
    const int planes = 4 + 2 * a.rz;
    for (int hz = 0; hz < planes; ++hz) {
        const int pz = Z0 - a.rz + hz;
        if (hz) __syncthreads();
        stage_plane<C, true, false>(a, KL, a.ksn, VL, a.vsn, pz, Y0, X0, Kr, Vr, Kt, nullptr, TPS);
        __syncthreads();
        if ((unsigned)pz >= (unsigned)a.Z) continue;
        // Column block nb holds query planes 2nb and 2nb + 1.
        if (hz < 2 * nb || hz > 2 * nb + 1 + 2 * a.rz) continue;
        const bool zok = (unsigned)(hz - qz) <= (unsigned)(2 * a.rz) && live;
#pragma unroll
        for (int c = 0; c < 2; ++c) {
            if (4 * c >= 4 + 2 * a.ry) continue;
            const int kap = kperm<C::E, C::KS>(qi);
            typename C::Frag kf[C::NT], vf[C::NT], tf[C::MB * C::KSTEPS];
            load_kfrags<C>(Kr + chunk_pos(wy, wx, c, kap) * C::KSTR + C::E * g, kf);
            load_kfrags<C>(Vr + chunk_pos(wy, wx, c, kap) * C::KSTR + C::E * g, vf);
            trans_frags<C>(Kt, TPS, wy, wx, c, lane, tf);
            dq_chunk<C>(kf, vf, tf, qf, df, zok, kmask[c], a.scale_log2, lse2, delta, shift, acc);
        }
    }
    if (!qok) return;
    float* dq = a.dq + qidx * D;
    const float out_scale = ldexpf(a.scale, shift);
#pragma unroll
    for (int mb = 0; mb < C::MB; ++mb)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const int c = 32 * mb + acc_row(r, g);
            if (c < D) dq[c] = acc[mb][r] * out_scale;
        }
}

// k_local_dq_grid with the planes copied by the LDS DMA (kBwdPlaneDma types).
template <typename T, int D>
__global__ __launch_bounds__(64 * kWaves) void k_local_dq_grid_dma(LbDev a) {
    typedef Cfg<T, D> C;
    typedef BwdPlaneDma<C, false> PD;
    extern __shared__ __align__(16) unsigned char smem[];
    int* const rowtab = reinterpret_cast<int*>(smem + 2 * PD::BUF);

    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, g = lane >> 5, qi = lane & 31;
    const int bh = blockIdx.y, b = bh / a.H, h = bh % a.H, kvh = h / (a.H / a.G);
    const int brick = xcd_brick(blockIdx.x, gridDim.x);
    const int Z0 = 4 * (brick / (a.bricks_y * a.bricks_x));
    const int Y0 = 8 * ((brick / a.bricks_x) % a.bricks_y);
    const int X0 = 8 * (brick % a.bricks_x);
    const int nb = wave >> 2, wy = (wave >> 1) & 1, wx = wave & 1;
    const int qy = (qi >> 2) & 3, qx = qi & 3;
    const int qz = 2 * nb + (qi >> 4);
    const int planes = 4 + 2 * a.rz;
    const T* KL = tp<T>(a.kl) + b * a.ksb + kvh * a.ksh;
    const T* VL = tp<T>(a.vl) + b * a.vsb + kvh * a.vsh;
    PD::fill_rows(a, Z0, Y0, X0, planes, rowtab);
    __syncthreads();
    const int uwave = __builtin_amdgcn_readfirstlane(wave);
    if ((unsigned)(Z0 - a.rz) < (unsigned)a.Z) PD::copy(KL, a.ksn, VL, a.vsn, rowtab, smem, uwave, lane);

    const int gz = Z0 + qz, gy = Y0 + 4 * wy + qy, gx = X0 + 4 * wx + qx;
    const bool qok = gz < a.Z && gy < a.Y && gx < a.X;
    const int64_t qrow = qok ? packed_row(a, gz, gy, gx) : 0;
    const int64_t qidx = (int64_t)bh * a.N + qrow;
    typename C::Frag qf[C::NT], df[C::NT];
    row_frags<C>(tp<T>(a.q) + b * a.qsb + h * a.qsh + qrow * a.qsn, qok, g, qf);
    row_frags<C>(tp<T>(a.dol) + qidx * D, qok, g, df);
    const float lse = qok ? a.lse[qidx] : -INFINITY;
    const bool live = lse != -INFINITY;  // an all-masked row has no local gradient
    const float lse2 = live ? lse * kLog2e : 0.f;
    const float delta = qok ? a.delta[qidx] : 0.f;
    f32x16 acc[C::MB];
#pragma unroll
    for (int mb = 0; mb < C::MB; ++mb)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[mb][r] = 0.f;
    int shift = 0;
    const uint32_t kmask[2] = {chunk_mask<C>(a, 0, g, qy, qx, Y0 + 4 * wy, X0 + 4 * wx),
                               chunk_mask<C>(a, 1, g, qy, qx, Y0 + 4 * wy, X0 + 4 * wx)};
    for (int hz = 0; hz < planes; ++hz) {
        const int pz = Z0 - a.rz + hz;
        // Plane hz has landed, and every wave is done with plane hz - 1,
        // whose buffer takes the copy of plane hz + 1.
        dma_wait();
        __syncthreads();
        if (hz + 1 < planes && (unsigned)(pz + 1) < (unsigned)a.Z)
            PD::copy(KL, a.ksn, VL, a.vsn, rowtab + (hz + 1) * kPlaneKeys, smem + ((hz + 1) & 1) * PD::BUF, uwave,
                     lane);
        if ((unsigned)pz >= (unsigned)a.Z) continue;
        // Column block nb holds query planes 2nb and 2nb + 1.
        if (hz < 2 * nb || hz > 2 * nb + 1 + 2 * a.rz) continue;
        const T* Kb = reinterpret_cast<const T*>(smem + (hz & 1) * PD::BUF);
        const T* Vb = reinterpret_cast<const T*>(smem + (hz & 1) * PD::BUF + PD::REGION);
        const bool zok = (unsigned)(hz - qz) <= (unsigned)(2 * a.rz) && live;
#pragma unroll
        for (int c = 0; c < 2; ++c) {
            if (4 * c >= 4 + 2 * a.ry) continue;
            const int kap = kperm<C::E, C::KS>(qi);
            typename C::Frag kf[C::NT], vf[C::NT], tf[C::MB * C::KSTEPS];
            load_kfrags<C>(Kb + chunk_pos(wy, wx, c, kap) * C::KSTR + C::E * g, kf);
            load_kfrags<C>(Vb + chunk_pos(wy, wx, c, kap) * C::KSTR + C::E * g, vf);
            PD::tfrags(Kb, wy, wx, c, lane, tf);
            dq_chunk<C>(kf, vf, tf, qf, df, zok, kmask[c], a.scale_log2, lse2, delta, shift, acc);
        }
    }
    if (!qok) return;
    float* dq = a.dq + qidx * D;
    const float out_scale = ldexpf(a.scale, shift);
#pragma unroll
    for (int mb = 0; mb < C::MB; ++mb)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const int c = 32 * mb + acc_row(r, g);
            if (c < D) dq[c] = acc[mb][r] * out_scale;
        }
}

// lse (log2 units; +inf where the position has no gradient: outside the grid
// or the halo, or an all-masked row) and Delta of halo position p of plane
// pz for query head plane bh; rows: that plane's row table.
__device__ __forceinline__ void plane_side(const LbDev& a, int64_t bh, int pz, int Y0, int X0, int p,
                                           const int* rows, float& l2, float& dl) {
    const int py = p / kPlane, px = p - py * kPlane;
    const int qy = Y0 - a.ry + py, qx = X0 - a.rx + px;
    const bool in = (unsigned)pz < (unsigned)a.Z && (unsigned)qy < (unsigned)a.Y && (unsigned)qx < (unsigned)a.X &&
                    py < 8 + 2 * a.ry && px < 8 + 2 * a.rx;
    l2 = INFINITY, dl = 0.f;
    if (in) {
        const int64_t qidx = bh * a.N + rows[p];
        const float l = a.lse[qidx];
        l2 = l == -INFINITY ? INFINITY : l * kLog2e;  // all-masked rows carry no gradient
        dl = a.delta[qidx];
    }
}

template <typename T, int D>
__global__ __launch_bounds__(64 * kWaves) void k_local_dkv_grid(LbDev a) {
    typedef Cfg<T, D> C;
    constexpr int EP = Piece<T>::N;
    constexpr int TPS = kPlaneKeys + EP;
    extern __shared__ __align__(16) unsigned char smem[];
    T* Qr = reinterpret_cast<T*>(smem);
    T* Dr = Qr + kPlaneKeys * C::KSTR;
    T* Qt = Dr + kPlaneKeys * C::KSTR;
    T* Dt = Qt + 32 * C::MB * TPS;
    float* lse2s = reinterpret_cast<float*>(Dt + 32 * C::MB * TPS);
    float* dlts = lse2s + kPlaneKeys;

    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, g = lane >> 5, ki = lane & 31;
    const int bg = blockIdx.y, b = bg / a.G, kvh = bg % a.G, rep = a.H / a.G;
    const int brick = xcd_brick(blockIdx.x, gridDim.x);
    const int Z0 = 4 * (brick / (a.bricks_y * a.bricks_x));
    const int Y0 = 8 * ((brick / a.bricks_x) % a.bricks_y);
    const int X0 = 8 * (brick % a.bricks_x);
    const int nb = wave >> 2, wy = (wave >> 1) & 1, wx = wave & 1;
    const int ky = (ki >> 2) & 3, kx = ki & 3;
    const int kz = 2 * nb + (ki >> 4);

    const int gz = Z0 + kz, gy = Y0 + 4 * wy + ky, gx = X0 + 4 * wx + kx;
    const bool kok = gz < a.Z && gy < a.Y && gx < a.X;
    const int64_t krow = kok ? packed_row(a, gz, gy, gx) : 0;
    typename C::Frag kf[C::NT], vf[C::NT];
    row_frags<C>(tp<T>(a.kl) + b * a.ksb + kvh * a.ksh + krow * a.ksn, kok, g, kf);
    row_frags<C>(tp<T>(a.vl) + b * a.vsb + kvh * a.vsh + krow * a.vsn, kok, g, vf);
    f32x16 acck[C::MB], accv[C::MB];
#pragma unroll
    for (int mb = 0; mb < C::MB; ++mb)
#pragma unroll
        for (int r = 0; r < 16; ++r) acck[mb][r] = accv[mb][r] = 0.f;
    int shift = 0;

    const uint32_t qmask[2] = {chunk_mask<C>(a, 0, g, ky, kx, Y0 + 4 * wy, X0 + 4 * wx),
                               chunk_mask<C>(a, 1, g, ky, kx, Y0 + 4 * wy, X0 + 4 * wx)};
    zero_pad_rows<C>(Qt, TPS);
    zero_pad_rows<C>(Dt, TPS);
    const int planes = 4 + 2 * a.rz;
    for (int hh = 0; hh < rep; ++hh) {
        const int h = kvh * rep + hh;
        const int64_t bh = (int64_t)b * a.H + h;
        const T* Q = tp<T>(a.q) + b * a.qsb + h * a.qsh;
        const T* DO = tp<T>(a.dol) + bh * a.N * D;
        for (int hz = 0; hz < planes; ++hz) {
            const int pz = Z0 - a.rz + hz;
            __syncthreads();
            stage_plane<C, true, true>(a, Q, a.qsn, DO, D, pz, Y0, X0, Qr, Dr, Qt, Dt, TPS);
            for (int p = tid; p < kPlaneKeys; p += 64 * kWaves) {
                const int py = p / kPlane, px = p - py * kPlane;
                const int qy = Y0 - a.ry + py, qx = X0 - a.rx + px;
                const bool in = (unsigned)pz < (unsigned)a.Z && (unsigned)qy < (unsigned)a.Y &&
                                (unsigned)qx < (unsigned)a.X && py < 8 + 2 * a.ry && px < 8 + 2 * a.rx;
                float l2 = INFINITY, dl = 0.f;
                if (in) {
                    const int64_t qidx = bh * a.N + packed_row(a, pz, qy, qx);
                    const float l = a.lse[qidx];
                    l2 = l == -INFINITY ? INFINITY : l * kLog2e;  // all-masked rows carry no gradient
                    dl = a.delta[qidx];
                }
                lse2s[p] = l2;
                dlts[p] = dl;
            }
            __syncthreads();
            if ((unsigned)pz >= (unsigned)a.Z) continue;
            if (hz < 2 * nb || hz > 2 * nb + 1 + 2 * a.rz) continue;
            const bool zok = (unsigned)(hz - kz) <= (unsigned)(2 * a.rz);
#pragma unroll
            for (int c = 0; c < 2; ++c) {
                if (4 * c >= 4 + 2 * a.ry) continue;
                const int kap = kperm<C::E, C::KS>(ki);
                typename C::Frag qa[C::NT], da[C::NT], qt[C::MB * C::KSTEPS], dt[C::MB * C::KSTEPS];
                load_kfrags<C>(Qr + chunk_pos(wy, wx, c, kap) * C::KSTR + C::E * g, qa);
                load_kfrags<C>(Dr + chunk_pos(wy, wx, c, kap) * C::KSTR + C::E * g, da);
                trans_frags<C>(Qt, TPS, wy, wx, c, lane, qt);
                trans_frags<C>(Dt, TPS, wy, wx, c, lane, dt);
                dkv_chunk<C>(qa, da, qt, dt, kf, vf, zok, qmask[c], a.scale_log2, lse2s, dlts, wy, wx, c, g, shift,
                             acck, accv);
            }
        }
    }
    if (!kok) return;
    const int64_t kidx = (int64_t)bg * a.N + krow;
    float* dk = a.dk + kidx * D;
    T* dv = reinterpret_cast<T*>(a.dv) + b * a.dvsb + kvh * a.dvsh + (int64_t)krow * a.dvsn;
    const float out_scale = ldexpf(a.scale, shift);
#pragma unroll
    for (int mb = 0; mb < C::MB; ++mb)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const int c = 32 * mb + acc_row(r, g);
            if (c < D) {
                dk[c] = acck[mb][r] * out_scale;
                dv[c] = from_f32<T>(accv[mb][r]);
            }
        }
}

// k_local_dkv_grid with the planes copied by the LDS DMA (kBwdPlaneDma types).
// The (query head, plane) steps of the kv group run as one sequence; a
// step's lse / Delta are loaded into registers while the step before it is
// processed and written into its buffer after that.
template <typename T, int D>
__global__ __launch_bounds__(64 * kWaves) void k_local_dkv_grid_dma(LbDev a) {
    typedef Cfg<T, D> C;
    typedef BwdPlaneDma<C, true> PD;
    extern __shared__ __align__(16) unsigned char smem[];
    int* const rowtab = reinterpret_cast<int*>(smem + 2 * PD::BUF);

    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, g = lane >> 5, ki = lane & 31;
    const int bg = blockIdx.y, b = bg / a.G, kvh = bg % a.G, rep = a.H / a.G;
    const int brick = xcd_brick(blockIdx.x, gridDim.x);
    const int Z0 = 4 * (brick / (a.bricks_y * a.bricks_x));
    const int Y0 = 8 * ((brick / a.bricks_x) % a.bricks_y);
    const int X0 = 8 * (brick % a.bricks_x);
    const int nb = wave >> 2, wy = (wave >> 1) & 1, wx = wave & 1;
    const int ky = (ki >> 2) & 3, kx = ki & 3;
    const int kz = 2 * nb + (ki >> 4);
    const int planes = 4 + 2 * a.rz;
    const int steps = rep * planes;
    PD::fill_rows(a, Z0, Y0, X0, planes, rowtab);
    __syncthreads();
    const int uwave = __builtin_amdgcn_readfirstlane(wave);
    const int h0 = kvh * rep;
    // Step i: query head h0 + i / planes, plane i % planes.
    auto copy_step = [&](int i) __attribute__((always_inline)) {
        const int hh = i / planes, hz = i - hh * planes;
        if ((unsigned)(Z0 - a.rz + hz) >= (unsigned)a.Z) return;
        const int h = h0 + hh;
        PD::copy(tp<T>(a.q) + b * a.qsb + h * a.qsh, a.qsn, tp<T>(a.dol) + ((int64_t)b * a.H + h) * a.N * D, D,
                 rowtab + hz * kPlaneKeys, smem + (i & 1) * PD::BUF, uwave, lane);
    };
    auto side_step = [&](int i, float& l2, float& dl) __attribute__((always_inline)) {
        const int hh = i / planes, hz = i - hh * planes;
        l2 = INFINITY, dl = 0.f;
        if (tid < kPlaneKeys)
            plane_side(a, (int64_t)b * a.H + h0 + hh, Z0 - a.rz + hz, Y0, X0, tid, rowtab + hz * kPlaneKeys, l2, dl);
    };
    auto side_store = [&](int i, float l2, float dl) __attribute__((always_inline)) {
        if (tid < kPlaneKeys) {
            float* side = reinterpret_cast<float*>(smem + (i & 1) * PD::BUF + 2 * PD::REGION);
            side[tid] = l2;
            side[kPlaneKeys + tid] = dl;
        }
    };
    {
        float l2, dl;
        side_step(0, l2, dl);
        copy_step(0);
        side_store(0, l2, dl);
    }

    const int gz = Z0 + kz, gy = Y0 + 4 * wy + ky, gx = X0 + 4 * wx + kx;
    const bool kok = gz < a.Z && gy < a.Y && gx < a.X;
    const int64_t krow = kok ? packed_row(a, gz, gy, gx) : 0;
    typename C::Frag kf[C::NT], vf[C::NT];
    row_frags<C>(tp<T>(a.kl) + b * a.ksb + kvh * a.ksh + krow * a.ksn, kok, g, kf);
    row_frags<C>(tp<T>(a.vl) + b * a.vsb + kvh * a.vsh + krow * a.vsn, kok, g, vf);
    f32x16 acck[C::MB], accv[C::MB];
#pragma unroll
    for (int mb = 0; mb < C::MB; ++mb)
#pragma unroll
        for (int r = 0; r < 16; ++r) acck[mb][r] = accv[mb][r] = 0.f;
    int shift = 0;
    const uint32_t qmask[2] = {chunk_mask<C>(a, 0, g, ky, kx, Y0 + 4 * wy, X0 + 4 * wx),
                               chunk_mask<C>(a, 1, g, ky, kx, Y0 + 4 * wy, X0 + 4 * wx)};
    for (int i = 0; i < steps; ++i) {
        const int hz = i % planes;
        const int pz = Z0 - a.rz + hz;
        // Step i's copies and side values have landed, and every wave is done
        // with step i - 1, whose buffer takes step i + 1.
        dma_wait();
        __syncthreads();
        const bool more = i + 1 < steps;
        float l2n = INFINITY, dln = 0.f;
        if (more) {
            side_step(i + 1, l2n, dln);
            copy_step(i + 1);
        }
        if ((unsigned)pz < (unsigned)a.Z && hz >= 2 * nb && hz <= 2 * nb + 1 + 2 * a.rz) {
            const unsigned char* buf = smem + (i & 1) * PD::BUF;
            const T* Qb = reinterpret_cast<const T*>(buf);
            const T* Db = reinterpret_cast<const T*>(buf + PD::REGION);
            const float* lse2s = reinterpret_cast<const float*>(buf + 2 * PD::REGION);
            const float* dlts = lse2s + kPlaneKeys;
            const bool zok = (unsigned)(hz - kz) <= (unsigned)(2 * a.rz);
#pragma unroll
            for (int c = 0; c < 2; ++c) {
                if (4 * c >= 4 + 2 * a.ry) continue;
                const int kap = kperm<C::E, C::KS>(ki);
                typename C::Frag qa[C::NT], da[C::NT], qt[C::MB * C::KSTEPS], dt[C::MB * C::KSTEPS];
                load_kfrags<C>(Qb + chunk_pos(wy, wx, c, kap) * C::KSTR + C::E * g, qa);
                load_kfrags<C>(Db + chunk_pos(wy, wx, c, kap) * C::KSTR + C::E * g, da);
                PD::tfrags(Qb, wy, wx, c, lane, qt);
                PD::tfrags(Db, wy, wx, c, lane, dt);
                dkv_chunk<C>(qa, da, qt, dt, kf, vf, zok, qmask[c], a.scale_log2, lse2s, dlts, wy, wx, c, g, shift,
                             acck, accv);
            }
        }
        if (more) side_store(i + 1, l2n, dln);
    }
    if (!kok) return;
    const int64_t kidx = (int64_t)bg * a.N + krow;
    float* dk = a.dk + kidx * D;
    T* dv = reinterpret_cast<T*>(a.dv) + b * a.dvsb + kvh * a.dvsh + (int64_t)krow * a.dvsn;
    const float out_scale = ldexpf(a.scale, shift);
#pragma unroll
    for (int mb = 0; mb < C::MB; ++mb)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const int c = 32 * mb + acc_row(r, g);
            if (c < D) {
                dk[c] = acck[mb][r] * out_scale;
                dv[c] = from_f32<T>(accv[mb][r]);
            }
        }
}

template <typename T, int D>
size_t lds_dq_grid() {
    typedef Cfg<T, D> C;
    return ((size_t)2 * kPlaneKeys * C::KSTR + (size_t)32 * C::MB * (kPlaneKeys + Piece<T>::N)) * sizeof(T);
}

template <typename T, int D>
size_t lds_dkv_grid() {
    typedef Cfg<T, D> C;
    return ((size_t)2 * kPlaneKeys * C::KSTR + (size_t)2 * 32 * C::MB * (kPlaneKeys + Piece<T>::N)) * sizeof(T) +
           (size_t)2 * kPlaneKeys * sizeof(float);
}

template <typename T, int D>
int launch_t(const LbDev& d, hipStream_t s) {
    typedef Cfg<T, D> C;
    const int bricks = (int)(cdiv(d.Z, 4) * d.bricks_y * d.bricks_x);
    if constexpr (kBwdPlaneDma<C>) {
        constexpr size_t l1 = BwdPlaneDma<C, false>::BYTES, l2 = BwdPlaneDma<C, true>::BYTES;
        static_assert(l1 <= 160 * 1024 && l2 <= 160 * 1024, "plane buffers within LDS");
        k_local_dq_grid_dma<T, D><<<dim3(bricks, d.B * d.H), 64 * kWaves, l1, s>>>(d);
        k_local_dkv_grid_dma<T, D><<<dim3(bricks, d.B * d.G), 64 * kWaves, l2, s>>>(d);
    } else {
        const size_t l1 = lds_dq_grid<T, D>(), l2 = lds_dkv_grid<T, D>();
        if (l1 > 160 * 1024 || l2 > 160 * 1024) return fail(P3D_EUNSUPPORTED, "p3d_local_bwd_grid: planes exceed LDS");
        k_local_dq_grid<T, D><<<dim3(bricks, d.B * d.H), 64 * kWaves, l1, s>>>(d);
        k_local_dkv_grid<T, D><<<dim3(bricks, d.B * d.G), 64 * kWaves, l2, s>>>(d);
    }
    return P3D_OK;
}

template <int D>
int launch_d(const LbDev& d, int dtype, hipStream_t s) {
    switch (dtype) {
        case P3D_F32: return launch_t<float, D>(d, s);
        case P3D_F16: return launch_t<_Float16, D>(d, s);
        default: return launch_t<__bf16, D>(d, s);
    }
}

}  // namespace
}  // namespace p3d

using namespace p3d;

extern "C" int p3d_local_bwd_grid(const p3d_bwd_args* args, const int32_t grid[3], const int32_t radius[3],
                                  const int32_t* raster_to_packed, void* stream) {
    P3D_REQUIRE(args && grid && radius, "null argument");
    const p3d_bwd_args& x = *args;
    const int es = dtype_size(x.dtype);
    P3D_REQUIRE(x.dtype >= P3D_F32 && x.dtype <= P3D_BF16, "unknown dtype");
    P3D_REQUIRE(x.head_dim == 16 || x.head_dim == 32 || x.head_dim == 48 || x.head_dim == 64 || x.head_dim == 128,
                "head_dim must be 16, 32, 48, 64 or 128");
    P3D_REQUIRE(x.batch >= 1 && x.heads >= 1 && x.kv_heads >= 1 && x.heads % x.kv_heads == 0, "bad head counts");
    P3D_REQUIRE(grid[0] >= 1 && grid[1] >= 1 && grid[2] >= 1 &&
                    (int64_t)grid[0] * grid[1] * grid[2] == (int64_t)x.tokens,
                "grid must cover the tokens");
    P3D_REQUIRE(radius[0] >= 0 && radius[0] <= 2 && radius[1] >= 0 && radius[1] <= 2 && radius[2] >= 0 &&
                    radius[2] <= 2,
                "grid radius must be 0..2 per axis");
    P3D_REQUIRE(view_ok(x.q, es) && view_ok(x.kl, es) && view_ok(x.vl, es), "q/k/v rows must be 16-byte aligned");
    P3D_REQUIRE(x.dol && x.lse_local && x.delta_local && x.dq_local && x.dk_local && view_ok(x.dv_local, es),
                "null pointer argument");
    LbDev d{};
    d.B = x.batch, d.H = x.heads, d.G = x.kv_heads, d.N = x.tokens;
    d.Z = grid[0], d.Y = grid[1], d.X = grid[2];
    d.rz = radius[0], d.ry = radius[1], d.rx = radius[2];
    d.bricks_y = (int)cdiv(d.Y, 8), d.bricks_x = (int)cdiv(d.X, 8);
    d.q = (const char*)x.q.data, d.qsb = x.q.sb, d.qsh = x.q.sh, d.qsn = x.q.sn;
    d.kl = (const char*)x.kl.data, d.ksb = x.kl.sb, d.ksh = x.kl.sh, d.ksn = x.kl.sn;
    d.vl = (const char*)x.vl.data, d.vsb = x.vl.sb, d.vsh = x.vl.sh, d.vsn = x.vl.sn;
    d.dol = (const char*)x.dol;
    d.lse = x.lse_local, d.delta = x.delta_local;
    d.map = raster_to_packed;
    d.dq = x.dq_local, d.dk = x.dk_local, d.dv = (char*)x.dv_local.data;
    d.dvsb = x.dv_local.sb, d.dvsh = x.dv_local.sh, d.dvsn = x.dv_local.sn;
    d.scale = 1.f / sqrtf((float)x.head_dim);
    d.scale_log2 = kLog2e * d.scale;
    hipStream_t s = as_stream(stream);
    int rc = P3D_OK;
    switch (x.head_dim) {
        case 16: rc = launch_d<16>(d, x.dtype, s); break;
        case 32: rc = launch_d<32>(d, x.dtype, s); break;
        case 48: rc = launch_d<48>(d, x.dtype, s); break;
        case 64: rc = launch_d<64>(d, x.dtype, s); break;
        default: rc = launch_d<128>(d, x.dtype, s); break;
    }
    if (rc != P3D_OK) return rc;
    return check_launch("p3d_local_bwd_grid");
}
