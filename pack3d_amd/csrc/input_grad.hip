// Input gradient of the layer's three input projections in 16-bit training:
// the backward of q = xn Wq^T, kv = xn Wkv^T and the gate logits xn Wg^T + bg
// (attention.py:64-67,85 of amilworks/Pack3D) with respect to the normalised
// tokens xn, dxn = dq Wq + dkv Wkv + dg Wg, as one contraction over the
// concatenated output features k = [q | kv | gate] in a single pass over the
// three gradients.
//
// D = W^T dY^T on 32x32x16 MFMAs: the A operand is a 32-channel block of
// W^T ([dim][k_pad], the host's transposed concatenation, zero columns past
// the last feature), staged through LDS 64 features at a time and shared by
// the workgroup's waves; the B operand is a wave's 32 token rows of dY, read
// straight from the three gradient tensors (lane l: token l % 32, features
// 8 (l / 32) .. +8 of the k-step).  Lane l then holds channels
// 32 cb + acc_row(r, l / 32) of token l % 32.  Each wave keeps all of its
// token tile's channel blocks (CB = NB; WT = NB / CB waves per tile is 1 for
// every width taken: split over two waves, each tile's dY rows were read twice
// and the pass took 25% longer) for the whole contraction.  Widths past 256
// (384, 512) go to two channel halves on grid y, each workgroup computing one
// half (its W^T rows, its dx columns), so dY is read once per half; the
// registers of a whole 512-channel row would not fit.  The result goes
// through the wave's LDS tile and leaves as 16-byte row pieces, rounded once
// from the fp32 sum.
#include "attn_common.hpp"

namespace p3d {
namespace {

constexpr int kIgWaves = 8;
constexpr int kIgChunk = 64;  // features per staged W^T chunk (4 k-steps)

struct IgDev {
    const char *dq, *dkv, *dg;
    int64_t dq_s, dkv_s, dg_s;  // row strides (elements)
    int q_out, kv_out, k_end;   // feature ranges [0, q_out), [q_out, q_out + kv_out), [.., k_end)
    const char* wt;             // [dim][k_pad]
    int k_pad;
    char* dx;                   // [rows][ldx]
    int64_t rows;
    int ldx;                    // dx row stride (elements): the whole width
};

template <typename T>
__device__ __forceinline__ const T* tp(const char* p) { return reinterpret_cast<const T*>(p); }

template <typename T>
__device__ __forceinline__ void store4(T* dst, const float (&v)[4]) {
    typedef __attribute__((ext_vector_type(4))) T T4;
    T4 o;
#pragma unroll
    for (int i = 0; i < 4; ++i) o[i] = from_f32<T>(v[i]);
    *reinterpret_cast<T4*>(dst) = o;
}

// NB 32-channel blocks of dim, CB of them per wave (WT = NB / CB waves per
// 32-token tile).
template <typename T, int NB, int CB>
__global__ __launch_bounds__(64 * kIgWaves, 2) void k_input_grad(IgDev a) {
    typedef Mma<T> M;
    typedef typename M::Frag Frag;
    constexpr int DIM = 32 * NB, WT = NB / CB, TILES = kIgWaves / WT;
    constexpr int WS = kIgChunk + 8;                  // LDS W^T row stride (elements), 16-byte pad
    constexpr int PIECES = DIM * kIgChunk / 8;        // 16-byte pieces of a chunk
    constexpr int PPT = (PIECES + 64 * kIgWaves - 1) / (64 * kIgWaves);
    constexpr int KSC = kIgChunk / 16;                // k-steps per chunk
    constexpr int OS = 32 + 8;                        // output tile row stride (elements)
    static_assert(NB % CB == 0 && kIgWaves % WT == 0, "channel blocks per wave");
    __shared__ __align__(16) T wbuf[2][DIM * WS];
    __shared__ __align__(16) T otile[kIgWaves][32 * OS];

    const int lane = threadIdx.x & 63, g = lane >> 5, t = lane & 31, wave = threadIdx.x >> 6;
    const int tile = wave / WT, cb0 = (wave % WT) * CB;
    const int64_t tok0 = ((int64_t)blockIdx.x * TILES + tile) * 32;
    const int64_t trow = min(tok0 + t, a.rows - 1);  // dead lanes read the last row, their outputs are dropped
    const int chunks = a.k_pad / kIgChunk;
    // This workgroup's channel half (grid y): W^T rows and dx columns from DIM * blockIdx.y.
    const T* wt = tp<T>(a.wt) + (int64_t)blockIdx.y * DIM * a.k_pad;

    // W^T chunk c: rows = channels, 64 features each.
    u32x4 wreg[PPT];
    auto fetch = [&](int c) __attribute__((always_inline)) {
#pragma unroll
        for (int i = 0; i < PPT; ++i) {
            const int pc = min((int)threadIdx.x + i * 64 * kIgWaves, PIECES - 1);
            const int r = pc / (kIgChunk / 8), col = (pc % (kIgChunk / 8)) * 8;
            wreg[i] = *reinterpret_cast<const u32x4*>(wt + (int64_t)r * a.k_pad + (int64_t)c * kIgChunk + col);
        }
    };
    auto stage = [&](int buf) __attribute__((always_inline)) {
#pragma unroll
        for (int i = 0; i < PPT; ++i) {
            const int pc = threadIdx.x + i * 64 * kIgWaves;
            const int r = pc / (kIgChunk / 8), col = (pc % (kIgChunk / 8)) * 8;
            if (pc < PIECES) *reinterpret_cast<u32x4*>(&wbuf[buf][r * WS + col]) = wreg[i];
        }
    };
    // dY fragment of feature k0 .. k0 + 7 of this lane's token (zero past k_end).
    auto dy_frag = [&](int k0) __attribute__((always_inline)) -> Frag {
        const T* src;
        if (k0 < a.q_out)
            src = tp<T>(a.dq) + trow * a.dq_s + k0;
        else if (k0 < a.q_out + a.kv_out)
            src = tp<T>(a.dkv) + trow * a.dkv_s + (k0 - a.q_out);
        else
            src = tp<T>(a.dg) + trow * a.dg_s + (k0 < a.k_end ? k0 - a.q_out - a.kv_out : 0);
        const Frag f = __builtin_bit_cast(Frag, *reinterpret_cast<const u32x4*>(src));
        return k0 < a.k_end ? f : frag_fill<T>(0.f);
    };

    f32x16 acc[CB];
#pragma unroll
    for (int cb = 0; cb < CB; ++cb)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[cb][r] = 0.f;

    // The dY fragments of a chunk are loaded two chunks ahead, rotating
    // through three register sets (a copy from one set to another would wait
    // for the loads in flight).
    Frag b0[KSC], b1[KSC], b2[KSC];
#pragma unroll
    for (int ks = 0; ks < KSC; ++ks) b0[ks] = dy_frag(16 * ks + 8 * g);
    if (chunks > 1) {
#pragma unroll
        for (int ks = 0; ks < KSC; ++ks) b1[ks] = dy_frag(kIgChunk + 16 * ks + 8 * g);
    }
    fetch(0);
    stage(0);
    fetch(min(1, chunks - 1));
    __syncthreads();

    auto step = [&](int c, Frag (&cur)[KSC], Frag (&far)[KSC]) __attribute__((always_inline)) {
        if (c + 2 < chunks) {
#pragma unroll
            for (int ks = 0; ks < KSC; ++ks) far[ks] = dy_frag((c + 2) * kIgChunk + 16 * ks + 8 * g);
        }
        const T* wb = &wbuf[c & 1][(32 * cb0 + t) * WS + 8 * g];
#pragma unroll
        for (int ks = 0; ks < KSC; ++ks)
#pragma unroll
            for (int cb = 0; cb < CB; ++cb)
                acc[cb] = M::mfma(*reinterpret_cast<const Frag*>(wb + 32 * cb * WS + 16 * ks), cur[ks], acc[cb]);
        // Unconditional (a stage after the last chunk fills a buffer no one
        // reads), so that every chunk issues the same loads.
        stage((c + 1) & 1);
        fetch(min(c + 2, chunks - 1));
        __syncthreads();
    };
    for (int c = 0; c < chunks; c += 3) {
        step(c, b0, b2);
        if (c + 1 < chunks) step(c + 1, b1, b0);
        if (c + 2 < chunks) step(c + 2, b2, b1);
    }

    // Each block through the wave's tile: row t, channels acc_row(4 qd, g) ..
    // +3, then 16-byte pieces (token tt, channels 8 pp .. +7), four lanes per
    // token.
    T* tl = otile[wave];
    T* dx = reinterpret_cast<T*>(a.dx) + (int64_t)blockIdx.y * DIM;
#pragma unroll
    for (int cb = 0; cb < CB; ++cb) {
#pragma unroll
        for (int qd = 0; qd < 4; ++qd) {
            const float v[4] = {acc[cb][4 * qd], acc[cb][4 * qd + 1], acc[cb][4 * qd + 2], acc[cb][4 * qd + 3]};
            store4<T>(tl + t * OS + acc_row(4 * qd, g), v);
        }
        wave_lds_sync();
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const int tt = 16 * i + (lane >> 2), pp = lane & 3;
            const u32x4 piece = *reinterpret_cast<const u32x4*>(tl + tt * OS + 8 * pp);
            if (tok0 + tt < a.rows)
                *reinterpret_cast<u32x4*>(dx + (tok0 + tt) * a.ldx + 32 * (cb0 + cb) + 8 * pp) = piece;
        }
        wave_lds_sync();  // the next block's tile writes follow these reads
    }
}

template <typename T, int NB, int CB>
void launch_ig(const IgDev& d, int halves, hipStream_t s) {
    constexpr int TILES = kIgWaves / (NB / CB);
    const int64_t blocks = cdiv(d.rows, 32 * TILES);
    k_input_grad<T, NB, CB><<<dim3((unsigned)blocks, (unsigned)halves), 64 * kIgWaves, 0, s>>>(d);
}

template <typename T>
int dispatch_ig(const IgDev& d, int dim, hipStream_t s) {
    switch (dim) {
        case 64: launch_ig<T, 2, 2>(d, 1, s); break;
        case 96: launch_ig<T, 3, 3>(d, 1, s); break;
        case 128: launch_ig<T, 4, 4>(d, 1, s); break;
        case 192: launch_ig<T, 6, 6>(d, 1, s); break;
        case 256: launch_ig<T, 8, 8>(d, 1, s); break;
        case 384: launch_ig<T, 6, 6>(d, 2, s); break;
        case 512: launch_ig<T, 8, 8>(d, 2, s); break;
        default: return fail(P3D_EUNSUPPORTED, "p3d_input_grad: dim must be 64, 96, 128, 192, 256, 384 or 512");
    }
    return P3D_OK;
}

}  // namespace
}  // namespace p3d

using namespace p3d;

extern "C" int p3d_input_grad(const void* dq, int64_t dq_stride, int32_t q_out, const void* dkv, int64_t dkv_stride,
                              int32_t kv_out, const void* dg, int64_t dg_stride, int32_t g_out, const void* wt,
                              int32_t k_pad, void* dx, int64_t rows, int32_t dim, int32_t dtype, void* stream) {
    P3D_REQUIRE(dq && dkv && dg && wt && dx, "null pointer argument");
    P3D_REQUIRE(dtype == P3D_F16 || dtype == P3D_BF16, "dtype must be fp16 or bf16");
    P3D_REQUIRE(rows >= 1 && rows < (1LL << 40), "bad row count");
    P3D_REQUIRE(q_out >= 8 && kv_out >= 8 && g_out >= 8 && q_out % 8 == 0 && kv_out % 8 == 0 && g_out % 8 == 0,
                "q_out, kv_out and g_out must be positive multiples of 8");
    const int64_t k_end = (int64_t)q_out + kv_out + g_out;
    P3D_REQUIRE(k_pad % kIgChunk == 0 && k_pad >= k_end && k_pad < (1 << 20),
                "k_pad must be a multiple of 64 covering q_out + kv_out + g_out");
    P3D_REQUIRE(dq_stride >= q_out && dkv_stride >= kv_out && dg_stride >= g_out && dq_stride % 8 == 0 &&
                    dkv_stride % 8 == 0 && dg_stride % 8 == 0,
                "row strides must cover the rows and keep 16-byte alignment");
    P3D_REQUIRE(aligned16(dq) && aligned16(dkv) && aligned16(dg) && aligned16(wt) && aligned16(dx),
                "pointers must be 16-byte aligned");
    IgDev d;
    d.dq = (const char*)dq, d.dkv = (const char*)dkv, d.dg = (const char*)dg;
    d.dq_s = dq_stride, d.dkv_s = dkv_stride, d.dg_s = dg_stride;
    d.q_out = q_out, d.kv_out = kv_out, d.k_end = (int)k_end;
    d.wt = (const char*)wt, d.k_pad = k_pad, d.dx = (char*)dx, d.rows = rows, d.ldx = dim;
    hipStream_t s = as_stream(stream);
    const int rc = dtype == P3D_F16 ? dispatch_ig<_Float16>(d, dim, s) : dispatch_ig<__bf16>(d, dim, s);
    if (rc != P3D_OK) return rc;
    return check_launch("p3d_input_grad");
}
