/*
 * pack3d_hip.h -- C ABI of the MI355X (gfx950) PACK3D attention backend.
 *
 * Every entry point takes plain device pointers, sizes and a hipStream_t
 * (passed as void*), launches asynchronously on that stream, allocates no
 * memory and never synchronises, except where stated.  Each returns 0 on
 * success or a nonzero P3D_E* code; the message of the last failure on the
 * calling thread is p3d_last_error().  No exception crosses this boundary.
 *
 * The boundary replaces, in amilworks/Pack3D:
 *   - the CPU geometry construction of build_layout / prepare_geometry /
 *     TokenLayout.repack (src/pack3d/geometry.py:53-101,189-220,223-266);
 *   - the staged Triton forward of the core contract
 *     core(q, kl, vl, kg, vg, weight, bias, gate, sl, sg, geometry, temperature)
 *     (src/pack3d/backends/triton/kernels.py:289-311, autograd.py:40-64),
 *     with the rotary pre-pass rotate_projections (rotary.py:94-106) fused
 *     into the attention and pooling loads;
 *   - the explicit backward (kernels.py:314-356, rotary.py:64-70).
 */
#ifndef PACK3D_HIP_H
#define PACK3D_HIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define P3D_ABI_VERSION 19

enum p3d_status { P3D_OK = 0, P3D_EINVAL = 1, P3D_EHIP = 2, P3D_EUNSUPPORTED = 3 };
enum p3d_dtype { P3D_F32 = 0, P3D_F16 = 1, P3D_BF16 = 2 };

/* A rank-4 tensor [B, H, N, C] whose channel stride is 1: element (b,h,n,c)
 * lives at data + b*sb + h*sh + n*sn + c (strides in elements).  Rows must
 * start on 16-byte boundaries. */
typedef struct p3d_view {
    void* data;
    int64_t sb, sh, sn;
} p3d_view;

/* Axial rotary embedding, applied on load (rope.py:15-48).  For rotary pair
 * j (channels 2j, 2j+1) with pairs[j] = {base, stride, axis}, the rotation is
 * table[base + stride * pos_axis] = (cos, sin).  pos is the token's (z,y,x)
 * coordinate (coords[n] or, in the grid kernels, the brick coordinate) or,
 * when packed != 0, (packed row, 0, 0).  A one-entry table {1, 0} with all
 * strides 0 is the exact identity (pre-rotated inputs). */
typedef struct p3d_rope {
    const float* table;     /* float2 entries (cos, sin), built on the host */
    const int32_t* pairs;   /* [head_dim/2][3] */
    const int64_t* coords;  /* [N, 3] (z, y, x) or NULL when packed != 0 */
    int32_t packed;
    int32_t table_entries;  /* number of float2 entries in table */
} p3d_rope;

const char* p3d_last_error(void);
int p3d_abi_version(void);

/* ---- geometry (replaces geometry.py:223-266, 53-101, 189-220) ---------- */

/* build_layout for a complete grid: packed order, coordinates, raster->packed
 * map, neighbour table [N, W] in itertools.product offset order, and the
 * fine blocks [N/V, V] = arange.  morton != 0 selects native_block_morton
 * (Morton-ranked blocks, Morton-ranked slots); 0 selects raster_block.
 * Replaces geometry.py:241-260. */
int p3d_build_layout(const int64_t grid[3], const int64_t block[3], const int64_t radius[3],
                     int32_t morton, int64_t* order, int64_t* coords,
                     int32_t* raster_to_packed, int32_t* neighbors, int32_t* blocks,
                     void* stream);

/* prepare_geometry pass 1 (geometry.py:61-95): copies neighbours and blocks
 * (int32 or int64 input, is64 flags) to int32, and counts into flags[8]:
 *   [0] out-of-range neighbours  [1] out-of-range block members
 *   [2] rows with duplicate edges [3] tokens not covered exactly once
 *   [4] empty coarse groups       [5] maximum in-degree
 * degree[n] receives the in-degree of each token.  flags and degree are
 * cleared by the call.  The caller reads flags back (one small copy). */
int p3d_geometry_check(const void* neighbors, int32_t nb_is64, int64_t n, int32_t width,
                       const void* blocks, int32_t blocks_is64, int64_t fine, int32_t slots,
                       int32_t pool_size, int32_t* neighbors32, int32_t* blocks32,
                       int32_t* degree, int32_t* cover, int32_t* flags, void* stream);

/* Reverse adjacency (geometry.py:88-99): reverse[j] lists ascending the rows i
 * whose neighbour row contains j, padded with -1 to rwidth columns.  cursor[n]
 * is scratch (cleared by the call). */
int p3d_reverse_adjacency(const int32_t* neighbors, int64_t n, int32_t width, int32_t* cursor,
                          int32_t* reverse, int32_t rwidth, void* stream);

/* TokenLayout.repack (geometry.py:189-220): new row i = old row perm[i].
 * inverse[n] (int64 scratch) receives perm^-1.  flags[0] counts entries of perm
 * that are out of range or repeated (cleared by the call).  raster_map may be
 * NULL (identity); raster_map_out may be NULL (no grid tag). */
int p3d_repack(const int64_t* perm, int64_t n, const int32_t* neighbors, int32_t width,
               const int32_t* blocks, int64_t fine, int32_t slots, const int64_t* order,
               const int64_t* coords, const int32_t* raster_map, int64_t* inverse,
               int32_t* neighbors_out, int32_t* blocks_out, int64_t* order_out,
               int64_t* coords_out, int32_t* raster_map_out, int32_t* flags, void* stream);

/* TokenLayout validation (geometry.py:145-160): flags[0] counts tokens whose
 * order entry is out of range or repeated or whose coordinate disagrees with
 * order.  scratch[n] is cleared by the call. */
int p3d_check_layout(const int64_t grid[3], const int64_t* order, const int64_t* coords,
                     int32_t* scratch, int32_t* flags, void* stream);

/* Whether a neighbour table is a complete grid stencil.  The reference tags
 * only the radius-one stencils that build_layout makes (geometry.py:262-265,
 * _radius_one_grid) and transports the tag through repack (geometry.py:211-
 * 217); this call proves the tag for any radius from a layout's order, so a
 * reference-built layout can take the brick kernels.  It writes
 * raster_to_packed[t] = packed row of raster index t (-1 when order misses
 * t) and counts into flags[8] (cleared by the call):
 *   [0] order entries outside [0, n)
 *   [1] entries of neighbors [n, width] that differ from the product-order
 *       stencil of `radius` on `grid` (geometry.py:253-259).
 * width must equal prod(2 radius + 1).  The caller reads flags back. */
int p3d_stencil_match(const int64_t grid[3], const int64_t radius[3], const int64_t* order,
                      const int32_t* neighbors, int32_t width, int32_t* raster_to_packed,
                      int32_t* flags, void* stream);

/* ---- forward (replaces kernels.py:289-311 and rotary.py:94-106) -------- */

/* Two-stage summary pooling with the key rotation fused (compression.py:28-44,
 * kernels.py:12-40).  Outputs, for M summaries padded to Mp = ceil(M/32)*32:
 *   sk  [B, G, Mp, D]           pooled rotated keys times key_scale (dtype),
 *                               pad rows zero
 *   svt [B, G, Mp/32, D, 32]    pooled values, transposed per 32 summaries
 *   sk_norm_max [B, G, 64] (fp32)  maxima of the 2-norms of the stored
 *                               (rounded) sk rows, summary m reducing into
 *                               slot m % 64; their max bounds every summary
 *                               score of a query (Cauchy-Schwarz)
 * The call clears sk_norm_max with a launch of its own before pooling,
 * unless norms_cleared is nonzero: the caller then guarantees that the 64
 * slots per (batch, kv head) hold zeros (a buffer allocated zeroed for this
 * call, say). */
typedef struct p3d_pool_args {
    int32_t batch, kv_heads, tokens, head_dim, dtype;
    int32_t fine_blocks, slots, pool_size, summaries;
    float temperature;
    float key_scale;            /* sk is stored multiplied by this (the attention
                                   kernels pass log2(e)/sqrt(d)) */
    p3d_view kg, vg;
    const int32_t* blocks;      /* [F, V] */
    const float* weight;        /* [D] fp32 */
    const float* bias;          /* [V] fp32 */
    p3d_rope rope;
    void* sk;
    void* svt;
    float* sk_norm_max;
    int32_t norms_cleared;      /* nonzero: sk_norm_max already zero, no clear */
} p3d_pool_args;
int p3d_pool_fwd(const p3d_pool_args* args, void* stream);

/* Fused local + global attention with the fusion epilogue
 * y = sl * o_L + gate * sg * o_G (reference.py:20-31; kernels.py:43-103).
 * Two online-softmax states (local over the neighbourhood, global over all
 * summaries) are kept and combined at the end.
 *
 * p3d_attn_fwd_grid: complete-grid layouts (build_layout and its repacks).
 *   Queries are tiled by 3-D bricks in coordinate space; the local pathway
 *   reads the radius (<= 2 per axis) stencil from an LDS halo, so the
 *   neighbour table is not read.  raster_to_packed may be NULL (identity).
 * p3d_attn_fwd_rows: any validated geometry.  Queries are tiled by packed
 *   rows; the local branch is y itself when o_local_in is NULL (y holds
 *   sl * o_L from p3d_local_fwd_indexed), else o_local_in (fp32 [B,H,N,D],
 *   contiguous). */
typedef struct p3d_attn_args {
    int32_t batch, heads, kv_heads, tokens, head_dim, dtype;
    int32_t summaries;          /* M */
    int32_t gate_dtype;
    p3d_view q, kl, vl;         /* q [B,H,N,D]; kl, vl [B,G,N,D] */
    p3d_view gate;              /* [B,H,N]; only sb, sh, sn are used */
    const float* local_scale;   /* [D] fp32 */
    const float* global_scale;  /* [D] fp32 */
    const void* sk;             /* from p3d_pool_fwd */
    const void* svt;
    const float* sk_norm_max;   /* from p3d_pool_fwd */
    p3d_rope rope;
    int32_t grid[3];            /* grid kernel: (Z, Y, X) */
    int32_t radius[3];          /* grid kernel: per-axis radius, each <= 2 */
    const int32_t* raster_to_packed;
    const float* o_local_in;    /* rows kernel: fp32 [B,H,N,D] contiguous */
    p3d_view y;                 /* output [B,H,N,D], dtype */
    /* optional saved state for backward (NULL to skip), contiguous: */
    float* lse_local;           /* [B,H,N] */
    float* lse_global;          /* [B,H,N] */
    void* o_local;              /* [B,H,N,D] dtype */
    void* o_global;             /* [B,H,N,D] dtype */
    int32_t kl_rotated;         /* nonzero: kl already holds R(pos) kl rounded to
                                   dtype (p3d_project_pool with rotate_kl, or
                                   p3d_rotate); the grid kernel then rotates
                                   only q.  The rows and indexed kernels always
                                   take kl rotated. */
} p3d_attn_args;
int p3d_attn_fwd_grid(const p3d_attn_args* args, void* stream);
int p3d_attn_fwd_rows(const p3d_attn_args* args, void* stream);

/* p3d_pool_fwd followed by p3d_attn_fwd_grid, allocating nothing.  No
 * counterpart in the reference: it serves callers that cannot allocate
 * device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc).  The pooled summaries and the norm
 * slots -- the forward's only memory beyond its inputs and outputs -- live
 * in a file-scope device array of 8 MiB that each GPU holds until the
 * process ends; the sk, svt, sk_norm_max and norms_cleared fields of both
 * argument blocks are ignored.  The summaries must fit: 2 *
 * round256(B * G * ceil32(M) * D * element size) + round256(B * G * 256)
 * bytes <= 8 MiB (c2 in bf16 needs 3.2 MB), else P3D_EINVAL before any
 * launch.  Every call on a GPU uses that GPU's one array, so calls that
 * overlap on one GPU race; the stream must belong to the current device.
 * The two argument blocks must agree on batch, kv_heads, tokens, head_dim,
 * dtype and summaries. */
int p3d_attn_fwd_grid_noalloc(const p3d_pool_args* pool, const p3d_attn_args* args, void* stream);

/* Indexed local attention for arbitrary validated graphs (reference.py:23-30;
 * replaces the reference's _local_fwd, kernels.py:43-66), neighbours
 * neighbors [N, width], -1 = absent.  q is rotated on load with args->rope
 * (identity for pre-rotated q); kl must already be rotated.  Writes
 * y = sl * o_L in the storage type (the rows kernel's epilogue then adds the
 * global branch, with o_local_in NULL) and, if non-NULL, o_local [B,H,N,D]
 * in the storage type and lse_local [B,H,N].  An all-masked row gives 0 and
 * lse = -inf.  The sk / svt / norm fields of args are not read. */
int p3d_local_fwd_indexed(const p3d_attn_args* args, const int32_t* neighbors, int32_t width, void* stream);

/* Standalone rotation (rotary.py:10-45): y = R(pos) x, or R(pos)^T x when
 * inverse != 0, for x and y [B, H, N, D] views of dtype; D in {16, 32, 48,
 * 64, 128}, as for the attention kernels. */
int p3d_rotate(p3d_view x, p3d_view y, int32_t batch, int32_t heads, int32_t tokens,
               int32_t head_dim, int32_t dtype, const p3d_rope* rope, int32_t inverse, void* stream);

/* ---- layer (attention.py:64) ------------------------------------------- */

/* nn.LayerNorm over the last dimension of x [rows, dim] (contiguous, dtype):
 * y = (x - mean) / sqrt(var + eps) * weight + bias, statistics in fp32,
 * weight / bias [dim] of param_dtype.  dim must be a multiple of the 16-byte
 * piece and at most 512. */
int p3d_layer_norm(const void* x, const void* weight, const void* bias, int32_t param_dtype, void* y,
                   int64_t rows, int32_t dim, int32_t dtype, float eps, void* stream);

/* The same LayerNorm for training (the forward of torch's layer_norm under
 * autocast, with its output rounded to the compute type that the next
 * linear maps cast it to): x [rows, dim] of x_dtype, y [rows, dim] of
 * y_dtype, and each row's mean and 1/sqrt(var + eps) as fp32 [rows] for the
 * backward.  x_copy (may be NULL): x rounded to y_dtype [rows, dim], the
 * residual operand of the layer's output product under autocast
 * (attention.py:89), written from the same read of x.  dim a multiple of
 * x's 16-byte piece, at most 512. */
int p3d_layer_norm_train(const void* x, const void* weight, const void* bias, int32_t param_dtype, void* y,
                         void* x_copy, float* mean, float* rstd, int64_t rows, int32_t dim, int32_t x_dtype,
                         int32_t y_dtype, float eps, void* stream);

/* LayerNorm backward (torch's layer_norm backward): with xhat = (x - mean)
 * rstd and g = dy * weight, dx = rstd (g - mean(g) - xhat mean(g xhat)) per
 * row, plus dres (may be NULL; [rows, dim] of dx_dtype: the gradient that
 * reaches x through the residual branch) added in fp32, written as dx_dtype;
 * the affine gradients as fp32 partial sums over `parts` row ranges,
 * partial[part][0][dim] = sum dy xhat and partial[part][1][dim] = sum dy (the
 * caller sums the parts).  mean / rstd from p3d_layer_norm_train. */
int p3d_layer_norm_bwd(const void* dy, const void* dres, const void* x, const void* weight, int32_t param_dtype,
                       const float* mean, const float* rstd, void* dx, float* partial, int64_t rows, int32_t dim,
                       int32_t dy_dtype, int32_t x_dtype, int32_t dx_dtype, int32_t parts, void* stream);

/* Fused input projections of the layer (attention.py:64-67,85): LayerNorm
 * of x [rows, dim], then q = xn Wq^T [rows, q_out], kv = xn Wkv^T
 * [rows, kv_out] (the chunks kl | vl | kg | vg of to_kv) and, for each of
 * the `heads` gate pairs, gate[row, h] = softmax(xn Wg^T + b_g)[2h + 1]
 * [rows, heads], where Wg is [2 heads, dim].  x, the weights and the outputs
 * have dtype (fp16 or bf16); the LayerNorm parameters and the gate bias have
 * their own dtypes.  Rounding points are those of the torch ops it replaces:
 * the normalised tokens, the linear outputs (the gate's after its bias) and
 * the gate probability are rounded to dtype.  Replaces nn.LayerNorm, the
 * to_q / to_kv / gate nn.Linear calls and the gate softmax of the layer's
 * no-grad forward.  dim in {64, 96, 128, 192, 256, 384, 512}; q_out and
 * kv_out multiples of 16; x, the weights, q and kv 16-byte aligned, all
 * contiguous. */
typedef struct p3d_project_args {
    const void* x;
    const void* ln_weight;
    const void* ln_bias;
    const void* wq;
    const void* wkv;
    const void* wg;
    const void* gate_bias;
    void* q;
    void* kv;
    void* gate;
    int64_t rows;
    int32_t dim, q_out, kv_out, heads;
    int32_t dtype, ln_dtype, gate_bias_dtype;
    float eps;
} p3d_project_args;

int p3d_project(const p3d_project_args* args, void* stream);

/* The three input projections of tokens that are already normalised: the
 * to_q, to_kv and gate nn.Linear calls of attention.py:64-67,85 in 16-bit
 * training, where the LayerNorm output is its own tensor (kept for the
 * backward).  q = x Wq^T, kv = x Wkv^T and the gate logits x Wg^T +
 * gate_bias, written as [rows, 2 heads] to `gate`; each output accumulated in
 * fp32 and rounded once to dtype, as torch.mm / torch.addmm of the 16-bit
 * operands (the summation order differs, so values can differ in the last
 * bit).  ln_weight, ln_bias, ln_dtype and eps are not read; every other
 * argument and limit is p3d_project's.  Replaces the three GEMMs of the
 * training layer's input projections with one pass over x. */
int p3d_project_linear(const p3d_project_args* args, void* stream);

/* The projections of p3d_project with the summary pooling (compression.py:
 * 28-44, the pooling p3d_pool_fwd performs) fused in, for the no-grad
 * forward: writes q, kl, vl (the first 2 * kv_heads * head_dim columns of
 * each kv row) and gate, and the summaries sk, svt and the key-norm slots of
 * `pool`, from the kg and vg values it computes; the kg and vg columns of kv
 * are left unwritten.  Replaces, in the layer's no-grad forward
 * (attention.py:64-67 followed by the core's pooling, reference.py:13-14),
 * the projections and the pooling pass over kg / vg.  Contract: the layout's
 * fine block f of each batch is rows [64 f, 64 f + 64) of that batch (the
 * blocks of this package's build_layout), pool_size 1, 64 slots; pool->kg,
 * pool->vg and pool->blocks are not read.  Returns P3D_EUNSUPPORTED, before
 * launching anything, for shapes outside head_dim 16/32/48/64, kv_heads *
 * head_dim <= 192, tokens a multiple of 64 and dim 64/96/128/192/256 (the
 * caller then runs p3d_project and p3d_pool_fwd); P3D_EINVAL for arguments
 * either would reject.  rotate_kl nonzero: kl is written rotated by
 * pool->rope (rounded to dtype, rotated in fp32, rounded again -- the values
 * the attention kernels rotate it to), for p3d_attn_args.kl_rotated. */
int p3d_project_pool(const p3d_project_args* args, const p3d_pool_args* pool, int32_t rotate_kl, void* stream);

/* Output projection with the residual (attention.py:89): out = x + y Wo^T for
 * y [rows, k] (the core's output, heads concatenated) and Wo [dim, k] of
 * dtype (fp16 or bf16), x and out [rows, dim] of res_dtype, all contiguous
 * and 16-byte aligned.  res_dtype == dtype: fp32 accumulation and one
 * rounding of x + y Wo^T, as torch.addmm(x, y, Wo^T); it replaces the
 * layer's to_out nn.Linear and residual add in the no-grad forward.
 * res_dtype == P3D_F32 (autocast over an fp32 input): y Wo^T rounded to dtype
 * and added to the unrounded x in fp32, as the reference's sum of an fp32
 * residual and a 16-bit to_out output.  k in {64, 96, 128, 192, 256, 384,
 * 512}; dim a multiple of 32, at most 512. */
int p3d_out_residual(const void* y, const void* wo, const void* x, void* out, int64_t rows, int32_t k,
                     int32_t dim, int32_t dtype, int32_t res_dtype, void* stream);

/* Copy of a [batch, heads, tokens, head_dim] tensor between two strided
 * views with contiguous, 16-byte aligned rows: a dense gradient of the
 * backward (the local pass's dvl) into the token-major layout of the layer's
 * to_kv output (attention.py:64-67), so that autograd receives the
 * projections' gradients whole instead of transposing and stacking views.
 * batch < 65536. */
int p3d_copy_rows(p3d_view src, p3d_view dst, int64_t batch, int32_t heads, int64_t tokens, int32_t head_dim,
                  int32_t dtype, void* stream);

/* Input gradient of the layer's three input projections in 16-bit training
 * (the backward of attention.py:64-67,85 with respect to the normalised
 * tokens; torch's autograd computes it as three products dq Wq, dkv Wkv,
 * dgl Wg and adds them): dx = dq Wq + dkv Wkv + dg Wg as one contraction over
 * the concatenated features, summed in fp32 and rounded once to dtype.
 * dq [rows, q_out], dkv [rows, kv_out], dg [rows, g_out] with row strides in
 * elements (multiples of 8, 16-byte aligned rows); wt = [Wq; Wkv; Wg]^T as a
 * contiguous [dim][k_pad] matrix whose columns past q_out + kv_out + g_out
 * are zero, k_pad a multiple of 64; dx [rows, dim] contiguous.  q_out, kv_out,
 * g_out positive multiples of 8; dim 64, 96, 128, 192, 256, 384 or 512 (the
 * last two in two channel halves, the gradients read once per half); fp16 /
 * bf16. */
int p3d_input_grad(const void* dq, int64_t dq_stride, int32_t q_out, const void* dkv, int64_t dkv_stride,
                   int32_t kv_out, const void* dg, int64_t dg_stride, int32_t g_out, const void* wt, int32_t k_pad,
                   void* dx, int64_t rows, int32_t dim, int32_t dtype, void* stream);

/* Weight gradient of a linear map y = x W^T (the W part of the backward of
 * the layer's to_q, to_kv, gate and to_out nn.Linear maps, attention.py:64-67,
 * 85,89; torch computes it as dy^T x): dw[o][i] = sum over rows n of
 * dy[n][o] x[n][i] with fp32 accumulation, written as fp32 [out_features,
 * in_features].  dy [rows, out_features] and x [rows, in_features] are
 * fp16 or bf16 with row strides ldy, ldx (elements, multiples of 8, 16-byte
 * aligned rows).  The rows are split into `splits` ranges whose fp32
 * partials go to workspace [splits, out_features, in_features] and are then
 * summed in order (deterministic).  out_features a positive multiple of 8;
 * in_features a multiple of 32 up to 256, or a multiple of 256 up to 2048
 * (taken in column blocks of 256, dy read once per block). */
int p3d_weight_grad(const void* dy, int64_t ldy, const void* x, int64_t ldx, float* dw, float* workspace,
                    int64_t rows, int32_t out_features, int32_t in_features, int32_t splits, int32_t dtype,
                    void* stream);

/* p3d_weight_grad of three linear maps that share their input x (the
 * layer's to_q, to_kv and gate, attention.py:64-67,85) in one pass over x:
 * dw [out0 + out1 + out2, in_features] fp32 holds dW of dy0, then of dy1,
 * then of dy2, each dy with its own row stride.  Same rules as
 * p3d_weight_grad; the out counts positive multiples of 8. */
int p3d_weight_grad3(const void* dy0, int64_t ld0, int32_t out0, const void* dy1, int64_t ld1, int32_t out1,
                     const void* dy2, int64_t ld2, int32_t out2, const void* x, int64_t ldx, float* dw,
                     float* workspace, int64_t rows, int32_t in_features, int32_t splits, int32_t dtype,
                     void* stream);

/* ---- backward (replaces kernels.py:313-356, autograd.py:19-28) --------- */

/* Shared argument block of the backward passes.  q and kl are the ROTATED
 * inputs (the host rotates them once); sk / svt / lse / o_* are the forward's
 * outputs.  Every buffer is caller-owned device memory; [B,H,N,D] buffers are
 * contiguous unless given as a p3d_view. */
typedef struct p3d_bwd_args {
    int32_t batch, heads, kv_heads, tokens, head_dim, dtype;
    int32_t summaries, gate_dtype;
    int32_t parts;              /* p3d_mix_bwd: blocks, rows of dsl_part / dsg_part */
    int32_t splits;             /* p3d_global_bwd: query splits of the summary dK/dV */
    p3d_view q, kl, vl;         /* rotated q [B,H,N,D]; rotated kl, vl [B,G,N,D] */
    p3d_view gate;              /* [B,H,N] of gate_dtype */
    const float* local_scale;   /* [D] fp32 */
    const float* global_scale;  /* [D] fp32 */
    const void* sk;             /* [B,G,Mp,D] pooled keys times key_scale */
    const void* svt;            /* [B,G,Mp/32,D,32] */
    float key_scale;
    int32_t pad_;
    const void* o_local;        /* [B,H,N,D] saved o_L (dtype) */
    const void* o_global;       /* [B,H,N,D] saved o_G (dtype) */
    const float* lse_local;     /* [B,H,N] natural-log lse of the local softmax */
    const float* lse_global;    /* [B,H,N] */
    p3d_view dy;                /* upstream gradient [B,H,N,D] (dtype) */
    void* dol;                  /* out of mix: dy * sl rounded (dtype) */
    void* dog;                  /* out of mix: dy * gate * sg rounded (dtype) */
    float* delta_local;         /* out of mix: [B,H,N] sum dO_L o_L */
    float* delta_global;        /* out of mix: [B,H,N] sum dO_G o_G */
    void* dgate;                /* out of mix: [B,H,N] of gate_dtype */
    float* dsl_part;            /* out of mix: [parts, D] partial dsl */
    float* dsg_part;            /* out of mix: [parts, D] partial dsg */
    void* sv_rows;              /* workspace [B,G,Mp,D] (dtype) */
    void* skt;                  /* workspace [B,G,Mp/32,D,32] (dtype) */
    float* dq_local;            /* out: [B,H,N,D] fp32, rotated space */
    float* dq_global;           /* out: [B,H,N,D] fp32, rotated space */
    float* dk_local;            /* out: [B,G,N,D] fp32, rotated space */
    p3d_view dv_local;          /* out: [B,G,N,D] view (dtype), 16-byte aligned rows */
    float* dsk_part;            /* out: [splits,B,G,Mp,D] fp32, true key units */
    float* dsv_part;            /* out: [splits,B,G,Mp,D] fp32 */
    const void* q_t;            /* optional: rotated q transposed, [B*H][D][N] (p3d_transpose_rows) */
    const void* dog_t;          /* optional: dog transposed, [B*H][D][N]; with both, fp16 / bf16,
                                   N >= 64 and N a multiple of 8, p3d_global_bwd_dkv copies its
                                   transposed query stages from them by LDS DMA */
} p3d_bwd_args;

/* Fusion step (kernels.py:106-127): dO_L = round(dy sl), dO_G = round(dy gate
 * sg), Delta_L = sum dO_L o_L, Delta_G = sum dO_G o_G, dgate = sum dy sg o_G,
 * and per-block partial sums of dsl = sum dy o_L, dsg = sum dy gate o_G. */
int p3d_mix_bwd(const p3d_bwd_args* args, void* stream);

/* Local pathway backward for any validated graph (kernels.py:130-181): dq_local
 * over the neighbour rows, dk_local / dv_local over the reverse adjacency. */
int p3d_local_bwd_indexed(const p3d_bwd_args* args, const int32_t* neighbors, int32_t width,
                          const int32_t* reverse, int32_t rwidth, void* stream);

/* Local pathway backward for complete-grid layouts (build_layout and its
 * repacks; the brick decomposition of p3d_attn_fwd_grid): dq_local, dk_local
 * and dv_local as p3d_local_bwd_indexed, from halo planes in LDS on MFMA,
 * without the neighbour tables.  grid (Z, Y, X), per-axis radius <= 2.
 * Returns P3D_EUNSUPPORTED when a halo plane does not fit in LDS (fp32 with
 * head_dim 128). */
int p3d_local_bwd_grid(const p3d_bwd_args* args, const int32_t grid[3], const int32_t radius[3],
                       const int32_t* raster_to_packed, void* stream);

/* Summary pathway backward (kernels.py:184-237): dq_global and the split
 * partials dsk_part / dsv_part (sv_rows and skt are filled first). */
int p3d_global_bwd(const p3d_bwd_args* args, void* stream);

/* The two halves of p3d_global_bwd, for callers that time or order them
 * separately: _dq fills sv_rows and skt and computes dq_global
 * (kernels.py:179-207, the _global_dq pass); _dkv computes the split
 * partials dsk_part / dsv_part (kernels.py:209-240, the _global_dkv pass)
 * and reads the skt / sv_rows that _dq wrote, so it runs after it on the
 * same stream. */
int p3d_global_bwd_dq(const p3d_bwd_args* args, void* stream);
int p3d_global_bwd_dkv(const p3d_bwd_args* args, void* stream);

/* dst[(b H + h) D + c][n] = src[b][h][n][c] for fp16 / bf16 (tokens a
 * multiple of 8, src rows 16-byte aligned): the transposed copies q_t and
 * dog_t of p3d_bwd_args.  The reference has no counterpart (its Triton dK/dV
 * kernel loads q and dO tiles transposed, kernels.py:209-240); this build
 * stages them for the summary dK/dV pass. */
int p3d_transpose_rows(p3d_view src, void* dst, int32_t batch, int32_t heads, int32_t tokens, int32_t head_dim,
                       int32_t dtype, void* stream);

/* dq = R^T round(round(dq_local) + round(dq_global)) and dkl = R^T round(dk_local)
 * (kernels.py:202-206 rounding; R^T the inverse rotation of rope), written
 * into the views dq [B,H,N,D] and dkl [B,G,N,D] of dtype (16-byte aligned
 * rows; e.g. the q and kl column ranges of the projections' gradients). */
int p3d_finish_bwd(const p3d_bwd_args* args, const p3d_rope* rope, p3d_view dq, p3d_view dkl, void* stream);

/* Pooling backward (kernels.py:240-270): from the split partials of dsk / dsv,
 * writes dkg (gradient of the UNROTATED kg: R^T applied) and dvg into
 * [B,G,N,D] views of dtype (16-byte aligned rows), and per-summary partials
 * dw_part [B*G*Mp, D] and db_part [B*G*Mp, slots]. */
int p3d_pool_bwd(const p3d_pool_args* pool, const float* dsk_part, const float* dsv_part, int32_t splits,
                 p3d_view dkg, p3d_view dvg, float* dw_part, float* db_part, void* stream);

/* ---- self-tests (no counterpart in the reference) ---------------------- */

/* One MFMA of the kind the attention kernels issue for dtype (32x32x16 bf16 /
 * f16, 32x32x2 f32), loading A [32 x K] and B [K x 32] (row-major, dtype) with
 * the fragment layout the kernels assume and storing D = A B (fp32, row-major
 * 32 x 32) with the assumed accumulator layout.  Tests compare D with a
 * matmul to pin that layout on the device. */
int p3d_selftest_mfma(int32_t dtype, const void* a, const void* b, float* d, void* stream);


/* sizeof of p3d_view, p3d_rope, p3d_pool_args, p3d_attn_args, p3d_bwd_args,
 * p3d_project_args into out[6], so a binding can check its struct mirrors. */
int p3d_struct_sizes(int64_t* out);

#ifdef __cplusplus
}
#endif
#endif /* PACK3D_HIP_H */
