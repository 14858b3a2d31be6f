// The fused forward without allocation: pooling plus the brick attention
// kernel, with the pooled summaries (sk, svt) and the key-norm slots -- the
// only device memory the forward needs beyond its inputs and outputs -- kept
// in a file-scope device array instead of caller workspace.  For callers
// that cannot allocate (code under HIP graph capture, serving loops).
//
// Each GPU holds its own copy of the array until the process ends.  Every
// call on a GPU shares that GPU's copy, so calls that overlap on one GPU
// (different streams, or threads) race; the norm slots are cleared by every
// call before the pooling kernel reduces into them.
#include <mutex>

#include "common.hpp"

namespace p3d {

constexpr size_t kScratchBytes = (size_t)8 << 20;  // 8 MiB per GPU
static __device__ __align__(256) unsigned char scratch[kScratchBytes];

namespace {

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mutex;
void* g_scratch[kMaxDevices];  // device address of `scratch` per device; null until resolved

// The array's address on the current device, looked up once per device with
// that device current.  In host code `scratch` names a host-side stand-in,
// never the device memory: only this address may reach a kernel or a copy.
int scratch_on_current_device(void** out) {
    int dev = -1;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return fail(P3D_EHIP, std::string("hipGetDevice: ") + hipGetErrorString(e));
    if (dev < 0 || dev >= kMaxDevices) return fail(P3D_EUNSUPPORTED, "device index beyond the scratch table");
    std::lock_guard<std::mutex> lock(g_scratch_mutex);
    if (!g_scratch[dev]) {
        void* p = nullptr;
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !p)
            return fail(P3D_EHIP, std::string("hipGetSymbolAddress(scratch): ") + hipGetErrorString(e));
        g_scratch[dev] = p;
    }
    *out = g_scratch[dev];
    return P3D_OK;
}

int64_t round256(int64_t x) { return (x + 255) & ~(int64_t)255; }

}  // namespace
}  // namespace p3d

using namespace p3d;

extern "C" int p3d_attn_fwd_grid_noalloc(const p3d_pool_args* pool, const p3d_attn_args* args, void* stream) {
    P3D_REQUIRE(pool && args, "null args");
    P3D_REQUIRE(pool->batch == args->batch && pool->kv_heads == args->kv_heads && pool->tokens == args->tokens &&
                    pool->head_dim == args->head_dim && pool->dtype == args->dtype &&
                    pool->summaries == args->summaries,
                "pooling and attention arguments disagree");
    P3D_REQUIRE(args->dtype >= P3D_F32 && args->dtype <= P3D_BF16, "unknown dtype");
    P3D_REQUIRE(args->batch >= 1 && args->kv_heads >= 1 && args->head_dim >= 1 && args->summaries >= 1,
                "bad sizes");
    const int64_t es = args->dtype == P3D_F32 ? 4 : 2;
    const int64_t mp = ((int64_t)args->summaries + 31) / 32 * 32;
    const int64_t bg = (int64_t)args->batch * args->kv_heads;
    const int64_t sk_bytes = round256(bg * mp * args->head_dim * es);  // sk; svt has the same size
    const int64_t norm_bytes = round256(bg * 64 * 4);
    const int64_t need = 2 * sk_bytes + norm_bytes;
    if (need > (int64_t)kScratchBytes)
        return fail(P3D_EINVAL, "p3d_attn_fwd_grid_noalloc: the summaries need " + std::to_string(need) +
                                    " bytes of scratch, more than its " + std::to_string(kScratchBytes) +
                                    " (batch * kv_heads * ceil32(summaries) * head_dim * element size must "
                                    "stay below about 4 MiB)");
    void* base = nullptr;
    int rc = scratch_on_current_device(&base);
    if (rc) return rc;
    char* p = static_cast<char*>(base);
    p3d_pool_args pa = *pool;
    pa.sk = p;
    pa.svt = p + sk_bytes;
    pa.sk_norm_max = reinterpret_cast<float*>(p + 2 * sk_bytes);
    pa.norms_cleared = 0;  // the array keeps the last call's maxima: clear them first
    p3d_attn_args aa = *args;
    aa.sk = pa.sk;
    aa.svt = pa.svt;
    aa.sk_norm_max = pa.sk_norm_max;
    rc = p3d_pool_fwd(&pa, stream);
    if (rc) return rc;
    return p3d_attn_fwd_grid(&aa, stream);
}
