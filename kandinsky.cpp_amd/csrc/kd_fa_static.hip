// kd_fa_static.hip - kd_fa_dit_run_static: kd_fa_dit_run whose workspace
// is a file-scope device array of the library instead of a caller buffer,
// for callers that cannot allocate device memory (code under stream capture,
// tight serving loops, harnesses that forbid hipMalloc).
//
// The array `scratch` (KD_FA_STATIC_SCRATCH_BYTES) exists once per GPU the
// library runs on and lives until the process ends.  Its device address is
// taken per device, with that device current, by hipGetSymbolAddress on the
// entry point's first call there; only a successful lookup is kept (a failed
// one is tried again on the next call).  Host code then uses only that
// address (the array's name in host code is a host-side stand-in, not
// device memory).  The K / V pre-pass and the mask summary pass overwrite
// every byte of the workspace they use before the attention reads it, so
// nothing has to start at zero; two calls that overlap on one GPU (e.g. on
// two streams) share the array and race.
#include <hip/hip_runtime.h>

#include <atomic>
#include <mutex>

#include "../../include/kd_fa.h"
#include "kd_fa_kernel.h"

namespace {

static __device__ __align__(256) char scratch[KD_FA_STATIC_SCRATCH_BYTES];

constexpr int kMaxDevices = 64;
std::atomic<void *> g_scratch[kMaxDevices];
std::mutex g_lookup;

// The current device's address of `scratch`.
int scratch_ptr(void **out) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return KD_FA_ERR_DEVICE;
    void *p = g_scratch[dev].load(std::memory_order_acquire);
    if (!p) {
        std::lock_guard<std::mutex> lock(g_lookup);
        p = g_scratch[dev].load(std::memory_order_relaxed);
        if (!p) {
            if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) != hipSuccess || p == nullptr) return KD_FA_ERR_DEVICE;
            g_scratch[dev].store(p, std::memory_order_release);
        }
    }
    *out = p;
    return KD_FA_OK;
}

}  // namespace

extern "C" int kd_fa_dit_run_static(const kd_fa_desc *desc, const kd_fa_rope *rope, const kd_fa_qk_norm *norm,
                                    void *stream) {
    int st = KD_FA_OK;
    bool f32_kv = false;
    const size_t cast_need = kdfa::cast_workspace_need(desc, rope, norm, &st, &f32_kv);
    if (st != KD_FA_OK) return st;
    if (cast_need > KD_FA_STATIC_SCRATCH_BYTES) {
        // an F32 K or V is cast only through a workspace; 16-bit operands
        // run without one (K transformed in staged groups or on load: the
        // same result, bitwise)
        if (f32_kv) return KD_FA_ERR_SCRATCH;
        return kdfa::run_node(desc, rope, norm, nullptr, 0, stream);
    }
    // the transformed K, the cast V and the mask summary of a masked
    // short-key node; a summary that does not fit is left out (the call
    // then loads the mask chunks of every tile, with the same result)
    const size_t need = kdfa::workspace_need(desc, rope, norm, &st);
    if (need == 0) return kdfa::run_node(desc, rope, norm, nullptr, 0, stream);
    st = kdfa::device_gfx950();
    if (st != KD_FA_OK) return st;
    void *ws = nullptr;
    st = scratch_ptr(&ws);
    if (st != KD_FA_OK) return st;
    return kdfa::run_node(desc, rope, norm, ws, KD_FA_STATIC_SCRATCH_BYTES, stream);
}
