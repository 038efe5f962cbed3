// kd_fa_static.hip - kd_fa_dit_run_static: kd_fa_dit_run whose K workspace
// is a file-scope device array of the library instead of a caller buffer,
// for callers that cannot allocate device memory (code under stream capture,
// tight serving loops, harnesses that forbid hipMalloc).
//
// The array `scratch` (KD_FA_STATIC_SCRATCH_BYTES) exists once per GPU the
// library runs on and lives until the process ends.  Its device address is
// taken once per device, with that device current, by hipGetSymbolAddress on
// the entry point's first call there; host code then uses only that address
// (the array's name in host code is a host-side stand-in, not device
// memory).  The K pre-pass and the mask summary pass overwrite every byte
// of the workspace they use before the attention reads it, so nothing has
// to start at zero; two calls
// that overlap on one GPU (e.g. on two streams) share the array and race.
#include <hip/hip_runtime.h>

#include <mutex>

#include "../../include/kd_fa.h"
#include "kd_fa_kernel.h"

namespace {

static __device__ __align__(256) char scratch[KD_FA_STATIC_SCRATCH_BYTES];

struct ScratchSlot {
    std::once_flag once;
    void *ptr = nullptr;
    int status = KD_FA_ERR_DEVICE;
};
constexpr int kMaxDevices = 64;
ScratchSlot g_slot[kMaxDevices];

// The current device's address of `scratch` (looked up once per device).
int scratch_ptr(void **out) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return KD_FA_ERR_DEVICE;
    ScratchSlot &s = g_slot[dev];
    std::call_once(s.once, [&s] {
        void *p = nullptr;
        if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) == hipSuccess && p != nullptr) {
            s.ptr = p;
            s.status = KD_FA_OK;
        }
    });
    *out = s.ptr;
    return s.status;
}

}  // namespace

extern "C" int kd_fa_dit_run_static(const kd_fa_desc *desc, const kd_fa_rope *rope, const kd_fa_qk_norm *norm,
                                    void *stream) {
    int st = KD_FA_OK;
    const size_t k_need = kdfa::k_workspace_need(desc, rope, norm, &st);
    if (st != KD_FA_OK) return st;
    if (k_need > KD_FA_STATIC_SCRATCH_BYTES) return KD_FA_ERR_SCRATCH;
    // the transformed K and the mask summary of a masked short-key node; a
    // summary that does not fit is left out (the call then loads the mask
    // chunks of every tile, with the same result)
    const size_t need = kdfa::workspace_need(desc, rope, norm, &st);
    if (need == 0) return kdfa::run_node(desc, rope, norm, nullptr, 0, stream);
    st = kdfa::device_gfx950();
    if (st != KD_FA_OK) return st;
    void *ws = nullptr;
    st = scratch_ptr(&ws);
    if (st != KD_FA_OK) return st;
    return kdfa::run_node(desc, rope, norm, ws, KD_FA_STATIC_SCRATCH_BYTES, stream);
}
