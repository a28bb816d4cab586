// mp_hip_paged_attention_decode_noalloc: the stand-alone paged GQA decode
// attention without any allocation, for callers that cannot allocate
// device memory (code under HIP graph capture, serving loops that forbid
// allocation).
//
// mp_hip_paged_attention_decode keeps the scores of a long row in global
// memory it allocates per call. Here that buffer is `scratch`, a
// file-scope device array of kScratchFloats floats (1 MiB) that every GPU
// running the library holds until the process ends. A row fits when
// heads * round_up(length, 16) <= kScratchFloats. The kernel writes every
// score slot before reading it, so the array needs no clearing between
// calls; calls that overlap on one GPU share it and race.
#include <hip/hip_runtime.h>

#include <mutex>
#include <string>

#include "../../../include/mp_hip.h"
#include "kernels.h"

namespace {

constexpr size_t kScratchFloats = 262144;  // 1 MiB

__device__ __align__(256) float scratch[kScratchFloats];

// Device address of `scratch` on each device, looked up once per device
// with that device current. The host-side name is only a stand-in and is
// never passed to a kernel or a copy.
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mutex;
float* g_scratch_address[kMaxDevices] = {};

int scratch_for_current_device(float** out, std::string* error) {
    int device = 0;
    hipError_t e = hipGetDevice(&device);
    if (e != hipSuccess) {
        *error = std::string("hipGetDevice: ") + hipGetErrorString(e);
        return MP_DEVICE_ERROR;
    }
    if (device < 0 || device >= kMaxDevices) {
        *error = "device index beyond the scratch table";
        return MP_DEVICE_ERROR;
    }
    std::lock_guard<std::mutex> lock(g_scratch_mutex);
    if (!g_scratch_address[device]) {
        void* address = nullptr;
        e = hipGetSymbolAddress(&address, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !address) {
            *error = std::string("hipGetSymbolAddress(scratch): ") + hipGetErrorString(e);
            return MP_DEVICE_ERROR;
        }
        g_scratch_address[device] = static_cast<float*>(address);
    }
    *out = g_scratch_address[device];
    return MP_OK;
}

}  // namespace

namespace mphip {
// Message of the last failed context-free call on this thread (mp_hip_last_error(NULL)).
void set_free_error(const std::string& message);
}  // namespace mphip

extern "C" int mp_hip_paged_attention_decode_noalloc(const float* q, const float* keys, const float* values,
                                                     const int32_t* table, int32_t length, int32_t layer,
                                                     int32_t layers, int32_t block_tokens, int32_t heads,
                                                     int32_t kv_heads, int32_t dim, float* out, void* stream) {
    if (!q || !keys || !values || !table || !out || length < 1 || layer < 0 || layer >= layers ||
        block_tokens < 1 || heads < 1 || kv_heads < 1 || heads % kv_heads || dim < 4 || dim % 4 || dim > 256 ||
        heads / kv_heads > 8) {
        mphip::set_free_error("invalid paged attention arguments");
        return MP_INVALID_ARGUMENT;
    }
    const size_t stride = (size_t)((length + 15) & ~15);
    if ((size_t)heads * stride > kScratchFloats) {
        mphip::set_free_error("row too long for the allocation-free attention: heads * round_up(length, 16) = " +
                              std::to_string((size_t)heads * stride) + " floats exceeds the " +
                              std::to_string(kScratchFloats) + "-float scratch");
        return MP_INVALID_ARGUMENT;
    }
    float* buffer = nullptr;
    std::string error;
    const int status = scratch_for_current_device(&buffer, &error);
    if (status) {
        mphip::set_free_error(error);
        return status;
    }
    const hipError_t e = mphip::launch_attention_single(static_cast<hipStream_t>(stream), q, keys, values, table,
                                                        length, layer, layers, block_tokens, heads, kv_heads, dim,
                                                        out, buffer);
    if (e != hipSuccess) {
        mphip::set_free_error(std::string("paged attention launch: ") + hipGetErrorString(e));
        return MP_DEVICE_ERROR;
    }
    return MP_OK;
}
