// Token choice with no device allocation: esp_pick_noalloc's scratch is one
// fixed file-scope device array instead of the KV handle's grow-on-demand
// buffers. Each GPU holds its own copy of the array from the moment the
// library's code object is loaded there until the process ends; every call
// on that GPU reuses it, so calls that overlap on one GPU race.
//
// Layout of one call's use of `scratch` (offsets 256-byte aligned):
//   [pick scratch of pick_layout(n, V), only when samplers are given]
//   [n u64 advanced sampler states]
//   [n u8 flags, only when the caller passes no flags buffer]
#include <mutex>

#include "common.hpp"

namespace esp {

constexpr size_t kFixedScratchBytes = ESP_PICK_NOALLOC_SCRATCH_BYTES;

static __device__ __align__(256) unsigned char scratch[kFixedScratchBytes];

namespace {

constexpr int kMaxDevices = 64;
std::mutex g_mu;
void *g_addr[kMaxDevices] = {};

inline size_t align256(size_t n) { return (n + 255) / 256 * 256; }

// Restores the caller's current device on scope exit.
struct DeviceScope {
    int prev = -1;
    explicit DeviceScope(int dev) {
        ESP_HIP(hipGetDevice(&prev));
        if (prev != dev) ESP_HIP(hipSetDevice(dev));
    }
    ~DeviceScope() {
        int cur = -1;
        if (hipGetDevice(&cur) == hipSuccess && cur != prev) (void)hipSetDevice(prev);
    }
};

}  // namespace

// Device address of `scratch` on `device`, looked up once per device with
// that device current. In host code `scratch` names a host-side stand-in,
// so kernels and copies must only ever see this address.
static void *fixed_scratch(int device) {
    if (device < 0 || device >= kMaxDevices) fail(ESP_BACKEND, "pick_noalloc: device id out of range");
    std::lock_guard<std::mutex> lk(g_mu);
    if (!g_addr[device]) {
        DeviceScope ds(device);
        void *p = nullptr;
        hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !p)
            fail(ESP_BACKEND, std::string("pick_noalloc: hipGetSymbolAddress(scratch): ") +
                                  hipGetErrorString(e));
        g_addr[device] = p;
    }
    return g_addr[device];
}

size_t pick_fixed_scratch_need(int n, int V, bool sampled, bool own_flags) {
    size_t need = sampled ? align256(pick_scratch_bytes(n, V)) : 0;
    need += align256((size_t)n * 8);
    if (!own_flags) need += align256((size_t)n);
    return need;
}

// esp_pick's host commit of advanced states (a sampled row keeps its new
// state unless it had no eligible token), done on the device.
__global__ void pick_commit_states_k(esp_sampler *smp, const uint64_t *state,
                                     const uint8_t *flags, int n) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    if (smp[i].temperature > 0.f && !(flags[i] & ESP_PICK_NO_ELIGIBLE)) smp[i].state = state[i];
}

void launch_pick_fixed(int device, const float *logits, int n, int V, const uint32_t *allowed_dev,
                       esp_sampler *samplers_dev, uint32_t *ids_dev, uint8_t *flags_dev,
                       hipStream_t s) {
    const bool sampled = samplers_dev != nullptr;
    const size_t need = pick_fixed_scratch_need(n, V, sampled, flags_dev != nullptr);
    if (need > kFixedScratchBytes)
        fail(ESP_INVALID_REQUEST,
             "pick_noalloc: " + std::to_string(n) + " rows over a vocabulary of " +
                 std::to_string(V) + " need " + std::to_string(need) +
                 " bytes of scratch, above the fixed " + std::to_string(kFixedScratchBytes));
    char *base = (char *)fixed_scratch(device);
    size_t off = 0;
    PickArgs a{};
    a.logits = logits;
    a.n = n;
    a.V = V;
    a.allowed = allowed_dev;
    a.samplers = samplers_dev;
    a.ids_out = ids_dev;
    if (sampled) {
        a.scratch = base;
        a.scratch_bytes = pick_scratch_bytes(n, V);
        off = align256(a.scratch_bytes);
    }
    a.state_out = (uint64_t *)(base + off);
    off += align256((size_t)n * 8);
    a.flags_out = flags_dev ? flags_dev : (uint8_t *)(base + off);
    launch_pick(a, s);
    if (sampled)
        pick_commit_states_k<<<(n + 255) / 256, 256, 0, s>>>(samplers_dev, a.state_out,
                                                              a.flags_out, n);
    ESP_HIP(hipGetLastError());
}

}  // namespace esp
