// hn_expert_mlp_int4_noalloc: hn_expert_mlp_int4 for callers that cannot
// allocate device memory (code under HIP graph capture, tight serving loops,
// harnesses that forbid hipMalloc).  No counterpart in the reference.
//
// The two scratch buffers of hn_expert_mlp_int4 -- h [T, I] fp16 and the
// split-K workspace (counters in its first 2 MiB, fp32 partials after) --
// live in one file-scope device array of kScratchBytes per GPU, held until
// the process ends.  Layout: [0, kWorkBytes) workspace, [kWorkBytes,
// kScratchBytes) h.  The caller passes inputs and outputs only; nothing here
// allocates or frees.
//
// Per device, on the first call with that device current, the array's
// device address is looked up (hipGetSymbolAddress) and kept; the host
// never passes the array's name to a kernel or copy (on the host it is a
// stand-in, not a device address).  The same first call clears the counter
// region with a fill kernel (no hipMemsetAsync, so a first call under graph
// capture records a kernel node); the kernels leave the counters at zero
// after every call, so later calls need no clearing.  h and the partials are
// written before they are read in every call.
//
// Every call on a GPU shares that GPU's array: calls that overlap on one GPU
// (concurrent streams) race; calls ordered on one stream do not.
#include "hn_common.h"

#include <mutex>

extern "C" int hn_expert_mlp_int4(const void* x, const void* gq, const void* gs, const void* uq,
                                  const void* us, const void* dq, const void* ds, void* out,
                                  long T, long H, long I, long group, void* h_ws, void* work,
                                  long work_bytes, void* stream);
extern "C" long hn_skinny_workspace_bytes(int kind, long M, long N, long K, long E);

namespace {

constexpr long kWorkBytes = 16L << 20;     // split-K workspace
constexpr long kHBytes = 1L << 20;         // h [T, I] fp16
constexpr long kScratchBytes = kWorkBytes + kHBytes;
constexpr long kCounterBytes = 2L << 20;   // counter region at the workspace's start
constexpr long kMaxTokens = 16;
constexpr int kMaxDevices = 64;

__device__ __align__(256) unsigned char scratch[kScratchBytes];

__global__ void clear_words(uint32_t* p, long n) {
  for (long i = (long)blockIdx.x * blockDim.x + threadIdx.x; i < n;
       i += (long)gridDim.x * blockDim.x)
    p[i] = 0u;
}

std::mutex g_init_mu;
unsigned char* g_scratch[kMaxDevices];  // device address of `scratch`, per device

// The device address of this device's array; on the first call per device
// also clears its counter region on `s`.  nullptr after an error (message set).
unsigned char* scratch_ptr(hipStream_t s) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) {
    hn_set_error("hn_expert_mlp_int4_noalloc: hipGetDevice failed: %s", hipGetErrorString(e));
    return nullptr;
  }
  if (dev < 0 || dev >= kMaxDevices) {
    hn_set_error("hn_expert_mlp_int4_noalloc: device %d beyond the %d supported", dev,
                 kMaxDevices);
    return nullptr;
  }
  std::lock_guard<std::mutex> lock(g_init_mu);
  if (g_scratch[dev] == nullptr) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || p == nullptr) {
      hn_set_error("hn_expert_mlp_int4_noalloc: hipGetSymbolAddress failed: %s",
                   hipGetErrorString(e));
      return nullptr;
    }
    hipLaunchKernelGGL(clear_words, dim3(256), dim3(256), 0, s, (uint32_t*)p,
                       kCounterBytes / 4);
    e = hipGetLastError();
    if (e != hipSuccess) {
      hn_set_error("hn_expert_mlp_int4_noalloc: clearing the counters failed: %s",
                   hipGetErrorString(e));
      return nullptr;
    }
    g_scratch[dev] = (unsigned char*)p;
  }
  return g_scratch[dev];
}

}  // namespace

extern "C" int hn_expert_mlp_int4_noalloc(const void* x, const void* gq, const void* gs,
                                          const void* uq, const void* us, const void* dq,
                                          const void* ds, void* out, long T, long H, long I,
                                          long group, void* stream) {
  HN_ARG_CHECK(T >= 0 && T <= kMaxTokens,
               "hn_expert_mlp_int4_noalloc: T=%ld tokens, at most %ld (the static scratch "
               "is sized for decode batches)", T, kMaxTokens);
  HN_ARG_CHECK(H > 0 && I > 0 && H % 2 == 0 && I % 2 == 0,
               "hn_expert_mlp_int4_noalloc: bad dims H=%ld I=%ld", H, I);
  const long need_h = T * I * 2;
  HN_ARG_CHECK(need_h <= kHBytes,
               "hn_expert_mlp_int4_noalloc: h needs %ld bytes, the scratch holds %ld", need_h,
               kHBytes);
  const long need_w = hn_skinny_workspace_bytes(2, T, H, I, 0);
  HN_ARG_CHECK(need_w <= kWorkBytes,
               "hn_expert_mlp_int4_noalloc: the workspace needs %ld bytes, the scratch holds "
               "%ld", need_w, kWorkBytes);
  hipStream_t s = (hipStream_t)stream;
  unsigned char* p = scratch_ptr(s);
  if (p == nullptr) return -5; /* -EIO: message set */
  return hn_expert_mlp_int4(x, gq, gs, uq, us, dq, ds, out, T, H, I, group, p + kWorkBytes, p,
                            kWorkBytes, stream);
}
