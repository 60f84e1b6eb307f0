// w4a8_linear_noalloc: the dense linear for callers that cannot allocate device memory (code under
// HIP graph capture, tight serving loops, harnesses that forbid hipMalloc). It is w4a8_linear with
// its workspace (the fp8 codes and scales of x that the act-quant launch writes before the GEMM)
// taken from a fixed device array instead of the caller.
//
// The array `scratch` is a file-scope device symbol: every GPU the library runs on holds its own
// copy, at its own address, until the process ends. In host code the name `scratch` is only a
// host-side stand-in for the symbol, never a device address, so it is used for nothing but the
// hipGetSymbolAddress lookup; the device address that lookup returns (one per device, kept in
// g_scratch) is what reaches the kernels. Calls on one GPU share that GPU's array and overlapping
// calls race; nothing in it needs to start at zero (the act-quant launch writes every byte the
// GEMM reads).
#include <stdarg.h>
#include <stdio.h>

#include <mutex>

#include <hip/hip_runtime.h>

#include "../../include/w4a8_mi355x.h"

namespace w4a8 {
int set_last_error(int code, const char* msg);       // abi.hip
int64_t linear_workspace_min(int64_t M, int64_t K);  // abi.hip: the row-major part w4a8_linear accepts
}

static constexpr int64_t kScratchBytes = 64ll << 20;  // 64 MiB per device
static __device__ __align__(256) unsigned char scratch[kScratchBytes];

namespace {

constexpr int kMaxDevices = 64;

std::mutex g_mu;
void* g_scratch[kMaxDevices];  // device address of `scratch` on each device, once looked up

int failf(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
int failf(int code, const char* fmt, ...) {
  char msg[320];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(msg, sizeof msg, fmt, ap);
  va_end(ap);
  return w4a8::set_last_error(code, msg);
}

// Device address of this device's `scratch`, looked up on the first call on the device (with the
// device current); null on failure, with the reason in the library's error slot.
void* scratch_on_current_device() {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) {
    failf(3, "w4a8_linear_noalloc: no current HIP device (or device id >= %d)", kMaxDevices);
    return nullptr;
  }
  std::lock_guard<std::mutex> lock(g_mu);
  if (!g_scratch[dev]) {
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p) {
      failf(3, "w4a8_linear_noalloc: hipGetSymbolAddress(scratch) failed on device %d (%s)", dev, hipGetErrorString(e));
      return nullptr;
    }
    g_scratch[dev] = p;
  }
  return g_scratch[dev];
}

}  // namespace

extern "C" {

int64_t w4a8_linear_noalloc_max_bytes(void) { return kScratchBytes; }

int w4a8_linear_noalloc(const void* x, int x_dtype, int64_t M, int64_t K, int64_t ldx, const void* w_tile, int64_t N,
                        const void* scales, int scale_fmt, const int32_t* zeros, int wfmt, int64_t group_size,
                        void* out, int out_dtype, int64_t ldo, int silu, int kernel, void* stream) {
  // the scratch holds at least the row-major codes and scales; a prefill call that would also take
  // the tiled copy falls back to the row-major GEMM (the same results) when that does not fit
  const int64_t need = w4a8::linear_workspace_min(M, K);
  if (need < 0) return failf(1, "w4a8_linear_noalloc: bad sizes M=%lld K=%lld", (long long)M, (long long)K);
  if (need > kScratchBytes)
    return failf(1,
                 "w4a8_linear_noalloc: M=%lld x K=%lld needs %lld workspace bytes, over the %lld-byte static scratch; "
                 "call w4a8_linear with a caller workspace",
                 (long long)M, (long long)K, (long long)need, (long long)kScratchBytes);
  void* ws = scratch_on_current_device();
  if (!ws) return 3;
  return w4a8_linear(x, x_dtype, M, K, ldx, w_tile, N, scales, scale_fmt, zeros, wfmt, group_size, out, out_dtype,
                     ldo, silu, ws, kScratchBytes, kernel, stream);
}

}  // extern "C"
