// Library-wide C-ABI entry points: version, error state, device info, and the
// fp8 conversion test hook.
#include "common.h"

namespace prism {

namespace {
thread_local std::string g_last_error;
}

void set_error(const char* fmt, ...) {
  char buf[1024];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_last_error = buf;
}

void clear_error() { g_last_error.clear(); }

int check_hip(hipError_t err, const char* what) {
  if (err == hipSuccess) return PRISM_OK;
  set_error("%s: %s (%d)", what, hipGetErrorString(err), static_cast<int>(err));
  return PRISM_ERR_HIP;
}

int device_cu_count() {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return 256;
  int cus = 0;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0)
    return 256;
  return cus;
}

__global__ void __launch_bounds__(256) fp8_encode_kernel(const float* __restrict__ in,
                                                         uint32_t* __restrict__ out, int64_t n4) {
  int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
  for (; i < n4; i += stride) {
    float4 v = reinterpret_cast<const float4*>(in)[i];
    out[i] = fp8_encode4(v.x, v.y, v.z, v.w);
  }
}

}  // namespace prism

extern "C" {

int prism_abi_version(void) { return 2; }

const char* prism_last_error(void) { return prism::g_last_error.c_str(); }

int prism_device_cu_count(void) { return prism::device_cu_count(); }

int prism_preload(void) {
  prism::clear_error();
  hipFuncAttributes attr;
  if (int rc = prism::check_hip(hipFuncGetAttributes(&attr, reinterpret_cast<const void*>(&prism::fp8_encode_kernel)),
                                "prism_preload"))
    return rc;
  if (int rc = prism::preload_kv_store()) return rc;
  if (int rc = prism::preload_kv_compaction()) return rc;
  if (int rc = prism::preload_paged_prefill()) return rc;
  return prism::preload_paged_decode();
}

int prism_debug_fp8_encode(const float* in, uint8_t* out, int64_t n, void* stream) {
  prism::clear_error();
  if (n < 0 || (n % 4) != 0) {
    prism::set_error("prism_debug_fp8_encode: n must be a non-negative multiple of 4, got %lld",
                     static_cast<long long>(n));
    return PRISM_ERR_INVALID;
  }
  if (!prism::aligned(in, 16) || !prism::aligned(out, 4)) {
    prism::set_error("prism_debug_fp8_encode: input must be 16-byte and output 4-byte aligned");
    return PRISM_ERR_LAYOUT;
  }
  if (n == 0) return PRISM_OK;
  int64_t n4 = n / 4;
  int blocks = static_cast<int>(std::min<int64_t>(prism::ceil_div(n4, 256), 65536));
  hipLaunchKernelGGL(prism::fp8_encode_kernel, dim3(blocks), dim3(256), 0,
                     static_cast<hipStream_t>(stream), in, reinterpret_cast<uint32_t*>(out), n4);
  return prism::check_launch("fp8_encode_kernel launch");
}

}  // extern "C"
