// Library context, error reporting, memory and the seeded generator.
#include <cmath>
#include <cstring>
#include <mutex>
#include <string>

#include "common.h"

namespace ms {

static thread_local std::string g_err;
static Ctx g_ctx;

void set_error(const std::string &msg) { g_err = msg; }
int fail(int code, const std::string &msg) {
  g_err = msg;
  return code;
}
Ctx &ctx() { return g_ctx; }
int require_init() {
  if (g_ctx.device < 0) return fail(MS_E_STATE, "ms_init() has not been called");
  return MS_OK;
}

int scratch(size_t bytes, void **out) {
  if (bytes > g_ctx.scratch_bytes) {
    if (g_ctx.scratch) {
      MS_HIP_TRY(hipStreamSynchronize(g_ctx.stream));
      MS_HIP_TRY(hipFree(g_ctx.scratch));
      g_ctx.scratch = nullptr;
      g_ctx.scratch_bytes = 0;
    }
    const size_t sz = bytes < (1u << 20) ? (1u << 20) : bytes;
    MS_HIP_TRY(hipMalloc(&g_ctx.scratch, sz));
    g_ctx.scratch_bytes = sz;
  }
  *out = g_ctx.scratch;
  return MS_OK;
}

__global__ void k_fill_random(uint8_t *dst, size_t n, uint64_t seed, uint64_t stream,
                              int balanced) {
  const size_t w = (size_t)blockIdx.x * kBlock + threadIdx.x;
  const size_t i0 = w * 8;
  if (i0 >= n) return;
  uint64_t r = rand_word(seed, stream, w);
  if (balanced) r = balance_q4_word(r);
  if (i0 + 8 <= n && ((reinterpret_cast<uintptr_t>(dst) & 7) == 0)) {
    *reinterpret_cast<uint64_t *>(dst + i0) = r;
  } else {
    for (int b = 0; b < 8 && i0 + b < n; ++b) dst[i0 + b] = (uint8_t)(r >> (8 * b));
  }
}

}  // namespace ms

using namespace ms;

extern "C" const char *ms_last_error(void) { return g_err.c_str(); }

extern "C" int ms_init(int device) {
  if (g_ctx.device >= 0) {
    if (g_ctx.device == device) return MS_OK;
    return fail(MS_E_STATE, "ms_init: already initialised on another device");
  }
  int n = 0;
  MS_HIP_TRY(hipGetDeviceCount(&n));
  MS_CHECK_ARG(device >= 0 && device < n, "ms_init: no such device");
  MS_HIP_TRY(hipSetDevice(device));
  hipDeviceProp_t prop;
  MS_HIP_TRY(hipGetDeviceProperties(&prop, device));
  if (std::strncmp(prop.gcnArchName, "gfx950", 6) != 0)
    return fail(MS_E_STATE, std::string("ms_init: built for gfx950, device is ") +
                                prop.gcnArchName);
  if (int rc = q4_noalloc_init(device)) return rc;
  MS_HIP_TRY(hipStreamCreateWithFlags(&g_ctx.stream, hipStreamNonBlocking));
  MS_HIP_TRY(hipStreamCreateWithFlags(&g_ctx.copy_stream, hipStreamNonBlocking));
  g_ctx.n_cu = prop.multiProcessorCount;
  g_ctx.device = device;
  return MS_OK;
}

extern "C" int ms_shutdown(void) {
  if (g_ctx.device < 0) return MS_OK;
  (void)hipStreamSynchronize(g_ctx.stream);
  if (g_ctx.scratch) (void)hipFree(g_ctx.scratch);
  (void)hipStreamDestroy(g_ctx.stream);
  (void)hipStreamDestroy(g_ctx.copy_stream);
  g_ctx = Ctx{};
  return MS_OK;
}

extern "C" int ms_synchronize(void) {
  if (int rc = require_init()) return rc;
  MS_HIP_TRY(hipStreamSynchronize(g_ctx.stream));
  return MS_OK;
}

extern "C" int ms_device_info(char *name, size_t name_len, int *n_cu, size_t *hbm_bytes) {
  if (int rc = require_init()) return rc;
  hipDeviceProp_t prop;
  MS_HIP_TRY(hipGetDeviceProperties(&prop, g_ctx.device));
  if (name && name_len) {
    char dev[256] = {0};
    if (prop.name[0])
      std::snprintf(dev, sizeof dev, "%s", prop.name);
    else if (hipDeviceGetName(dev, sizeof dev, g_ctx.device) != hipSuccess)
      dev[0] = 0;
    if (dev[0])
      std::snprintf(name, name_len, "%s (%s)", dev, prop.gcnArchName);
    else
      std::snprintf(name, name_len, "%s", prop.gcnArchName);
  }
  if (n_cu) *n_cu = prop.multiProcessorCount;
  if (hbm_bytes) *hbm_bytes = prop.totalGlobalMem;
  return MS_OK;
}

extern "C" int ms_malloc(void **d_ptr, size_t bytes) {
  if (int rc = require_init()) return rc;
  MS_CHECK_ARG(d_ptr, "ms_malloc: null out pointer");
  if (hipMalloc(d_ptr, bytes ? bytes : 1) != hipSuccess)
    return fail(MS_E_NOMEM, "ms_malloc: out of device memory");
  return MS_OK;
}
extern "C" int ms_free(void *d_ptr) {
  if (int rc = require_init()) return rc;
  if (!d_ptr) return MS_OK;
  MS_HIP_TRY(hipStreamSynchronize(g_ctx.stream));
  MS_HIP_TRY(hipFree(d_ptr));
  return MS_OK;
}
extern "C" int ms_memcpy_h2d(void *d_dst, const void *h_src, size_t bytes) {
  if (int rc = require_init()) return rc;
  MS_HIP_TRY(hipMemcpyAsync(d_dst, h_src, bytes, hipMemcpyHostToDevice, g_ctx.stream));
  MS_HIP_TRY(hipStreamSynchronize(g_ctx.stream));
  return MS_OK;
}
extern "C" int ms_memcpy_d2h(void *h_dst, const void *d_src, size_t bytes) {
  if (int rc = require_init()) return rc;
  MS_HIP_TRY(hipMemcpyAsync(h_dst, d_src, bytes, hipMemcpyDeviceToHost, g_ctx.stream));
  MS_HIP_TRY(hipStreamSynchronize(g_ctx.stream));
  return MS_OK;
}
extern "C" int ms_memcpy_d2d(void *d_dst, const void *d_src, size_t bytes) {
  if (int rc = require_init()) return rc;
  MS_HIP_TRY(hipMemcpyAsync(d_dst, d_src, bytes, hipMemcpyDeviceToDevice, g_ctx.stream));
  return MS_OK;
}
extern "C" int ms_memset(void *d_dst, int value, size_t bytes) {
  if (int rc = require_init()) return rc;
  MS_HIP_TRY(hipMemsetAsync(d_dst, value, bytes, g_ctx.stream));
  return MS_OK;
}
extern "C" int ms_host_alloc(void **h_ptr, size_t bytes) {
  if (int rc = require_init()) return rc;
  if (hipHostMalloc(h_ptr, bytes ? bytes : 1, hipHostMallocDefault) != hipSuccess)
    return fail(MS_E_NOMEM, "ms_host_alloc: pinned allocation failed");
  return MS_OK;
}
extern "C" int ms_host_free(void *h_ptr) {
  if (int rc = require_init()) return rc;
  if (!h_ptr) return MS_OK;
  MS_HIP_TRY(hipHostFree(h_ptr));
  return MS_OK;
}

extern "C" int ms_fill_random_q4(uint8_t *d_dst, size_t n, uint64_t seed, uint64_t stream,
                                 int balanced) {
  if (int rc = require_init()) return rc;
  const size_t words = (n + 7) / 8;
  hipLaunchKernelGGL(k_fill_random, dim3(cdiv((long)words, kBlock)), dim3(kBlock), 0,
                     g_ctx.stream, d_dst, n, seed, stream, balanced ? 1 : 0);
  MS_HIP_TRY(hipGetLastError());
  return MS_OK;
}

extern "C" int ms_fill_random_u8(uint8_t *d_dst, size_t n, uint64_t seed, uint64_t stream) {
  return ms_fill_random_q4(d_dst, n, seed, stream, 0);
}

extern "C" void ms_host_fill_random_q4(uint8_t *h_dst, size_t n, uint64_t seed,
                                       uint64_t stream, int balanced) {
  const size_t words = (n + 7) / 8;
  for (size_t w = 0; w < words; ++w) {
    uint64_t r = rand_word(seed, stream, w);
    if (balanced) r = balance_q4_word(r);
    const size_t i0 = w * 8;
    if (i0 + 8 <= n) {
      std::memcpy(h_dst + i0, &r, 8);  // little-endian host, same as the device
    } else {
      for (int b = 0; b < 8 && i0 + b < n; ++b) h_dst[i0 + b] = (uint8_t)(r >> (8 * b));
    }
  }
}

extern "C" void ms_host_fill_random_u8(uint8_t *h_dst, size_t n, uint64_t seed,
                                       uint64_t stream) {
  ms_host_fill_random_q4(h_dst, n, seed, stream, 0);
}

extern "C" float ms_host_uniform(uint64_t seed, uint64_t stream, uint64_t index, float lo,
                                 float hi) {
  const uint64_t r = rand_word(seed, stream, index);
  const double u = (double)(r >> 40) / (double)(1ull << 24);  // [0,1), 24 bits
  return (float)(lo + (hi - lo) * u);
}

extern "C" void ms_host_fill_normal(float *h_dst, size_t n, uint64_t seed, uint64_t stream) {
  for (size_t i = 0; i < n; i += 2) {
    const uint64_t r = rand_word(seed, stream, i / 2);
    const double u1 = ((double)(r >> 40) + 1.0) / (double)(1ull << 24);  // (0,1]
    const double u2 = (double)(r & 0xFFFFFFull) / (double)(1ull << 24);
    const double rad = std::sqrt(-2.0 * std::log(u1));
    h_dst[i] = (float)(rad * std::cos(2.0 * M_PI * u2));
    if (i + 1 < n) h_dst[i + 1] = (float)(rad * std::sin(2.0 * M_PI * u2));
  }
}
