// Internal helpers shared by the HIP translation units of libms_gpu.so.
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>
#include <string>

#include "../../include/ms_gpu.h"

namespace ms {

// ---- error handling ---------------------------------------------------------
void set_error(const std::string &msg);
int fail(int code, const std::string &msg);
#define MS_HIP_TRY(expr)                                                        \
  do {                                                                          \
    hipError_t _e = (expr);                                                     \
    if (_e != hipSuccess)                                                       \
      return ::ms::fail(MS_E_HIP, std::string(#expr) + ": " +                   \
                                      hipGetErrorString(_e));                   \
  } while (0)
#define MS_CHECK_ARG(cond, msg)                                                 \
  do {                                                                          \
    if (!(cond)) return ::ms::fail(MS_E_INVALID, msg);                          \
  } while (0)

// Library state: one device, one stream (all launches are ordered on it).
struct Ctx {
  int device = -1;
  hipStream_t stream = nullptr;
  hipStream_t copy_stream = nullptr;  // streaming-mode weight uploads
  int n_cu = 0;
  void *scratch = nullptr;  // kernel-level entry points' temporary buffer
  size_t scratch_bytes = 0;
};
Ctx &ctx();
int require_init();
// Grows the kernel-level scratch buffer (eager use only, never under capture).
int scratch(size_t bytes, void **out);
// Device address of the no-allocation scratch array on `device` (the current
// device), taken once (q4.hip); called by ms_init.
int q4_noalloc_init(int device);

// ---- vector types -------------------------------------------------------------
typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
typedef float float4_t __attribute__((ext_vector_type(4)));

// ---- seeded generator (identical on host and device) -----------------------
__host__ __device__ inline uint64_t mix64(uint64_t z) {
  z += 0x9E3779B97F4A7C15ull;
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}
__host__ __device__ inline uint64_t rand_word(uint64_t seed, uint64_t stream,
                                              uint64_t i) {
  return mix64(mix64(seed ^ mix64(stream)) + i);
}
// Balanced Q4 bytes: every zero nibble of the word becomes 8, so a nibble is
// 1..15 (8 twice as often) with mean 8, the zero point: zero-mean weights.
__host__ __device__ inline uint64_t balance_q4_word(uint64_t r) {
  uint64_t t = r | (r >> 1);
  t |= t >> 2;  // bit 4i: OR of the four bits of nibble i
  return r | ((~t & 0x1111111111111111ull) << 3);
}

// ---- Q4 panel layout ---------------------------------------------------------
// A [K][N] Q4 matrix is stored as N/16 column panels of 16 columns; panel nb
// holds K/128 super-tiles of 1 KiB.  Super-tile G of panel nb covers rows
// 128G..128G+127; lane l (0..63) owns 16 bytes at offset 16*l holding the 32
// nibbles of column 16*nb + (l%16), rows 128G + 32*(l/16) + 0..31.  Dword t
// (0..3) of those 16 bytes covers rows +8t..+8t+7; row offset e (0..7) sits in
// nibble q(e) = (e>>1) + 4*(e&1).  Dwords 2h and 2h+1 are the B operand of
// MFMA h of the super-tile for v_mfma_i32_16x16x64_i8 (B[k][j]: lane
// j + 16*(k/16), byte k%16): their low nibbles and their high nibbles, each
// masked to bytes, give rows {0,4,1,5} / {2,6,3,7} of each 8-row group, an
// order the activation operand is stored in to match.
constexpr int kPanelCols = 16;
// Threads per block of the simple 1-D kernels.  Device code uses this
// constant rather than blockDim, whose value is loaded from the dispatch packet.
constexpr int kBlock = 256;

constexpr int kSuperK = 128;
__host__ __device__ inline size_t panel_offset(int K, int nb, int G, int lane) {
  return (size_t)nb * (size_t)K * 8 + (size_t)G * 1024 + (size_t)lane * 16;
}
// Byte/nibble of logical (k, n) inside the panel layout.
__host__ __device__ inline void panel_locate(int K, int k, int n, size_t *byte,
                                             int *hi_nibble) {
  const int nb = n / 16, j = n % 16, G = k / 128, r = k % 128;
  const int g = r / 32, t = (r % 32) / 8, e = r % 8;
  const int lane = j + 16 * g;
  const int q = (e >> 1) + 4 * (e & 1);
  *byte = panel_offset(K, nb, G, lane) + (size_t)t * 4 + (size_t)(q >> 1);
  *hi_nibble = q & 1;
}

// ---- activation hi/lo split -----------------------------------------------------
// x ~= hi + lo with hi = fp16(x), lo = fp16(x - hi): relative error ~2^-22
// (inputs are pre-scaled by a power of two so |x| stays inside fp16 range).
__device__ inline void split_hi_lo(float x, _Float16 *hi, _Float16 *lo) {
  const _Float16 h = (_Float16)x;
  *hi = h;
  *lo = (_Float16)(x - (float)h);
}

// ---- misc -------------------------------------------------------------------------
inline int cdiv(long a, long b) { return (int)((a + b - 1) / b); }

}  // namespace ms
