// Token sampling on the device: temperature_sampling (lm_head.mojo:198-254)
// with a caller-given seed where the reference reads the clock (:246).
//
// One block of kSampleThreads threads per row of logits, three passes over
// the row, every intermediate written back in place as in the reference:
//   penalty  each id of the row's history that is below n, once per
//            occurrence: a positive logit divided by the penalty, any other
//            multiplied (:211-220).  A thread takes the first occurrence of an
//            id in the history (staged in LDS) and applies the operation as
//            many times as the id occurs, which is the reference's sequence
//            of operations on that logit.
//   greedy   temperature <= 0.01: the first index of the maximum (:222-228).
//   softmax  exp((v - max) / T), the sum, the division (:230-243).
//   draw     one LCG step of the seed (:246-248; in the model the seed of draw
//            k of sequence b is draw_seed(seed, b, k)); the first index whose
//            running sum reaches the target, else n - 1 (:250-254).  Thread t
//            owns the contiguous slice t of the row; the slices' sums are
//            added in slice order, then the slice holding the crossing is
//            walked element by element.
// The parallel sums round differently from the reference's one running sum,
// so a draw whose target lies within rounding of a slice boundary of the
// cumulative distribution may pick the neighbouring index.
#include "common.h"
#include "sample.h"

#include <cmath>

namespace ms {
namespace {

constexpr int kSampleThreads = 1024;

template <class T>
__device__ inline T sld(const T *p) {
  return *(const __attribute__((address_space(1))) T *)p;
}

// lm_head.mojo:247-248 in wrapping 64-bit arithmetic
__device__ inline float lcg_target(uint64_t seed) {
  const uint64_t lcg = (seed * 6364136223846793005ull + 1442695040888963407ull) & 0x7FFFFFFFull;
  return (float)lcg / (float)0x7FFFFFFF;
}

__global__ __launch_bounds__(kSampleThreads) void k_sample(SampleArgs a) {
  constexpr int NT = kSampleThreads;
  __shared__ int32_t hist[kSampleMaxHistory];
  __shared__ float rv[NT];
  __shared__ int ri[NT];
  const int tid = threadIdx.x, row = blockIdx.x;
  const int n = a.n;
  float *v = a.logits + (size_t)row * a.ld;

  // ---- repetition penalty
  if (a.penalty > 1.0f && a.hist) {
    const int32_t *h = a.hist + (size_t)row * a.hist_ld;
    const int nh = min(sld(a.hist_n + row), kSampleMaxHistory);
    for (int i = tid; i < nh; i += NT) hist[i] = sld(h + i);
    __syncthreads();
    for (int i = tid; i < nh; i += NT) {
      const int id = hist[i];
      if (id < 0 || id >= n) continue;
      bool first = true;
      for (int j = 0; j < i && first; ++j) first = hist[j] != id;
      if (!first) continue;
      int c = 1;
      for (int j = i + 1; j < nh; ++j) c += hist[j] == id;
      float x = v[id];
      for (int k = 0; k < c; ++k) x = x > 0.0f ? x / a.penalty : x * a.penalty;
      v[id] = x;
    }
    __syncthreads();
  }

  // ---- maximum (first index of it) over contiguous slices
  const int per = (n + NT - 1) / NT;
  const int c0 = min(n, tid * per), c1 = min(n, c0 + per);
  float lm = -INFINITY;
  int li = n;
  if (c0 < c1) {
    lm = v[c0];
    li = c0;
    for (int j = c0 + 1; j < c1; ++j)
      if (v[j] > lm) {
        lm = v[j];
        li = j;
      }
  }
  rv[tid] = lm;
  ri[tid] = li;
  __syncthreads();
  for (int s = NT / 2; s > 0; s >>= 1) {
    if (tid < s) {
      const float ov = rv[tid + s];
      const int oi = ri[tid + s];
      if (ov > rv[tid] || (ov == rv[tid] && oi < ri[tid])) {
        rv[tid] = ov;
        ri[tid] = oi;
      }
    }
    __syncthreads();
  }
  const float vmax = rv[0];
  const int imax = ri[0];
  __syncthreads();
  int result;
  if (a.temperature <= 0.01f) {
    result = imax;
  } else {
    // ---- softmax in place
    const float inv_t = 1.0f / a.temperature;
    float ls = 0.0f;
    for (int j = c0; j < c1; ++j) {
      const float e = expf((v[j] - vmax) * inv_t);
      v[j] = e;
      ls += e;
    }
    rv[tid] = ls;
    __syncthreads();
    if (tid == 0) {
      float s = 0.0f;
      for (int t = 0; t < NT; ++t) s += rv[t];
      rv[0] = s;
    }
    __syncthreads();
    const float inv_s = 1.0f / rv[0];
    __syncthreads();
    float lp = 0.0f;
    for (int j = c0; j < c1; ++j) {
      const float p = v[j] * inv_s;
      v[j] = p;
      lp += p;
    }
    rv[tid] = lp;
    __syncthreads();
    // ---- draw: slice sums in order, then the slice holding the crossing
    if (tid == 0) {
      float s = 0.0f;
      for (int t = 0; t < NT; ++t) {
        const float x = rv[t];
        rv[t] = s;
        s += x;
      }
    }
    __syncthreads();
    const uint64_t seed =
        a.step ? draw_seed(a.seed, (uint64_t)(a.seq0 + row), (uint64_t)sld(a.step)) : a.seed;
    const float target = lcg_target(seed);
    float cdf = rv[tid];
    int found = n;
    for (int j = c0; j < c1; ++j) {
      cdf += v[j];
      if (cdf >= target) {
        found = j;
        break;
      }
    }
    __syncthreads();
    ri[tid] = found;
    __syncthreads();
    for (int s = NT / 2; s > 0; s >>= 1) {
      if (tid < s) ri[tid] = min(ri[tid], ri[tid + s]);
      __syncthreads();
    }
    result = ri[0] < n ? ri[0] : n - 1;
  }
  if (tid == 0) {
    if (a.ids_out) a.ids_out[row] = result;
    if (a.tok_state) a.tok_state[row] = result;
    if (a.hist_append) {
      // the sampled id joins the row's history for the next draw
      const int nh = sld(a.hist_n + row);
      if (nh < a.hist_cap) a.hist[(size_t)row * a.hist_ld + nh] = result;
      a.hist_n[row] = min(nh + 1, a.hist_cap);
    }
  }
}

}  // namespace

int launch_sample(const SampleArgs &a, int rows, hipStream_t st) {
  MS_CHECK_ARG(a.logits && a.n >= 1 && a.ld >= a.n && rows >= 1, "sample: bad logits");
  MS_CHECK_ARG(a.temperature == a.temperature && a.penalty == a.penalty,
               "sample: temperature and penalty must be numbers");
  MS_CHECK_ARG(!(a.penalty > 1.0f) || (a.hist && a.hist_n),
               "sample: a penalty needs the token history");
  hipLaunchKernelGGL(k_sample, dim3(rows), dim3(kSampleThreads), 0, st, a);
  MS_HIP_TRY(hipGetLastError());
  return MS_OK;
}

}  // namespace ms

using namespace ms;

extern "C" int ms_sample(float *d_logits, int vocab, float temperature,
                         const int32_t *d_generated, int n_generated, float penalty,
                         uint64_t seed, int32_t *h_id) {
  if (int rc = require_init()) return rc;
  MS_CHECK_ARG(d_logits && vocab >= 1 && h_id, "sample: null argument or empty vocab");
  MS_CHECK_ARG(n_generated >= 0 && n_generated <= kSampleMaxHistory,
               "sample: history longer than 8192 ids");
  MS_CHECK_ARG(n_generated == 0 || d_generated, "sample: history pointer missing");
  hipStream_t st = ctx().stream;
  void *buf = nullptr;
  if (int rc = scratch(64, &buf)) return rc;
  // (a single draw: the seed goes to the LCG step as given)
  int32_t *d_n = static_cast<int32_t *>(buf), *d_id = d_n + 4;
  MS_HIP_TRY(hipMemcpyAsync(d_n, &n_generated, 4, hipMemcpyHostToDevice, st));
  SampleArgs a{};
  a.logits = d_logits;
  a.n = vocab;
  a.ld = vocab;
  a.temperature = temperature;
  a.penalty = penalty;
  a.hist = const_cast<int32_t *>(d_generated);
  a.hist_ld = n_generated;
  a.hist_n = d_n;
  a.seed = seed;
  a.ids_out = d_id;
  if (int rc = launch_sample(a, 1, st)) return rc;
  MS_HIP_TRY(hipMemcpyAsync(h_id, d_id, 4, hipMemcpyDeviceToHost, st));
  MS_HIP_TRY(hipStreamSynchronize(st));
  return MS_OK;
}

extern "C" uint64_t ms_sample_seed(uint64_t seed, int seq, uint64_t draw) {
  return draw_seed(seed, (uint64_t)seq, draw);
}
