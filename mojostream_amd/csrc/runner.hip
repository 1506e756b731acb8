// ModelRunner (loader.mojo:47-144): one square Q4 matrix per layer, read from
// <base>/layer_<i>.bin ([f32 scale][N * N/2 row-major Q4 bytes], the
// "row-major" layer files of create_fake_model.py:126-140) into one of two HBM
// slots, and C += A . deq(W) on the active slot.
//
// The reference measures a load and a compute one after the other and models
// the overlap analytically (wait = max(0, load_next - compute)).  Here the
// overlap is real: while layer i computes on the library stream, the host
// reads layer i+1's file, repacks it into pinned memory and copies it into
// the other slot on the copy stream.  Compute of layer i+1 waits for that
// copy with a stream event, and the wait is the measured idle time of the
// compute stream between the two layers.
#include <chrono>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <string>
#include <vector>

#include "common.h"

struct ms_runner {
  std::string base;
  int n_layers = 0, N = 0;
  size_t bytes = 0;              // N * N / 2
  uint8_t *slot[2] = {};         // device, panel layout
  float scale[2] = {0.1f, 0.1f};
  uint8_t *pin[2] = {};          // pinned staging of the packed bytes
  std::vector<uint8_t> file;     // one layer file
  hipEvent_t copied[2] = {};     // the copy into slot s has finished
  hipEvent_t freed[2] = {};      // the last compute reading slot s has finished
  int active = 0;
};

namespace ms {

static double now_ms() {
  return std::chrono::duration<double, std::milli>(
             std::chrono::steady_clock::now().time_since_epoch())
      .count();
}

// Reads layer idx's file, repacks it into pin[s] and queues its copy into
// slot s on the copy stream after the slot's last reader.  Returns the host
// time (file read + repack) in *host_ms; e0/e1 (optional) bracket the copy.
static int runner_stage(ms_runner *r, int s, int idx, double *host_ms, hipEvent_t e0,
                        hipEvent_t e1) {
  MS_CHECK_ARG(s == 0 || s == 1, "runner: slot must be 0 or 1");
  MS_CHECK_ARG(idx >= 0 && idx < r->n_layers, "runner: layer index out of range");
  const double t0 = now_ms();
  const std::string path = r->base + "/layer_" + std::to_string(idx) + ".bin";
  FILE *f = std::fopen(path.c_str(), "rb");
  if (!f) return fail(MS_E_IO, "runner: cannot open " + path);
  r->file.resize(4 + r->bytes);
  const size_t got = std::fread(r->file.data(), 1, r->file.size(), f);
  std::fclose(f);
  if (got != r->file.size())
    return fail(MS_E_IO, "runner: " + path + " holds " + std::to_string(got) +
                             " bytes, expected " + std::to_string(r->file.size()));
  float sc;
  std::memcpy(&sc, r->file.data(), 4);
  MS_CHECK_ARG(std::isfinite(sc), "runner: non-finite scale in " + path);
  // the pinned buffer may still feed the slot's previous copy
  MS_HIP_TRY(hipEventSynchronize(r->copied[s]));
  if (int rc = ms_host_q4_pack(r->pin[s], r->file.data() + 4, r->N, r->N)) return rc;
  r->scale[s] = sc;
  *host_ms = now_ms() - t0;
  hipStream_t cs = ctx().copy_stream;
  MS_HIP_TRY(hipStreamWaitEvent(cs, r->freed[s], 0));
  if (e0) MS_HIP_TRY(hipEventRecord(e0, cs));
  MS_HIP_TRY(hipMemcpyAsync(r->slot[s], r->pin[s], r->bytes, hipMemcpyHostToDevice, cs));
  if (e1) MS_HIP_TRY(hipEventRecord(e1, cs));
  MS_HIP_TRY(hipEventRecord(r->copied[s], cs));
  return MS_OK;
}

// C += A . deq(W_active) on the library stream once the active slot's copy
// has landed; e0/e1 bracket the product.
static int runner_enqueue_compute(ms_runner *r, float *d_C, const float *d_A, int M,
                                  hipEvent_t e0, hipEvent_t e1) {
  hipStream_t st = ctx().stream;
  const int s = r->active;
  MS_HIP_TRY(hipStreamWaitEvent(st, r->copied[s], 0));
  MS_HIP_TRY(hipEventRecord(e0, st));
  if (int rc = ms_q4_matmul(d_C, d_A, r->slot[s], M, r->N, r->N, r->scale[s], 1)) return rc;
  MS_HIP_TRY(hipEventRecord(e1, st));
  MS_HIP_TRY(hipEventRecord(r->freed[s], st));
  return MS_OK;
}

static float elapsed(hipEvent_t a, hipEvent_t b) {
  float v = 0.f;
  (void)hipEventElapsedTime(&v, a, b);
  return v;
}

}  // namespace ms

using namespace ms;

extern "C" int ms_runner_create(const char *base_path, int n_layers, int N, ms_runner **out) {
  if (int rc = require_init()) return rc;
  MS_CHECK_ARG(base_path && out, "runner_create: null argument");
  MS_CHECK_ARG(n_layers >= 1, "runner_create: n_layers must be >= 1");
  MS_CHECK_ARG(N > 0 && N % 128 == 0, "runner_create: N must be a positive multiple of 128");
  auto *r = new ms_runner();
  r->base = base_path;
  r->n_layers = n_layers;
  r->N = N;
  r->bytes = (size_t)N * N / 2;
  int rc = MS_OK;
  for (int s = 0; s < 2 && rc == MS_OK; ++s) {
    if (hipMalloc(&r->slot[s], r->bytes) != hipSuccess ||
        hipHostMalloc(&r->pin[s], r->bytes, hipHostMallocDefault) != hipSuccess)
      rc = fail(MS_E_NOMEM, "runner_create: slot allocation failed");
    else if (hipEventCreateWithFlags(&r->copied[s], hipEventDisableTiming) != hipSuccess ||
             hipEventCreateWithFlags(&r->freed[s], hipEventDisableTiming) != hipSuccess)
      rc = fail(MS_E_HIP, "runner_create: event creation failed");
  }
  if (rc == MS_OK) {
    // both slots start free and loaded with nothing
    for (int s = 0; s < 2; ++s) {
      (void)hipEventRecord(r->copied[s], ctx().copy_stream);
      (void)hipEventRecord(r->freed[s], ctx().stream);
    }
    *out = r;
    return MS_OK;
  }
  for (int s = 0; s < 2; ++s) {
    if (r->slot[s]) (void)hipFree(r->slot[s]);
    if (r->pin[s]) (void)hipHostFree(r->pin[s]);
    if (r->copied[s]) (void)hipEventDestroy(r->copied[s]);
    if (r->freed[s]) (void)hipEventDestroy(r->freed[s]);
  }
  delete r;
  return rc;
}

extern "C" int ms_runner_destroy(ms_runner *r) {
  if (!r) return MS_OK;
  (void)hipStreamSynchronize(ctx().stream);
  (void)hipStreamSynchronize(ctx().copy_stream);
  for (int s = 0; s < 2; ++s) {
    (void)hipFree(r->slot[s]);
    (void)hipHostFree(r->pin[s]);
    (void)hipEventDestroy(r->copied[s]);
    (void)hipEventDestroy(r->freed[s]);
  }
  delete r;
  return MS_OK;
}

extern "C" int ms_runner_load_into_slot(ms_runner *r, int slot, int idx, double *load_ms) {
  if (int rc = require_init()) return rc;
  MS_CHECK_ARG(r, "runner: null runner");
  const double t0 = now_ms();
  double host = 0.0;
  if (int rc = runner_stage(r, slot, idx, &host, nullptr, nullptr)) return rc;
  MS_HIP_TRY(hipEventSynchronize(r->copied[slot]));
  if (load_ms) *load_ms = now_ms() - t0;
  return MS_OK;
}

extern "C" int ms_runner_set_active(ms_runner *r, int slot) {
  MS_CHECK_ARG(r && (slot == 0 || slot == 1), "runner: slot must be 0 or 1");
  r->active = slot;
  return MS_OK;
}

extern "C" int ms_runner_active(const ms_runner *r, int *slot) {
  MS_CHECK_ARG(r && slot, "runner: null argument");
  *slot = r->active;
  return MS_OK;
}

extern "C" int ms_runner_compute_active(ms_runner *r, float *d_C, const float *d_A, int M,
                                        double *compute_ms) {
  if (int rc = require_init()) return rc;
  MS_CHECK_ARG(r && d_C && d_A && M >= 1, "runner_compute_active: bad arguments");
  hipEvent_t e0, e1;
  MS_HIP_TRY(hipEventCreate(&e0));
  MS_HIP_TRY(hipEventCreate(&e1));
  int rc = runner_enqueue_compute(r, d_C, d_A, M, e0, e1);
  if (rc == MS_OK && hipEventSynchronize(e1) != hipSuccess)
    rc = fail(MS_E_HIP, "runner_compute_active: synchronize failed");
  if (rc == MS_OK && compute_ms) *compute_ms = elapsed(e0, e1);
  (void)hipEventDestroy(e0);
  (void)hipEventDestroy(e1);
  return rc;
}

extern "C" int ms_runner_run_pipeline(ms_runner *r, float *d_C, const float *d_A, int M,
                                      ms_layer_stats *stats, float *d_taps) {
  if (int rc = require_init()) return rc;
  MS_CHECK_ARG(r && d_C && d_A && M >= 1 && stats, "runner_run_pipeline: bad arguments");
  hipStream_t st = ctx().stream;
  const int n = r->n_layers;
  const size_t c_bytes = (size_t)M * r->N * 4;
  // layer 0 cold: nothing to overlap with (loader.mojo:119-121)
  double host0 = 0.0;
  if (int rc = runner_stage(r, 0, 0, &host0, nullptr, nullptr)) return rc;
  r->active = 0;
  // per layer: compute start/end, end of the zeroing, copy start/end of the
  // load that follows it, host time of that load
  std::vector<hipEvent_t> cs(n), ce(n), ze(n), l0(n), l1(n);
  std::vector<double> host(n, 0.0);
  std::vector<hipEvent_t> all;
  int rc = MS_OK;
  auto mk = [&](hipEvent_t *e) {
    if (hipEventCreate(e) != hipSuccess) return fail(MS_E_HIP, "runner: event creation failed");
    all.push_back(*e);
    return MS_OK;
  };
  for (int i = 0; i < n && rc == MS_OK; ++i) {
    if ((rc = mk(&cs[i])) || (rc = mk(&ce[i])) || (rc = mk(&ze[i]))) break;
    if ((rc = runner_enqueue_compute(r, d_C, d_A, M, cs[i], ce[i]))) break;
    if (d_taps && hipMemcpyAsync(d_taps + (size_t)i * M * r->N, d_C, c_bytes,
                                 hipMemcpyDeviceToDevice, st) != hipSuccess) {
      rc = fail(MS_E_HIP, "runner: tap copy failed");
      break;
    }
    // C.zero() before the next layer (loader.mojo:141)
    if (hipMemsetAsync(d_C, 0, c_bytes, st) != hipSuccess ||
        hipEventRecord(ze[i], st) != hipSuccess) {
      rc = fail(MS_E_HIP, "runner: zeroing failed");
      break;
    }
    if (i + 1 < n) {
      // the next layer into the other slot while this one computes
      if ((rc = mk(&l0[i])) || (rc = mk(&l1[i]))) break;
      if ((rc = runner_stage(r, 1 - r->active, i + 1, &host[i], l0[i], l1[i]))) break;
    }
    r->active = 1 - r->active;
  }
  if (hipStreamSynchronize(st) != hipSuccess || hipStreamSynchronize(ctx().copy_stream) != hipSuccess)
    rc = rc ? rc : fail(MS_E_HIP, "runner: synchronize failed");
  if (rc == MS_OK) {
    for (int i = 0; i < n; ++i) {
      stats[i].compute_ms = elapsed(cs[i], ce[i]);
      stats[i].load_ms = i + 1 < n ? host[i] + elapsed(l0[i], l1[i]) : 0.0;
      // idle time of the compute stream before the next layer (its copy, or
      // the host still reading its file)
      const double w = i + 1 < n ? elapsed(ze[i], cs[i + 1]) : 0.0;
      stats[i].wait_ms = w > 0.0 ? w : 0.0;
    }
  }
  for (auto e : all) (void)hipEventDestroy(e);
  return rc;
}
