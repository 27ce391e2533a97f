// Workspace placement across the HBM regions of the device.
//
// Measured on MI355X (288 GB): device memory falls into regions of about
// 96 GB of physical address space, and the driver fills them in order.  Two
// buffers written at the same time run at about 5.5 TB/s together when they
// lie in one region and at about 6.8 TB/s when they lie in two (random 8 KB
// rows, non-temporal stores; one buffer alone about 5.4 TB/s).  The UVU
// backward writes its weight gradient and its per-edge gx messages together:
// with the message workspace in another region than the gradient, the
// config-2 backward takes 8.6-8.9 instead of 9.7 ms.
//
// luna_placed_alloc allocates a buffer outside the regions of a given buffer
// (or, without one, of a fresh reference allocation).  Which region an
// allocation lands in is only known by measurement: windows of each candidate
// are probed by writing 1 GB of the window and 1 GB of the reference at the
// same time (rows in a scrambled order), against the same write pair within
// the reference.  Candidates whose windows mostly share the given buffer's
// regions are held (so the allocator moves on) and released once one that
// does not is found, or when the spacer budget or free memory runs out; then
// the least overlapping candidate is returned and *moved is 0.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdio>
#include <cstdlib>
#include <vector>

#include "../../include/lunaeq_amd.h"
#include "common.h"

namespace {

constexpr size_t kProbeBytes = 1ull << 30;
constexpr size_t kRowBytes = 8192;
// Probe time ratio below which two windows are in different regions: across
// regions 0.75-0.80 was measured, within one region 0.90-1.10 (1 GB windows
// at different offsets of one allocation; 256 MB windows vary by +-12 %).
constexpr double kOtherRegion = 0.85;

typedef float float4_ __attribute__((ext_vector_type(4)));

// Workgroup b writes row (b * 40503) mod rows of a and of b (rows is a power
// of two and the multiplier odd, so every row is written once).
__global__ void __launch_bounds__(256) luna_probe_pair_write(float4_* a, float4_* b, unsigned rows) {
  const size_t row = ((size_t)blockIdx.x * 40503u) & (rows - 1);
  float4_* pa = a + row * (kRowBytes / 16);
  float4_* pb = b + row * (kRowBytes / 16);
  const float4_ v = {1.0f, 2.0f, 3.0f, 4.0f};
  for (unsigned i = threadIdx.x; i < kRowBytes / 16; i += 256) {
    __builtin_nontemporal_store(v, pa + i);
    __builtin_nontemporal_store(v, pb + i);
  }
}

// Best of three: milliseconds to write kProbeBytes of a and of b together.
float pair_write_ms(void* a, void* b, hipStream_t stream) {
  const unsigned rows = (unsigned)(kProbeBytes / kRowBytes);
  hipEvent_t start, stop;
  luna::check_hip(hipEventCreate(&start), "hipEventCreate");
  luna::check_hip(hipEventCreate(&stop), "hipEventCreate");
  float best = 1e30f;
  for (int r = 0; r < 3; ++r) {
    luna::check_hip(hipEventRecord(start, stream), "hipEventRecord");
    hipLaunchKernelGGL(luna_probe_pair_write, dim3(rows), dim3(256), 0, stream, (float4_*)a, (float4_*)b, rows);
    luna::check_hip(hipGetLastError(), "luna_probe_pair_write launch");
    luna::check_hip(hipEventRecord(stop, stream), "hipEventRecord");
    luna::check_hip(hipEventSynchronize(stop), "hipEventSynchronize");
    float ms = 0;
    luna::check_hip(hipEventElapsedTime(&ms, start, stop), "hipEventElapsedTime");
    best = std::min(best, ms);
  }
  hipEventDestroy(start);
  hipEventDestroy(stop);
  return best;
}

// Region classes along buffers, relative to a reference point.  A buffer of
// several GB may straddle two regions, so each buffer is sampled at up to
// four 1 GB windows (start, thirds, end); a window is in class 0 when
// writing it together with the reference is not faster than writing two
// halves of the reference's own 2 GB together.
struct RegionProbe {
  char* ref;
  hipStream_t stream;
  float same_ms;
  bool log;
  RegionProbe(void* reference, hipStream_t s) : ref((char*)reference), stream(s) {
    log = std::getenv("LUNAEQ_AMD_PROBE_LOG") != nullptr;
    same_ms = pair_write_ms(ref, ref + kProbeBytes, stream);
    if (log) std::fprintf(stderr, "probe ref %p: %.3f ms\n", (void*)ref, same_ms);
  }
  bool same(void* window) const {
    const float ms = pair_write_ms(ref, window, stream);
    if (log) std::fprintf(stderr, "probe %p: %.3f ms (%s)\n", window, ms, ms >= kOtherRegion * same_ms ? "same" : "other");
    return ms >= kOtherRegion * same_ms;
  }
  // Fraction of the sampled windows of [p, p + bytes) in the reference's class.
  double fraction_same(void* p, size_t bytes, bool p_is_ref) const {
    std::vector<size_t> offsets = {0};
    if (bytes >= 4 * kProbeBytes) offsets = {0, bytes / 3, 2 * bytes / 3, bytes - kProbeBytes};
    else if (bytes >= 2 * kProbeBytes) offsets = {0, bytes - kProbeBytes};
    int hits = 0;
    for (size_t off : offsets) {
      off &= ~(size_t)((2u << 20) - 1);
      if (p_is_ref && off < 2 * kProbeBytes) {
        ++hits;  // the reference's own 2 GB
        continue;
      }
      hits += same((char*)p + off) ? 1 : 0;
    }
    return (double)hits / (double)offsets.size();
  }
};

// Expected share of write pairs that meet in one region when a and b are
// written together (two region classes): fa fb + (1 - fa)(1 - fb).
double overlap(double fa, double fb) { return fa * fb + (1.0 - fa) * (1.0 - fb); }

constexpr double kAcceptOverlap = 0.25;

}  // namespace

extern "C" {

int luna_region_overlap(void* a, size_t a_bytes, void* b, size_t b_bytes, LunaStream stream, double* result) {
  return luna::guard_call([&] {
    if (!a || !b || !result) luna::fail("luna_region_overlap: null argument");
    if (a_bytes < 2 * kProbeBytes || b_bytes < kProbeBytes)
      luna::fail("luna_region_overlap: needs 2 GB of the first buffer and 1 GB of the second");
    RegionProbe probe(a, (hipStream_t)stream);
    *result = overlap(probe.fraction_same(a, a_bytes, true), probe.fraction_same(b, b_bytes, false));
  });
}

int luna_placed_alloc(size_t bytes, void* avoid, size_t avoid_bytes, size_t max_spacer_bytes, LunaStream stream,
                      void** out, int* moved) {
  std::vector<void*> held;
  void* reference = nullptr;
  auto release = [&](void* keep) {
    for (void* p : held)
      if (p != keep) hipFree(p);
    held.clear();
    if (reference) hipFree(reference);
    reference = nullptr;
  };
  const int status = luna::guard_call([&] {
    if (!out || !moved) luna::fail("luna_placed_alloc: null argument");
    *out = nullptr;
    *moved = 0;
    if (bytes < kProbeBytes) luna::fail("luna_placed_alloc: buffers below 1 GB are not placed");
    hipStream_t s = (hipStream_t)stream;
    if (max_spacer_bytes == 0) {
      // No search: an ordinary allocation, not probed.
      luna::check_hip(hipMalloc(out, bytes), "hipMalloc");
      return;
    }
    void* ref = avoid;
    size_t ref_bytes = avoid_bytes;
    if (!ref || avoid_bytes < 2 * kProbeBytes) {
      luna::check_hip(hipMalloc(&reference, 2 * kProbeBytes), "hipMalloc(probe reference)");
      ref = reference;
      ref_bytes = 2 * kProbeBytes;
    }
    RegionProbe probe(ref, s);
    const double f_ref = probe.fraction_same(ref, ref_bytes, true);
    size_t spacer = 0;
    void* best = nullptr;
    double best_overlap = 2.0;
    for (;;) {
      void* candidate = nullptr;
      if (hipMalloc(&candidate, bytes) != hipSuccess) {
        (void)hipGetLastError();
        break;
      }
      held.push_back(candidate);
      const double o = overlap(f_ref, probe.fraction_same(candidate, bytes, false));
      if (o < best_overlap) {
        best_overlap = o;
        best = candidate;
      }
      if (o <= kAcceptOverlap) break;
      spacer += bytes;
      size_t free_bytes = 0, total_bytes = 0;
      luna::check_hip(hipMemGetInfo(&free_bytes, &total_bytes), "hipMemGetInfo");
      if (spacer + bytes > max_spacer_bytes || free_bytes < 2 * bytes) break;
    }
    if (!best) luna::fail("luna_placed_alloc: hipMalloc of " + std::to_string(bytes) + " bytes failed");
    *out = best;
    *moved = best_overlap <= kAcceptOverlap ? 1 : 0;
  });
  release(status == 0 && out ? *out : nullptr);
  return status;
}

int luna_placed_free(void* pointer) {
  return luna::guard_call([&] {
    if (pointer) luna::check_hip(hipFree(pointer), "hipFree(placed buffer)");
  });
}

}  // extern "C"
