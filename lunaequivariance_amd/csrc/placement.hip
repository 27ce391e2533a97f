// Workspace placement across the HBM regions of the device.
//
// Measured on MI355X (288 GB): device memory falls into regions of about
// 96 GB of physical address space, and the driver fills them in order.  Two
// buffers written at the same time run at about 5.5 TB/s together when they
// lie in one region and at about 6.8 TB/s when they lie in two (random 8 KB
// rows, non-temporal stores; one buffer alone about 5.4 TB/s).  The UVU
// backward writes its weight gradient and its per-edge gx messages together,
// and the gx pass then reads the messages while writing gx: with the message
// workspace in another region than the tensors the caller allocated just
// before, the config-2 backward takes 8.6 instead of 9.7 ms and the gx pass
// 1.40 instead of 1.59 ms.
//
// luna_placed_alloc allocates a buffer outside the region of a given buffer
// (or, without one, of a fresh reference allocation).  Which region an
// allocation lands in is only known by measurement: each candidate is probed
// by writing 256 MB of it and 256 MB of the reference at the same time (rows
// in a scrambled order), against the same write pair within the reference.
// Candidates that share the reference's region are held (so the allocator
// moves on) and released once a candidate in another region is
// found, or when the spacer budget or free memory runs out; then the first
// candidate is returned and *moved is 0.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <vector>

#include "../../include/lunaeq_amd.h"
#include "common.h"

namespace {

constexpr size_t kProbeBytes = 256ull << 20;
constexpr size_t kRowBytes = 8192;
constexpr double kOtherRegion = 0.88;  // probe time ratio below which two buffers are in different regions

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

// 1 when b lies in the region of a: writing a and b together is not faster
// than writing two parts of a together.  Overwrites 512 MB of a and 256 MB of b.
int same_region(void* a, void* b, hipStream_t stream) {
  const float same = pair_write_ms(a, (char*)a + kProbeBytes, stream);
  return pair_write_ms(a, b, stream) < kOtherRegion * same ? 0 : 1;
}

}  // namespace

extern "C" {

int luna_same_region(void* a, size_t a_bytes, void* b, size_t b_bytes, LunaStream stream, int* same) {
  return luna::guard_call([&] {
    if (!a || !b || !same) luna::fail("luna_same_region: null argument");
    if (a_bytes < 2 * kProbeBytes || b_bytes < kProbeBytes)
      luna::fail("luna_same_region: needs 512 MB of the first buffer and 256 MB of the second");
    *same = same_region(a, b, (hipStream_t)stream);
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
    if (bytes < kProbeBytes) luna::fail("luna_placed_alloc: buffers below 256 MB are not placed");
    hipStream_t s = (hipStream_t)stream;
    if (max_spacer_bytes == 0) {
      // No search: an ordinary allocation, not probed.
      luna::check_hip(hipMalloc(out, bytes), "hipMalloc");
      return;
    }
    void* ref = avoid;
    if (!ref || avoid_bytes < 2 * kProbeBytes) {
      luna::check_hip(hipMalloc(&reference, 2 * kProbeBytes), "hipMalloc(probe reference)");
      ref = reference;
    }
    size_t spacer = 0;
    for (;;) {
      void* candidate = nullptr;
      if (hipMalloc(&candidate, bytes) != hipSuccess) {
        (void)hipGetLastError();
        break;
      }
      held.push_back(candidate);
      if (!same_region(ref, candidate, s)) {
        *out = candidate;
        *moved = 1;
        return;
      }
      spacer += bytes;
      size_t free_bytes = 0, total_bytes = 0;
      luna::check_hip(hipMemGetInfo(&free_bytes, &total_bytes), "hipMemGetInfo");
      if (spacer + bytes > max_spacer_bytes || free_bytes < 2 * bytes) break;
    }
    if (held.empty()) luna::fail("luna_placed_alloc: hipMalloc of " + std::to_string(bytes) + " bytes failed");
    *out = held.front();
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
