// Graph tables of the convolution on the GPU (the work of the reference's
// one-pass topology kernel, src/lunatp/utils/graph.py:142-846, and of
// make_graph / make_source_segments, src/lunatp/graph.py:49-141 and
// src/lunatp/uvu_conv/graph.py:38-99), as a short pipeline of integer
// kernels:
//   * CSR row pointers by binary search: rowptr[n] = first edge with key >= n
//     in a key-sorted edge list (dst as given; src after the sort below);
//   * edge ids by source: stable LSD radix sort of (src, edge id), 4-bit
//     digits, one upsweep (digit counts per 2048-edge tile), one scan and one
//     stable scatter per digit;
//   * node orders: the same sort on keys E - degree (descending degree,
//     ties by node id, as a stable descending argsort);
//   * node tiers: scan of the ordered degrees and a search for E/4, 2E/4, 3E/4;
//   * source segments: max(1, ceil(degree/32)) chunks per node, ordered by
//     descending length, then descending node degree, then segment index.
// Every buffer is the caller's; scratch comes from one caller-sized
// workspace.  Kernels are compiled with hipRTC once (code-object cache).
#include <algorithm>
#include <cstdint>
#include <memory>
#include <string>

#include "../../include/lunaeq_amd.h"
#include "common.h"

namespace luna {
namespace {

constexpr int kTile = 2048;    // elements per workgroup (256 threads x 8)
constexpr int kDigits = 16;    // radix 16 (4-bit digits)
constexpr int kSegment = 32;   // edges per source segment

const char* kGraphSource = R"(
typedef long long i64;
typedef unsigned int u32;

extern "C" __global__ void luna_graph_bounds_init(i64* status) {
  if (threadIdx.x == 0) {
    status[0] = 0x7fffffffffffffffLL;     // min index
    status[1] = -0x7fffffffffffffffLL - 1;  // max index
    status[2] = 0;                        // dst not sorted
    status[3] = 0;
  }
}

// min / max over src and dst, and whether dst descends anywhere.
template <typename T>
__device__ void bounds(const T* src, const T* dst, i64 E, i64* status) {
  i64 lo = 0x7fffffffffffffffLL, hi = -0x7fffffffffffffffLL - 1;
  int unsorted = 0;
  for (i64 i = (i64)blockIdx.x * blockDim.x + threadIdx.x; i < E; i += (i64)gridDim.x * blockDim.x) {
    const i64 s = (i64)src[i], d = (i64)dst[i];
    lo = min(lo, min(s, d));
    hi = max(hi, max(s, d));
    if (i + 1 < E && (i64)dst[i + 1] < d) unsorted = 1;
  }
  for (int m = 32; m >= 1; m >>= 1) {
    lo = min(lo, (i64)__shfl_xor(lo, m, 64));
    hi = max(hi, (i64)__shfl_xor(hi, m, 64));
    unsorted |= __shfl_xor(unsorted, m, 64);
  }
  if ((threadIdx.x & 63) == 0) {
    atomicMin((long long*)&status[0], (long long)lo);
    atomicMax((long long*)&status[1], (long long)hi);
    if (unsorted) atomicOr((unsigned long long*)&status[2], 1ULL);
  }
}
extern "C" __global__ void __launch_bounds__(256) luna_graph_bounds32(const int* src, const int* dst, i64 E,
                                                                      i64* status) {
  bounds(src, dst, E, status);
}
extern "C" __global__ void __launch_bounds__(256) luna_graph_bounds64(const i64* src, const i64* dst, i64 E,
                                                                      i64* status) {
  bounds(src, dst, E, status);
}

// int32 copies of the indices (values already checked to fit).
extern "C" __global__ void __launch_bounds__(256) luna_graph_narrow(const void* in, int is64, int* out, i64 n) {
  const i64 i = (i64)blockIdx.x * 256 + threadIdx.x;
  if (i >= n) return;
  out[i] = is64 ? (int)((const i64*)in)[i] : ((const int*)in)[i];
}

extern "C" __global__ void __launch_bounds__(256) luna_graph_iota(int* out, i64 n) {
  const i64 i = (i64)blockIdx.x * 256 + threadIdx.x;
  if (i < n) out[i] = (int)i;
}

// rowptr[n] = first index i with keys[i] >= n, for n = 0..N (keys ascending).
extern "C" __global__ void __launch_bounds__(256) luna_graph_rowptr(const int* keys, i64 E, int N, int* rowptr) {
  const i64 n = (i64)blockIdx.x * 256 + threadIdx.x;
  if (n > N) return;
  i64 lo = 0, hi = E;
  while (lo < hi) {
    const i64 mid = (lo + hi) >> 1;
    if (keys[mid] < n) lo = mid + 1; else hi = mid;
  }
  rowptr[n] = (int)lo;
}

// keys[n] = E - degree[n] with degree from a row-pointer array.
extern "C" __global__ void __launch_bounds__(256) luna_graph_degree_keys(const int* rowptr, int N, int E,
                                                                        u32* keys) {
  const int n = blockIdx.x * 256 + threadIdx.x;
  if (n < N) keys[n] = (u32)(E - (rowptr[n + 1] - rowptr[n]));
}

// ---- exclusive scan of int32 (tiles of 2048, block sums scanned recursively)
__device__ int block_exclusive_scan(int v, int* wsum, int* total) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  int inc = v;
  for (int m = 1; m < 64; m <<= 1) {
    const int o = __shfl_up(inc, m, 64);
    if (lane >= m) inc += o;
  }
  if (lane == 63) wsum[wave] = inc;
  __syncthreads();
  int before = 0, all = 0;
  for (int w = 0; w < 4; ++w) {
    before += w < wave ? wsum[w] : 0;
    all += wsum[w];
  }
  __syncthreads();
  *total = all;
  return before + inc - v;
}

// out[i] = exclusive prefix of in within its tile (in[i] = 0 past n_in), for
// i < n_out; sums[tile] = tile total.
extern "C" __global__ void __launch_bounds__(256) luna_graph_scan_tiles(const int* in, i64 n_in, int* out,
                                                                        i64 n_out, int* sums) {
  __shared__ int wsum[4];
  const i64 base = (i64)blockIdx.x * 2048 + threadIdx.x * 8;
  int v[8], s = 0;
  for (int j = 0; j < 8; ++j) {
    v[j] = base + j < n_in ? in[base + j] : 0;
    s += v[j];
  }
  int total;
  int run = block_exclusive_scan(s, wsum, &total);
  for (int j = 0; j < 8; ++j) {
    if (base + j < n_out) out[base + j] = run;
    run += v[j];
  }
  if (threadIdx.x == 0) sums[blockIdx.x] = total;
}

extern "C" __global__ void __launch_bounds__(256) luna_graph_scan_add(int* out, i64 n_out, const int* offsets) {
  const i64 i = (i64)blockIdx.x * 256 + threadIdx.x;
  if (i < n_out) out[i] += offsets[i / 2048];
}

// ---- stable LSD radix sort, 4-bit digits
// hist[d * tiles + tile] = count of digit d in the tile.
extern "C" __global__ void __launch_bounds__(256) luna_graph_radix_count(const u32* keys, i64 n, int shift,
                                                                         int* hist, int tiles) {
  __shared__ int table[16][256];
  const int t = threadIdx.x;
  for (int d = 0; d < 16; ++d) table[d][t] = 0;
  const i64 base = (i64)blockIdx.x * 2048 + t * 8;
  for (int j = 0; j < 8; ++j)
    if (base + j < n) ++table[(keys[base + j] >> shift) & 15][t];
  __syncthreads();
  if (t < 16) {
    int s = 0;
    for (int k = 0; k < 256; ++k) s += table[t][k];
    hist[(i64)t * tiles + blockIdx.x] = s;
  }
}

// Scatter of one tile: position = offsets[d][tile] + count of digit d in the
// earlier elements of the tile (threads own 8 consecutive elements, in order).
extern "C" __global__ void __launch_bounds__(256) luna_graph_radix_scatter(
    const u32* keys, const int* vals, u32* keys_out, int* vals_out, i64 n, int shift, const int* offsets,
    int tiles) {
  __shared__ int table[16][256];
  __shared__ int wsum[16][4];
  __shared__ int start[16];
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  for (int d = 0; d < 16; ++d) table[d][t] = 0;
  const i64 base = (i64)blockIdx.x * 2048 + t * 8;
  u32 k[8];
  for (int j = 0; j < 8; ++j) {
    k[j] = base + j < n ? keys[base + j] : 0u;
    if (base + j < n) ++table[(k[j] >> shift) & 15][t];
  }
  if (t < 16) start[t] = offsets[(i64)t * tiles + blockIdx.x];
  // Exclusive prefix over threads, for every digit.
  int inc[16];
  for (int d = 0; d < 16; ++d) {
    inc[d] = table[d][t];
    for (int m = 1; m < 64; m <<= 1) {
      const int o = __shfl_up(inc[d], m, 64);
      if (lane >= m) inc[d] += o;
    }
    if (lane == 63) wsum[d][wave] = inc[d];
  }
  __syncthreads();
  for (int d = 0; d < 16; ++d) {
    int before = 0;
    for (int w = 0; w < 4; ++w) before += w < wave ? wsum[d][w] : 0;
    table[d][t] = start[d] + before + inc[d] - table[d][t];
  }
  for (int j = 0; j < 8; ++j) {
    if (base + j >= n) break;
    const int pos = table[(k[j] >> shift) & 15][t]++;
    keys_out[pos] = k[j];
    vals_out[pos] = vals ? vals[base + j] : (int)(base + j);
  }
}

// Keys of the first pass from int32 indices.
extern "C" __global__ void __launch_bounds__(256) luna_graph_keys_from(const int* in, u32* keys, i64 n) {
  const i64 i = (i64)blockIdx.x * 256 + threadIdx.x;
  if (i < n) keys[i] = (u32)in[i];
}

// node_tiers[t-1] = (first i with cum[i] >= t*E/4) + 1, cum = inclusive scan of
// the degrees in node order (ex = its exclusive scan, ex[N] = E).
extern "C" __global__ void __launch_bounds__(256) luna_graph_tiers(const int* ex, int N, i64 E, int* tiers) {
  const int i = blockIdx.x * 256 + threadIdx.x;
  if (E == 0 || N == 0) {
    if (i < 3) tiers[i] = N;
    return;
  }
  if (i >= N) return;
  const i64 lo = ex[i], hi = ex[i + 1];
  for (int q = 1; q <= 3; ++q) {
    const i64 thr = q * E / 4;
    if (thr <= hi && (i == 0 || lo < thr)) tiers[q - 1] = i + 1;
  }
}

extern "C" __global__ void __launch_bounds__(256) luna_graph_gather_degree(const int* order, const int* rowptr,
                                                                          int N, int* out) {
  const int i = blockIdx.x * 256 + threadIdx.x;
  if (i < N) {
    const int n = order[i];
    out[i] = rowptr[n + 1] - rowptr[n];
  }
}

// Segments per node: max(1, ceil(degree / 32)).
extern "C" __global__ void __launch_bounds__(256) luna_graph_segment_counts(const int* rowptr, int N, int* count) {
  const int n = blockIdx.x * 256 + threadIdx.x;
  if (n < N) {
    const int d = rowptr[n + 1] - rowptr[n];
    count[n] = d > 0 ? (d + 31) / 32 : 1;
  }
}

extern "C" __global__ void __launch_bounds__(256) luna_graph_segments(const int* rowptr, const int* seg_rowptr,
                                                                     int N, int E, int* nodes, int* begin, int* end,
                                                                     u32* deg_key, u32* len_key) {
  const int n = blockIdx.x * 256 + threadIdx.x;
  if (n >= N) return;
  const int r0 = rowptr[n], r1 = rowptr[n + 1];
  for (int s = seg_rowptr[n], k = 0; s < seg_rowptr[n + 1]; ++s, ++k) {
    const int b = r0 + 32 * k, e = min(b + 32, r1);
    nodes[s] = n;
    begin[s] = b;
    end[s] = e;
    deg_key[s] = (u32)(E - (r1 - r0));
    len_key[s] = (u32)(32 - (e - b));
  }
}

// Past the real segments (seg_rowptr[N] of them): keys that sort after all.
extern "C" __global__ void __launch_bounds__(256) luna_graph_segment_padding(const int* seg_rowptr, int N, i64 S,
                                                                            int E, u32* deg_key, u32* len_key) {
  const i64 s = (i64)blockIdx.x * 256 + threadIdx.x;
  if (s < S && s >= seg_rowptr[N]) {
    deg_key[s] = (u32)E + 1u;
    len_key[s] = 63u;
  }
}

extern "C" __global__ void __launch_bounds__(256) luna_graph_gather_keys(const int* order, const u32* keys, i64 n,
                                                                        u32* out) {
  const i64 i = (i64)blockIdx.x * 256 + threadIdx.x;
  if (i < n) out[i] = keys[order[i]];
}
)";

struct GraphKernels {
  ModuleCache kernels;
  GraphKernels() { kernels.tag = "graph"; }
};

GraphKernels& graph_kernels() {
  static GraphKernels g;
  return g;
}

hipModule_t graph_module(const char* cache_dir) {
  GraphKernels& g = graph_kernels();
  if (cache_dir && g.kernels.cache_dir.empty()) g.kernels.cache_dir = cache_dir;
  return g.kernels.module_for("graph", [] { return std::string(kGraphSource); });
}

unsigned blocks_of(int64_t n, int64_t per) { return (unsigned)std::max<int64_t>(1, (n + per - 1) / per); }
int64_t tiles_of(int64_t n) { return (n + kTile - 1) / kTile; }
size_t align256(size_t n) { return (n + 255) & ~(size_t)255; }

// Bump allocator over the caller's workspace.
// Scratch is taken and released in stack order; `peak` sizes the workspace.
struct Arena {
  char* base;
  size_t size, used = 0, peak = 0;
  template <typename T>
  T* take(int64_t count) {
    const size_t bytes = align256((size_t)std::max<int64_t>(count, 1) * sizeof(T));
    if (base && used + bytes > size) fail("luna_graph_build: workspace too small");
    T* p = base ? (T*)(base + used) : nullptr;
    used += bytes;
    peak = std::max(peak, used);
    return p;
  }
};

struct Builder {
  hipModule_t module;
  hipStream_t stream;
  Arena& arena;

  void run(const char* name, dim3 grid, void** args) {
    launch(std::string("graph_") + name, function_for(module, std::string("luna_graph_") + name), grid, dim3(256),
           stream, args);
  }

  // out[0..n_out) = exclusive scan of in[0..n_in) (zero past n_in).
  void scan(const int* in, int64_t n_in, int* out, int64_t n_out) {
    if (n_out <= 0) return;
    const size_t mark = arena.used;
    const int64_t tiles = tiles_of(n_out);
    int* sums = arena.take<int>(tiles);
    int* offsets = tiles > 1 ? arena.take<int>(tiles) : nullptr;
    if (module) {
      void* a[] = {&in, &n_in, &out, &n_out, &sums};
      run("scan_tiles", blocks_of(n_out, kTile), a);
    }
    if (tiles > 1) {
      int64_t t = tiles;
      scan(sums, t, offsets, t);
      if (module) {
        void* b[] = {&out, &n_out, &offsets};
        run("scan_add", blocks_of(n_out, 256), b);
      }
    }
    arena.used = mark;
  }

  // Stable sort of (keys, vals) by the low `bits` of keys; vals == null means
  // the element index.  The sorted values land in vals_out (keys_out, if
  // given, receives the sorted keys).  keys is consumed.
  void sort(uint32_t* keys, const int* vals, int64_t n, int bits, int* vals_out, uint32_t* keys_out) {
    if (n <= 0) return;
    const size_t mark = arena.used;
    const int64_t tiles = tiles_of(n);
    uint32_t* k_tmp = arena.take<uint32_t>(n);
    uint32_t* k_tmp2 = arena.take<uint32_t>(n);
    int* v_tmp = arena.take<int>(n);
    int* hist = arena.take<int>(kDigits * tiles);
    int* offsets = arena.take<int>(kDigits * tiles);
    if (!module) {
      scan(hist, kDigits * tiles, offsets, kDigits * tiles);
      arena.used = mark;
      return;
    }
    const int passes = (bits + 3) / 4;
    uint32_t* k_in = keys;
    const int* v_in = vals;
    // Pass p writes buffer (passes - 1 - p) % 2, so the last pass writes
    // vals_out (and its keys to k_tmp); the input is read by pass 0 only.
    uint32_t* k_buf[2] = {k_tmp, k_tmp2};
    int* v_buf[2] = {vals_out, v_tmp};
    int t = (int)tiles;
    for (int p = 0; p < passes; ++p) {
      const int which = (passes - 1 - p) % 2;
      uint32_t* k_out = k_buf[which];
      int* v_out = v_buf[which];
      int shift = 4 * p;
      void* a[] = {&k_in, &n, &shift, &hist, &t};
      run("radix_count", blocks_of(n, kTile), a);
      scan(hist, kDigits * tiles, offsets, kDigits * tiles);
      void* b[] = {&k_in, &v_in, &k_out, &v_out, &n, &shift, &offsets, &t};
      run("radix_scatter", blocks_of(n, kTile), b);
      k_in = k_out;
      v_in = v_out;
    }
    if (passes == 0) {
      if (vals) fail("luna_graph_build: internal (zero-pass sort with values)");
      void* a[] = {&vals_out, &n};
      run("iota", blocks_of(n, 256), a);
    }
    if (keys_out && passes > 0) {
      // The last pass wrote its keys to k_buf[0] == k_tmp.
      check_hip(hipMemcpyAsync(keys_out, k_tmp, (size_t)n * sizeof(uint32_t), hipMemcpyDeviceToDevice, stream),
                "hipMemcpyAsync");
    }
    arena.used = mark;
  }
};

int bits_for(int64_t max_key) {
  int b = 0;
  while (b < 32 && (max_key >> b) != 0) ++b;
  return b;
}

struct Outputs {
  int32_t *src32, *dst32, *dst_rowptr, *src_rowptr, *edge_ids_by_src, *edge_ids_by_dst, *node_order,
      *source_node_order, *node_tiers, *seg_rowptr, *seg_nodes, *seg_begin, *seg_end, *seg_order;
};

// One pass with module == null sizes the workspace; a second one launches.
void build(hipModule_t module, hipStream_t stream, Arena& arena, const void* src, const void* dst, int is64,
           int64_t N, int64_t E, Outputs o) {
  Builder b{module, stream, arena};
  const int64_t seg_cap = N + E / kSegment + 1;
  uint32_t* keys = arena.take<uint32_t>(std::max(std::max(E, N), seg_cap));
  int* sorted_src = arena.take<int>(E);
  int* work = arena.take<int>(std::max(N + 1, seg_cap));
  uint32_t* keys2 = arena.take<uint32_t>(seg_cap);
  int* perm = arena.take<int>(seg_cap);
  int Ni = (int)N, Ei = (int)E;
  if (module) {
    void* a[] = {(void*)&src, &is64, &o.src32, &E};
    b.run("narrow", blocks_of(E, 256), a);
    void* c[] = {(void*)&dst, &is64, &o.dst32, &E};
    b.run("narrow", blocks_of(E, 256), c);
    void* d[] = {&o.edge_ids_by_dst, &E};
    b.run("iota", blocks_of(E, 256), d);
    void* r[] = {&o.dst32, &E, &Ni, &o.dst_rowptr};
    b.run("rowptr", blocks_of(N + 1, 256), r);
    void* k[] = {&o.src32, &keys, &E};
    b.run("keys_from", blocks_of(E, 256), k);
  }
  // Edge ids by source (stable), then the source CSR from the sorted keys.
  b.sort(keys, nullptr, E, bits_for(N > 0 ? N - 1 : 0), o.edge_ids_by_src, (uint32_t*)sorted_src);
  if (module) {
    if (bits_for(N > 0 ? N - 1 : 0) == 0 && E > 0) {
      // Every source is node 0: the keys are already "sorted".
      void* k[] = {&o.src32, &keys, &E};
      b.run("keys_from", blocks_of(E, 256), k);
      check_hip(hipMemcpyAsync(sorted_src, keys, (size_t)E * 4, hipMemcpyDeviceToDevice, stream), "hipMemcpyAsync");
    }
    void* r[] = {&sorted_src, &E, &Ni, &o.src_rowptr};
    b.run("rowptr", blocks_of(N + 1, 256), r);
  }
  // Node orders: descending degree, ties by node id.
  const int deg_bits = bits_for(E);
  for (int which = 0; which < 2; ++which) {
    const int32_t* rowptr = which == 0 ? o.dst_rowptr : o.src_rowptr;
    int32_t* order = which == 0 ? o.node_order : o.source_node_order;
    if (module && N > 0) {
      void* a[] = {&rowptr, &Ni, &Ei, &keys};
      b.run("degree_keys", blocks_of(N, 256), a);
    }
    b.sort(keys, nullptr, N, deg_bits, order, nullptr);
  }
  // Node tiers from the degrees in node order.
  if (module && N > 0) {
    void* a[] = {&o.node_order, &o.dst_rowptr, &Ni, &perm};
    b.run("gather_degree", blocks_of(N, 256), a);
  }
  b.scan(perm, N, work, N + 1);
  if (module) {
    void* a[] = {&work, &Ni, &E, &o.node_tiers};
    b.run("tiers", blocks_of(std::max<int64_t>(N, 3), 256), a);
  }
  // Source segments.
  if (module && N > 0) {
    void* a[] = {&o.src_rowptr, &Ni, &perm};
    b.run("segment_counts", blocks_of(N, 256), a);
  }
  b.scan(perm, N, o.seg_rowptr, N + 1);
  if (module && N > 0) {
    void* a[] = {&o.src_rowptr, &o.seg_rowptr, &Ni, &Ei, &o.seg_nodes, &o.seg_begin, &o.seg_end, &keys, &keys2};
    b.run("segments", blocks_of(N, 256), a);
  }
  // The segment count is only known on the device: sort the upper bound
  // seg_cap, with padding keys past the real segments that sort last.  The
  // real ones are a prefix of the result, because padding keys exceed every
  // real key (degree key E - d <= E < E + 1, length key 32 - len <= 31 < 32).
  int64_t S = N > 0 ? seg_cap : 0;
  if (module && S > 0) {
    void* a[] = {&o.seg_rowptr, &Ni, &S, &Ei, &keys, &keys2};
    b.run("segment_padding", blocks_of(S, 256), a);
  }
  b.sort(keys, nullptr, S, bits_for(E + 1), perm, nullptr);
  if (module && S > 0) {
    void* a[] = {&perm, &keys2, &S, &keys};
    b.run("gather_keys", blocks_of(S, 256), a);
  }
  b.sort(keys, perm, S, 6, o.seg_order, nullptr);
}

}  // namespace
}  // namespace luna

using namespace luna;

extern "C" {

int luna_graph_bounds(const void* src, const void* dst, int index_bits, int64_t num_edges, int64_t* status,
                      LunaStream stream) {
  return guard_call([&] {
    if (index_bits != 32 && index_bits != 64) fail("luna_graph_bounds: index_bits must be 32 or 64");
    if (num_edges < 0) fail("luna_graph_bounds: negative edge count");
    if (!status || (num_edges > 0 && (!src || !dst))) fail("luna_graph_bounds: null argument");
    hipModule_t module = graph_module(nullptr);
    hipStream_t s = (hipStream_t)stream;
    void* a[] = {&status};
    launch("graph_bounds_init", function_for(module, "luna_graph_bounds_init"), dim3(1), dim3(64), s, a);
    if (num_edges > 0) {
      void* b[] = {(void*)&src, (void*)&dst, &num_edges, &status};
      const unsigned grid = (unsigned)std::min<int64_t>(2048, (num_edges + 255) / 256);
      launch("graph_bounds", function_for(module, index_bits == 64 ? "luna_graph_bounds64" : "luna_graph_bounds32"),
             dim3(grid), dim3(256), s, b);
    }
  });
}

int luna_graph_workspace(int64_t num_nodes, int64_t num_edges, size_t* bytes) {
  return guard_call([&] {
    if (!bytes) fail("luna_graph_workspace: null argument");
    if (num_nodes < 0 || num_edges < 0) fail("luna_graph_workspace: negative size");
    if (num_nodes >= (1LL << 31) || num_edges >= (1LL << 31) - 1) fail("graph exceeds int32 indexing");
    Arena arena{nullptr, 0};
    Outputs o{};
    build(nullptr, nullptr, arena, nullptr, nullptr, 0, num_nodes, num_edges, o);
    *bytes = arena.peak;
  });
}

int luna_graph_build(const void* src, const void* dst, int index_bits, int64_t num_nodes, int64_t num_edges,
                     int32_t* src32, int32_t* dst32, int32_t* dst_rowptr, int32_t* src_rowptr,
                     int32_t* edge_ids_by_src, int32_t* edge_ids_by_dst, int32_t* node_order,
                     int32_t* source_node_order, int32_t* node_tiers, int32_t* seg_rowptr, int32_t* seg_nodes,
                     int32_t* seg_begin, int32_t* seg_end, int32_t* seg_order, void* workspace,
                     size_t workspace_bytes, LunaStream stream) {
  return guard_call([&] {
    if (index_bits != 32 && index_bits != 64) fail("luna_graph_build: index_bits must be 32 or 64");
    if (num_nodes < 0 || num_edges < 0) fail("luna_graph_build: negative size");
    if (num_nodes >= (1LL << 31) || num_edges >= (1LL << 31) - 1) fail("graph exceeds int32 indexing");
    if (!dst_rowptr || !src_rowptr || !node_tiers || !seg_rowptr) fail("luna_graph_build: null table");
    if (num_edges > 0 && (!src || !dst || !src32 || !dst32 || !edge_ids_by_src || !edge_ids_by_dst))
      fail("luna_graph_build: null edge table");
    if (num_nodes > 0 && (!node_order || !source_node_order || !seg_nodes || !seg_begin || !seg_end || !seg_order))
      fail("luna_graph_build: null node table");
    size_t need = 0;
    {
      Arena sizing{nullptr, 0};
      Outputs none{};
      build(nullptr, nullptr, sizing, nullptr, nullptr, 0, num_nodes, num_edges, none);
      need = sizing.peak;
    }
    if (!workspace || workspace_bytes < need) fail("luna_graph_build: workspace too small");
    Arena arena{(char*)workspace, workspace_bytes};
    Outputs o{src32, dst32, dst_rowptr, src_rowptr, edge_ids_by_src, edge_ids_by_dst, node_order,
              source_node_order, node_tiers, seg_rowptr, seg_nodes, seg_begin, seg_end, seg_order};
    build(graph_module(nullptr), (hipStream_t)stream, arena, src, dst, index_bits == 64, num_nodes, num_edges, o);
  });
}

int luna_graph_precompile(const char* cache_dir) {
  return guard_call([&] {
    GraphKernels& g = graph_kernels();
    if (cache_dir && g.kernels.cache_dir.empty()) g.kernels.cache_dir = cache_dir;
    g.kernels.code_for("graph", [] { return std::string(kGraphSource); });
  });
}

}  // extern "C"
