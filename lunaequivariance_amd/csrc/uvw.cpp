// Shared-weight UVW tensor product on CDNA4 matrix cores (fp32).
//
// For a path p (input block l1 with mul1 copies, edge block l2 with mul2
// copies, output block io with mul3 copies) and a batch row b:
//   Z_p[b, k, K=(u,v)] = sum_{(i,j)} c_ijk x[b, xo + u*d1 + i] y[b, yo + v*d2 + j]
//   out[b, oo + w*d3 + k] += sum_K Z_p[b, k, K] W_p[K, w]        (W_p = w[wo + K*mul3 + w])
// (e3nn's uvw connection, src/lunatp/uvw/kernels/forward.py:1082-1465).  The
// sparse CG producer is VALU work staged into LDS; the contraction over K is
// v_mfma_f32_32x32x2f32 with a 32-row tile of b as M and 32 output channels
// as N.  The backward is two more matrix-core passes:
//   dZ_p[b, k, K] = sum_w g[b, oo + w*d3 + k] W_p[K, w]  ->  gx, gy through the CG terms
//   dW_p[K, w]    = sum_{b,k} Z_p[b, k, K] g[b, oo + w*d3 + k]   (per row chunk, then reduced)
#include <algorithm>
#include <cstdio>
#include <cstdlib>
#include <map>
#include <memory>
#include <set>
#include <sstream>

#include "../../include/lunaeq_amd.h"
#include "common.h"

namespace luna {
namespace {

struct UvwTerm {
  int i, j, k;
  double c;
};

struct UvwPath {
  int x_off, y_off, out_off, w_off, mul1, mul2, mul3, d1, d2, d3;
  std::vector<UvwTerm> terms;
};

struct UvwSpec {
  int dtype_bits = 32;
  int in1 = 0, in2 = 0, out = 0, wnum = 0;
  std::vector<UvwPath> paths;
};

constexpr int kRows = 32;       // batch rows per workgroup tile
constexpr int kChunkTiles = 8;  // row tiles per workgroup in the weight-gradient pass

int read_int(std::istringstream& in, const char* what) {
  long long value;
  if (!(in >> value)) fail(std::string("uvw spec: expected integer for ") + what);
  if (value < 0 || value > (1LL << 31) - 1) fail(std::string("uvw spec: value out of range for ") + what);
  return (int)value;
}

UvwSpec parse(const std::string& text) {
  std::istringstream in(text);
  std::string magic;
  in >> magic;
  if (magic != "LUNAUVW1") fail("uvw spec: missing LUNAUVW1 header");
  UvwSpec s;
  s.dtype_bits = read_int(in, "dtype");
  if (s.dtype_bits != 32) fail("uvw spec: the matrix-core UVW path is fp32");
  s.in1 = read_int(in, "in1");
  s.in2 = read_int(in, "in2");
  s.out = read_int(in, "out");
  s.wnum = read_int(in, "weight_numel");
  const int npaths = read_int(in, "npaths");
  if (npaths <= 0) fail("uvw spec: no paths");
  for (int n = 0; n < npaths; ++n) {
    UvwPath p;
    p.x_off = read_int(in, "x_off");
    p.y_off = read_int(in, "y_off");
    p.out_off = read_int(in, "out_off");
    p.w_off = read_int(in, "w_off");
    p.mul1 = read_int(in, "mul1");
    p.mul2 = read_int(in, "mul2");
    p.mul3 = read_int(in, "mul3");
    p.d1 = read_int(in, "d1");
    p.d2 = read_int(in, "d2");
    p.d3 = read_int(in, "d3");
    const int nterms = read_int(in, "nterms");
    if (p.mul1 <= 0 || p.mul2 <= 0 || p.mul3 <= 0) fail("uvw spec: positive multiplicities required");
    if ((long)p.x_off + (long)p.mul1 * p.d1 > s.in1) fail("uvw spec: input block outside in1_dim");
    if ((long)p.y_off + (long)p.mul2 * p.d2 > s.in2) fail("uvw spec: edge block outside in2_dim");
    if ((long)p.out_off + (long)p.mul3 * p.d3 > s.out) fail("uvw spec: output block outside out_dim");
    if ((long)p.w_off + (long)p.mul1 * p.mul2 * p.mul3 > s.wnum) fail("uvw spec: weights outside weight_numel");
    if (p.d3 > 16) fail("uvw spec: output degree above 7 is not supported");
    if (p.mul1 * p.mul2 > 64 && 64 % p.mul2 != 0)
      fail("uvw spec: edge multiplicity must divide 64 when mul1*mul2 exceeds 64");
    for (int t = 0; t < nterms; ++t) {
      UvwTerm term;
      term.i = read_int(in, "i");
      term.j = read_int(in, "j");
      term.k = read_int(in, "k");
      std::string token;
      in >> token;
      char* end = nullptr;
      term.c = std::strtod(token.c_str(), &end);
      if (token.empty() || *end) fail("uvw spec: bad coefficient");
      if (term.i >= p.d1 || term.j >= p.d2 || term.k >= p.d3) fail("uvw spec: coefficient index out of range");
      p.terms.push_back(term);
    }
    s.paths.push_back(std::move(p));
  }
  return s;
}

struct Code {
  std::ostringstream s;
  template <typename... A>
  __attribute__((format(printf, 2, 0))) void line(const char* fmt, A... args) {
    const int size = std::snprintf(nullptr, 0, fmt, args...);
    std::string buffer(size + 1, '\0');
    std::snprintf(&buffer[0], buffer.size(), fmt, args...);
    buffer.resize(size);
    s << buffer << '\n';
  }
};

std::string flit(double c) {
  char b[48];
  std::snprintf(b, sizeof(b), "%.9ef", (double)(float)c);
  return b;
}

int round_up(int v, int m) { return (v + m - 1) / m * m; }

// Output blocks in first-use order, with the paths feeding each.
struct OutBlock {
  int out_off, mul3, d3;
  std::vector<int> paths;
};

std::vector<OutBlock> out_blocks(const UvwSpec& s) {
  std::vector<OutBlock> blocks;
  for (int p = 0; p < (int)s.paths.size(); ++p) {
    const UvwPath& q = s.paths[p];
    bool found = false;
    for (auto& b : blocks)
      if (b.out_off == q.out_off && b.mul3 == q.mul3 && b.d3 == q.d3) {
        b.paths.push_back(p);
        found = true;
      }
    if (!found) blocks.push_back({q.out_off, q.mul3, q.d3, {p}});
  }
  return blocks;
}

struct Dims {
  int kt;      // K tile (multiple of 8: two halves of s-steps, 4 at a time)
  int npad;    // output channels rounded up to 32
  int d3max;
};

Dims dims(const UvwSpec& s) {
  Dims d{0, 0, 0};
  for (const auto& p : s.paths) {
    d.npad = std::max(d.npad, round_up(p.mul3, 32));
    d.d3max = std::max(d.d3max, p.d3);
  }
  d.kt = 64;
  return d;
}

const char* kPrelude = R"(
typedef float real;
typedef long long i64;
typedef float floatx16 __attribute__((ext_vector_type(16)));
#define FMA(a, b, c) __builtin_fmaf((a), (b), (c))
__device__ __forceinline__ floatx16 mfma32(float a, float b, floatx16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, c, 0, 0, 0);
}
)";

// Emits the CG producer for one (row, K) pair of path q: z0..z{d3-1}.
void emit_producer(Code& c, const UvwSpec& s, const UvwPath& q, const char* row, const char* kvar, const char* ind) {
  c.line("%sconst int pu = %s / %d, pv = %s - (%s / %d) * %d;", ind, kvar, q.mul2, kvar, kvar, q.mul2, q.mul2);
  c.line("%sconst real* xq = x + (i64)%s * %d + %d + pu * %d;", ind, row, s.in1, q.x_off, q.d1);
  c.line("%sconst real* yq = y + (i64)%s * %d + %d + pv * %d;", ind, row, s.in2, q.y_off, q.d2);
  std::set<int> is, js;
  for (const auto& t : q.terms) {
    is.insert(t.i);
    js.insert(t.j);
  }
  for (int i : is) c.line("%sconst real px%d = xq[%d];", ind, i, i);
  for (int j : js) c.line("%sconst real py%d = yq[%d];", ind, j, j);
  for (int k = 0; k < q.d3; ++k) c.line("%sreal z%d = 0;", ind, k);
  for (const auto& t : q.terms)
    c.line("%sz%d = FMA(%s, px%d * py%d, z%d);", ind, t.k, flit(t.c).c_str(), t.i, t.j, t.k);
}

// ---------------------------------------------------------------- forward
std::string emit_forward(const UvwSpec& s) {
  const Dims d = dims(s);
  const int ZW = d.kt + 4;  // padded row of the LDS tiles (keeps 16-byte alignment)
  Code c;
  c.s << kPrelude;
  c.line("extern \"C\" __global__ void __launch_bounds__(256) luna_uvw_fwd(");
  c.line("    const real* __restrict__ x, const real* __restrict__ y, const real* __restrict__ wt,");
  c.line("    real* __restrict__ out, int B) {");
  c.line("  __shared__ __attribute__((aligned(16))) real zs[%d][%d][%d];", d.d3max, kRows, ZW);
  c.line("  __shared__ __attribute__((aligned(16))) real ws[%d][%d];", d.npad, ZW);
  c.line("  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;");
  c.line("  const int b0 = blockIdx.x * %d;", kRows);
  c.line("  const int half = lane >> 5, col = lane & 31;");
  for (const OutBlock& blk : out_blocks(s)) {
    const int nt = round_up(blk.mul3, 32) / 32;
    const int tiles = blk.d3 * nt;
    const int per_wave = (tiles + 3) / 4;
    c.line("  {");
    c.line("    floatx16 acc[%d];", per_wave);
    c.line("    for (int t = 0; t < %d; ++t) acc[t] = (floatx16)(0.0f);", per_wave);
    for (int p : blk.paths) {
      const UvwPath& q = s.paths[p];
      const int K = q.mul1 * q.mul2;
      for (int k0 = 0; k0 < K; k0 += d.kt) {
        c.line("    __syncthreads();");
        // Stage Z tile: kRows x kt pairs (b, K).
        c.line("    for (int idx = tid; idx < %d; idx += 256) {", kRows * d.kt);
        c.line("      const int kk = idx %% %d, b = idx / %d, kg = %d + kk;", d.kt, d.kt, k0);
        c.line("      const int row = b0 + b;");
        c.line("      if (kg < %d && row < B) {", K);
        emit_producer(c, s, q, "row", "kg", "        ");
        for (int k = 0; k < q.d3; ++k) c.line("        zs[%d][b][kk] = z%d;", k, k);
        c.line("      } else {");
        for (int k = 0; k < q.d3; ++k) c.line("        zs[%d][b][kk] = 0;", k);
        c.line("      }");
        c.line("    }");
        // Stage W transposed: ws[n][kk] = W[k0 + kk, n].
        c.line("    for (int idx = tid; idx < %d; idx += 256) {", d.kt * d.npad);
        c.line("      const int n = idx %% %d, kk = idx / %d, kg = %d + kk;", d.npad, d.npad, k0);
        c.line("      ws[n][kk] = (kg < %d && n < %d) ? wt[%d + (i64)kg * %d + n] : 0.0f;", K, q.mul3, q.w_off,
               q.mul3);
        c.line("    }");
        c.line("    __syncthreads();");
        // Matrix-core contraction over this K tile.
        for (int t = 0; t < tiles; ++t) {
          const int owner = t % 4, slot = t / 4, k = t / nt, n0 = (t % nt) * 32;
          c.line("    if (wave == %d) {", owner);
          c.line("      floatx16 a_acc = acc[%d];", slot);
          c.line("      for (int s = 0; s < %d; s += 4) {", d.kt / 2);
          c.line("        const float4 av = *(const float4*)&zs[%d][col][half * %d + s];", k, d.kt / 2);
          c.line("        const float4 bv = *(const float4*)&ws[%d + col][half * %d + s];", n0, d.kt / 2);
          c.line("        a_acc = mfma32(av.x, bv.x, a_acc);");
          c.line("        a_acc = mfma32(av.y, bv.y, a_acc);");
          c.line("        a_acc = mfma32(av.z, bv.z, a_acc);");
          c.line("        a_acc = mfma32(av.w, bv.w, a_acc);");
          c.line("      }");
          c.line("      acc[%d] = a_acc;", slot);
          c.line("    }");
        }
      }
    }
    // Store: acc register r of lane holds row 8*(r/4) + 4*half + r%4, channel n0 + col.
    for (int t = 0; t < tiles; ++t) {
      const int owner = t % 4, slot = t / 4, k = t / nt, n0 = (t % nt) * 32;
      c.line("    if (wave == %d && %d + col < %d) {", owner, n0, blk.mul3);
      c.line("      for (int r = 0; r < 16; ++r) {");
      c.line("        const int row = b0 + 8 * (r >> 2) + 4 * half + (r & 3);");
      c.line("        if (row < B) out[(i64)row * %d + %d + (%d + col) * %d + %d] = acc[%d][r];", s.out, blk.out_off,
             n0, blk.d3, k, slot);
      c.line("      }");
      c.line("    }");
    }
    c.line("  }");
  }
  c.line("}");
  return c.s.str();
}

// Store mode of every gx tile in emission order ('S' first write, 'A'
// accumulate).  Tiles of paths that share an input block but split it into
// different channel ranges make first writes ambiguous; then every tile
// accumulates and the caller zero-fills gx.
std::vector<char> gx_modes(const UvwSpec& s, bool* all_accumulate) {
  const Dims d = dims(s);
  std::map<int, std::vector<char>> touched;  // x_off -> per-u flag
  std::vector<std::pair<int, std::pair<int, int>>> tiles;  // (x_off, [u0, u1))
  for (const OutBlock& blk : out_blocks(s))
    for (int p : blk.paths) {
      const UvwPath& q = s.paths[p];
      const int K = q.mul1 * q.mul2;
      for (int k0 = 0; k0 < K; k0 += d.kt) {
        const int ku = std::min(d.kt, K - k0);
        tiles.push_back({q.x_off, {k0 / q.mul2, (k0 + ku + q.mul2 - 1) / q.mul2}});
      }
    }
  std::vector<char> modes;
  bool mixed = false;
  for (const auto& t : tiles) {
    const UvwPath* owner = nullptr;
    for (const auto& q : s.paths)
      if (q.x_off == t.first) owner = &q;
    auto& flags = touched[t.first];
    if (flags.empty()) flags.assign(owner->mul1, 0);
    int count = 0;
    for (int u = t.second.first; u < t.second.second; ++u) count += flags[u];
    const int width = t.second.second - t.second.first;
    if (count != 0 && count != width) mixed = true;
    modes.push_back(count == 0 ? 'S' : 'A');
    for (int u = t.second.first; u < t.second.second; ++u) flags[u] = 1;
  }
  if (mixed)
    for (char& m : modes) m = 'A';
  *all_accumulate = mixed;
  return modes;
}

// ---------------------------------------------------------------- backward: gx, gy
std::string emit_backward_xy(const UvwSpec& s) {
  const Dims d = dims(s);
  const int GW = d.npad + 4;  // padded rows of the g tile
  const int ZW = d.kt + 4;
  Code c;
  c.s << kPrelude;
  c.line("extern \"C\" __global__ void __launch_bounds__(256) luna_uvw_bwd_xy(");
  c.line("    const real* __restrict__ x, const real* __restrict__ y, const real* __restrict__ wt,");
  c.line("    const real* __restrict__ g, real* __restrict__ gx, real* __restrict__ gy, int B) {");
  c.line("  __shared__ __attribute__((aligned(16))) real gs[%d][%d][%d];", d.d3max, kRows, GW);
  c.line("  __shared__ __attribute__((aligned(16))) real ws[%d][%d];", d.kt, GW);
  c.line("  __shared__ real dz[%d][%d][%d];", d.d3max, kRows, d.kt + 1);
  c.line("  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;");
  c.line("  const int b0 = blockIdx.x * %d;", kRows);
  c.line("  const int half = lane >> 5, col = lane & 31;");
  // First touch of each gx / gy range stores, later paths accumulate.
  bool all_accumulate = false;
  const std::vector<char> modes = gx_modes(s, &all_accumulate);
  size_t tile_index = 0;
  std::set<std::pair<int, int>> y_done;
  for (const OutBlock& blk : out_blocks(s)) {
    // Stage the output seed tile: gs[k][b][w] = g[b0+b, oo + w*d3 + k].
    c.line("  __syncthreads();");
    c.line("  for (int idx = tid; idx < %d; idx += 256) {", kRows * blk.mul3 * blk.d3);
    c.line("    const int b = idx / %d, rest = idx - b * %d;", blk.mul3 * blk.d3, blk.mul3 * blk.d3);
    c.line("    const int wch = rest / %d, k = rest - wch * %d;", blk.d3, blk.d3);
    c.line("    const int row = b0 + b;");
    c.line("    gs[k][b][wch] = row < B ? g[(i64)row * %d + %d + rest] : 0.0f;", s.out, blk.out_off);
    c.line("  }");
    if (round_up(blk.mul3, 32) > blk.mul3) {
      c.line("  for (int idx = tid; idx < %d; idx += 256) {", kRows * blk.d3 * (d.npad - blk.mul3));
      c.line("    const int pad = idx %% %d, rest = idx / %d;", d.npad - blk.mul3, d.npad - blk.mul3);
      c.line("    gs[rest / %d][rest %% %d][%d + pad] = 0.0f;", kRows, kRows, blk.mul3);
      c.line("  }");
    }
    const int nsteps = round_up(blk.mul3, 8) / 2;  // MFMA K steps over w, split in two halves
    for (int p : blk.paths) {
      const UvwPath& q = s.paths[p];
      const int K = q.mul1 * q.mul2;
      for (int k0 = 0; k0 < K; k0 += d.kt) {
        const int ntile = (std::min(d.kt, K - k0) + 31) / 32;
        const int tiles = q.d3 * ntile;
        c.line("  __syncthreads();");
        // ws[kk][w] = W[k0 + kk, w] (w contiguous, zero padded).
        c.line("  for (int idx = tid; idx < %d; idx += 256) {", d.kt * d.npad);
        c.line("    const int kk = idx / %d, n = idx - kk * %d, kg = %d + kk;", d.npad, d.npad, k0);
        c.line("    ws[kk][n] = (kg < %d && n < %d) ? wt[%d + (i64)kg * %d + n] : 0.0f;", K, q.mul3, q.w_off, q.mul3);
        c.line("  }");
        c.line("  __syncthreads();");
        // dZ[b, k, kk] = sum_w gs[k][b][w] ws[kk][w]: M = b, N = kk, K = w.
        for (int t = 0; t < tiles; ++t) {
          const int owner = t % 4, k = t / ntile, n0 = (t % ntile) * 32;
          c.line("  if (wave == %d) {", owner);
          c.line("    floatx16 a_acc = (floatx16)(0.0f);");
          c.line("    for (int s = 0; s < %d; s += 4) {", nsteps);
          c.line("      const float4 av = *(const float4*)&gs[%d][col][half * %d + s];", k, nsteps);
          c.line("      const float4 bv = *(const float4*)&ws[%d + col][half * %d + s];", n0, nsteps);
          c.line("      a_acc = mfma32(av.x, bv.x, a_acc);");
          c.line("      a_acc = mfma32(av.y, bv.y, a_acc);");
          c.line("      a_acc = mfma32(av.z, bv.z, a_acc);");
          c.line("      a_acc = mfma32(av.w, bv.w, a_acc);");
          c.line("    }");
          c.line("    for (int r = 0; r < 16; ++r) dz[%d][8 * (r >> 2) + 4 * half + (r & 3)][%d + col] = a_acc[r];", k,
                 n0);
          c.line("  }");
        }
        c.line("  __syncthreads();");
        // gx[b, u, i] += sum_{v, j, k} c y_vj dZ[b, k, (u, v)]; gy[b, v, j] += sum_{u, i, k} c x_ui dZ[...].
        // Wave w takes rows w, w+4, ...; lane = u (looping when mul1 > 64).
        const int ku = std::min(d.kt, K - k0);
        std::set<int> is, js;
        for (const auto& t : q.terms) {
          is.insert(t.i);
          js.insert(t.j);
        }
        const bool x_first = modes[tile_index++] == 'S';
        c.line("  for (int b = wave; b < %d; b += 4) {", kRows);
        c.line("    const int row = b0 + b;");
        c.line("    if (row >= B) break;");
        // y values of this row (uniform).
        c.line("    const real* yq = y + (i64)row * %d + %d;", s.in2, q.y_off);
        for (int v = 0; v < q.mul2; ++v)
          for (int j : js) c.line("    real gy%d_%d = 0;", v, j);
        c.line("    for (int uu = lane; uu < %d; uu += 64) {", (ku + q.mul2 - 1) / q.mul2);
        c.line("      const int u = %d + uu;", k0 / q.mul2);
        c.line("      const real* xq = x + (i64)row * %d + %d + u * %d;", s.in1, q.x_off, q.d1);
        for (int i : is) c.line("      const real px%d = xq[%d];", i, i);
        for (int i : is) c.line("      real ax%d = 0;", i);
        for (int v = 0; v < q.mul2; ++v) {
          c.line("      {");
          c.line("        const int kk = uu * %d + %d;", q.mul2, v);
          for (int k = 0; k < q.d3; ++k) c.line("        const real dz%d = dz[%d][b][kk];", k, k);
          for (const auto& t : q.terms) {
            c.line("        ax%d = FMA(%s, yq[%d] * dz%d, ax%d);", t.i, flit(t.c).c_str(), v * q.d2 + t.j, t.k, t.i);
            c.line("        gy%d_%d = FMA(%s, px%d * dz%d, gy%d_%d);", v, t.j, flit(t.c).c_str(), t.i, t.k, v, t.j);
          }
          c.line("      }");
        }
        c.line("      real* gq = gx + (i64)row * %d + %d + u * %d;", s.in1, q.x_off, q.d1);
        for (int i = 0; i < q.d1; ++i) {
          const std::string value = is.count(i) ? "ax" + std::to_string(i) : std::string("0.0f");
          if (x_first)
            c.line("      gq[%d] = %s;", i, value.c_str());
          else if (is.count(i))
            c.line("      gq[%d] += %s;", i, value.c_str());
        }
        c.line("    }");
        // Sum the gy partials over the 64 lanes and let lane 0 write them.
        for (int v = 0; v < q.mul2; ++v)
          for (int j : js) {
            c.line("    for (int m = 32; m >= 1; m >>= 1) gy%d_%d += __shfl_xor(gy%d_%d, m, 64);", v, j, v, j);
          }
        const bool y_first = y_done.insert({q.y_off, 0}).second && k0 == 0;
        c.line("    if (lane == 0) {");
        c.line("      real* gq = gy + (i64)row * %d + %d;", s.in2, q.y_off);
        for (int v = 0; v < q.mul2; ++v)
          for (int j = 0; j < q.d2; ++j) {
            const std::string value = js.count(j) ? "gy" + std::to_string(v) + "_" + std::to_string(j) : "0.0f";
            if (y_first)
              c.line("      gq[%d] = %s;", v * q.d2 + j, value.c_str());
            else if (js.count(j))
              c.line("      gq[%d] += %s;", v * q.d2 + j, value.c_str());
          }
        c.line("    }");
        c.line("  }");
      }
    }
  }
  c.line("}");
  return c.s.str();
}

// ---------------------------------------------------------------- backward: weights
std::string emit_backward_w(const UvwSpec& s) {
  const Dims d = dims(s);
  Code c;
  c.s << kPrelude;
  // One kernel per path (launch grid.y = path); each workgroup accumulates
  // dW_p over kChunkTiles row tiles and writes one partial.
  for (int p = 0; p < (int)s.paths.size(); ++p) {
    const UvwPath& q = s.paths[p];
    const int K = q.mul1 * q.mul2;
    const int Q = kRows * q.d3;          // MFMA K extent per row tile: (b, k) pairs
    const int QP = round_up(Q, 8);       // padded to two halves of 4-steps
    const int mt = round_up(K, 32) / 32, nt = round_up(q.mul3, 32) / 32;
    const int tiles = mt * nt;
    const int per_wave = (tiles + 3) / 4;
    c.line("extern \"C\" __global__ void __launch_bounds__(256) luna_uvw_bwd_w%d(", p);
    c.line("    const real* __restrict__ x, const real* __restrict__ y, const real* __restrict__ g,");
    c.line("    real* __restrict__ part, int B) {");
    c.line("  __shared__ __attribute__((aligned(16))) real zs[%d][%d];", mt * 32, QP + 4);
    c.line("  __shared__ __attribute__((aligned(16))) real gs[%d][%d];", nt * 32, QP + 4);
    c.line("  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;");
    c.line("  const int half = lane >> 5, col = lane & 31;");
    c.line("  floatx16 acc[%d];", per_wave);
    c.line("  for (int t = 0; t < %d; ++t) acc[t] = (floatx16)(0.0f);", per_wave);
    c.line("  for (int tile = 0; tile < %d; ++tile) {", kChunkTiles);
    c.line("    const int b0 = (blockIdx.x * %d + tile) * %d;", kChunkTiles, kRows);
    c.line("    if (b0 >= B) break;");
    c.line("    __syncthreads();");
    // zs[K][(b,k)] = Z_p[b, k, K]
    c.line("    for (int idx = tid; idx < %d; idx += 256) {", kRows * mt * 32);
    c.line("      const int kg = idx %% %d, b = idx / %d;", mt * 32, mt * 32);
    c.line("      const int row = b0 + b;");
    c.line("      if (kg < %d && row < B) {", K);
    emit_producer(c, s, q, "row", "kg", "        ");
    for (int k = 0; k < q.d3; ++k) c.line("        zs[kg][b * %d + %d] = z%d;", q.d3, k, k);
    c.line("      } else {");
    for (int k = 0; k < q.d3; ++k) c.line("        zs[kg][b * %d + %d] = 0.0f;", q.d3, k);
    c.line("      }");
    c.line("    }");
    // gs[w][(b,k)] = g[b0+b, oo + w*d3 + k]
    c.line("    for (int idx = tid; idx < %d; idx += 256) {", kRows * nt * 32 * q.d3);
    c.line("      const int b = idx / %d, rest = idx - b * %d;", nt * 32 * q.d3, nt * 32 * q.d3);
    c.line("      const int wch = rest / %d, k = rest - wch * %d;", q.d3, q.d3);
    c.line("      const int row = b0 + b;");
    c.line("      gs[wch][b * %d + k] = (row < B && wch < %d) ? g[(i64)row * %d + %d + rest] : 0.0f;", q.d3, q.mul3,
           s.out, q.out_off);
    c.line("    }");
    if (QP > Q) {
      c.line("    for (int idx = tid; idx < %d; idx += 256) {", (QP - Q) * (mt * 32 + nt * 32));
      c.line("      const int r = idx / %d, pad = idx - r * %d;", QP - Q, QP - Q);
      c.line("      if (r < %d) zs[r][%d + pad] = 0.0f; else gs[r - %d][%d + pad] = 0.0f;", mt * 32, Q, mt * 32, Q);
      c.line("    }");
    }
    c.line("    __syncthreads();");
    for (int t = 0; t < tiles; ++t) {
      const int owner = t % 4, slot = t / 4, m0 = (t / nt) * 32, n0 = (t % nt) * 32;
      c.line("    if (wave == %d) {", owner);
      c.line("      floatx16 a_acc = acc[%d];", slot);
      c.line("      for (int s = 0; s < %d; s += 4) {", QP / 2);
      c.line("        const float4 av = *(const float4*)&zs[%d + col][half * %d + s];", m0, QP / 2);
      c.line("        const float4 bv = *(const float4*)&gs[%d + col][half * %d + s];", n0, QP / 2);
      c.line("        a_acc = mfma32(av.x, bv.x, a_acc);");
      c.line("        a_acc = mfma32(av.y, bv.y, a_acc);");
      c.line("        a_acc = mfma32(av.z, bv.z, a_acc);");
      c.line("        a_acc = mfma32(av.w, bv.w, a_acc);");
      c.line("      }");
      c.line("      acc[%d] = a_acc;", slot);
      c.line("    }");
    }
    c.line("  }");
    // part[chunk][wo + K*mul3 + w]
    for (int t = 0; t < tiles; ++t) {
      const int owner = t % 4, slot = t / 4, m0 = (t / nt) * 32, n0 = (t % nt) * 32;
      c.line("  if (wave == %d && %d + col < %d) {", owner, n0, q.mul3);
      c.line("    for (int r = 0; r < 16; ++r) {");
      c.line("      const int kg = %d + 8 * (r >> 2) + 4 * half + (r & 3);", m0);
      c.line("      if (kg < %d) part[(i64)blockIdx.x * %d + %d + kg * %d + %d + col] = acc[%d][r];", K, s.wnum,
             q.w_off, q.mul3, n0, slot);
      c.line("    }");
      c.line("  }");
    }
    c.line("}");
  }
  c.line("extern \"C\" __global__ void __launch_bounds__(256) luna_uvw_bwd_w_reduce(");
  c.line("    const real* __restrict__ part, real* __restrict__ gw, int chunks) {");
  c.line("  const int i = blockIdx.x * 256 + threadIdx.x;");
  c.line("  if (i >= %d) return;", s.wnum);
  c.line("  real acc = 0;");
  c.line("  for (int n = 0; n < chunks; ++n) acc += part[(i64)n * %d + i];", s.wnum);
  c.line("  gw[i] = acc;");
  c.line("}");
  return c.s.str();
}

struct UvwPlan {
  UvwSpec spec;
  ModuleCache kernels;
  bool out_needs_zero = false, gx_needs_zero = false, gy_needs_zero = false, gw_needs_zero = false;
};

std::string source_for(const UvwPlan& plan, const std::string& variant) {
  if (variant == "fwd") return emit_forward(plan.spec);
  if (variant == "bxy") return emit_backward_xy(plan.spec);
  return emit_backward_w(plan.spec);
}

bool covers(const std::vector<std::pair<long, long>>& ranges, long total) {
  std::vector<std::pair<long, long>> r = ranges;
  std::sort(r.begin(), r.end());
  long at = 0;
  for (const auto& x : r) {
    if (x.first > at) return false;
    at = std::max(at, x.second);
  }
  return at >= total;
}

}  // namespace
}  // namespace luna

using namespace luna;

struct LunaUvwPlan {
  UvwPlan plan;
};

namespace {

hipModule_t module_for(UvwPlan& plan, const std::string& variant) {
  return plan.kernels.module_for(variant, [&] { return source_for(plan, variant); });
}

int64_t chunks_for(int64_t rows) {
  const int64_t per = (int64_t)kRows * kChunkTiles;
  return (rows + per - 1) / per;
}

}  // namespace

extern "C" {

int luna_uvw_plan_create(const char* spec, const char* cache_dir, LunaUvwPlan** out) {
  return guard_call([&] {
    if (!spec || !out) fail("luna_uvw_plan_create: null argument");
    auto holder = std::make_unique<LunaUvwPlan>();
    UvwPlan& p = holder->plan;
    p.spec = parse(spec);
    p.kernels.cache_dir = cache_dir ? cache_dir : "";
    p.kernels.tag = "uvw";
    std::vector<std::pair<long, long>> outs, xs, ys, ws;
    for (const auto& q : p.spec.paths) {
      outs.push_back({q.out_off, q.out_off + (long)q.mul3 * q.d3});
      xs.push_back({q.x_off, q.x_off + (long)q.mul1 * q.d1});
      ys.push_back({q.y_off, q.y_off + (long)q.mul2 * q.d2});
      ws.push_back({q.w_off, q.w_off + (long)q.mul1 * q.mul2 * q.mul3});
    }
    p.out_needs_zero = !covers(outs, p.spec.out);
    bool all_accumulate = false;
    gx_modes(p.spec, &all_accumulate);
    p.gx_needs_zero = !covers(xs, p.spec.in1) || all_accumulate;
    p.gy_needs_zero = !covers(ys, p.spec.in2);
    p.gw_needs_zero = !covers(ws, p.spec.wnum);
    *out = holder.release();
  });
}

int luna_uvw_plan_destroy(LunaUvwPlan* plan) {
  return guard_call([&] { delete plan; });
}

int luna_uvw_plan_needs_zero(const LunaUvwPlan* plan, int32_t* flags) {
  return guard_call([&] {
    if (!plan || !flags) fail("luna_uvw_plan_needs_zero: null argument");
    flags[0] = plan->plan.out_needs_zero;
    flags[1] = plan->plan.gx_needs_zero;
    flags[2] = plan->plan.gy_needs_zero;
    flags[3] = plan->plan.gw_needs_zero;
  });
}

int luna_uvw_plan_precompile(LunaUvwPlan* plan) {
  return guard_call([&] {
    if (!plan) fail("luna_uvw_plan_precompile: null plan");
    for (const char* v : {"fwd", "bxy", "bw"})
      plan->plan.kernels.code_for(v, [&] { return source_for(plan->plan, v); });
  });
}

int luna_uvw_fwd(const LunaUvwPlan* cplan, const void* x, const void* y, const void* weight, void* out,
                 int64_t rows, LunaStream stream) {
  return guard_call([&] {
    if (!cplan) fail("luna_uvw_fwd: null plan");
    if (rows < 0 || rows > 0x7fffffffLL) fail("luna_uvw_fwd: bad row count");
    if (rows == 0) return;
    if (!x || !y || !weight || !out) fail("luna_uvw_fwd: null tensor");
    UvwPlan& plan = const_cast<LunaUvwPlan*>(cplan)->plan;
    hipModule_t module = module_for(plan, "fwd");
    int B = (int)rows;
    void* args[] = {&x, &y, &weight, &out, &B};
    launch("uvw_fwd", function_for(module, "luna_uvw_fwd"), dim3((unsigned)((rows + kRows - 1) / kRows)), dim3(256),
           (hipStream_t)stream, args);
  });
}

int luna_uvw_bwd_workspace(const LunaUvwPlan* plan, int64_t rows, size_t* bytes) {
  return guard_call([&] {
    if (!plan || !bytes) fail("luna_uvw_bwd_workspace: null argument");
    if (rows < 0) fail("negative row count");
    *bytes = (size_t)chunks_for(rows) * (size_t)plan->plan.spec.wnum * sizeof(float);
  });
}

int luna_uvw_bwd(const LunaUvwPlan* cplan, const void* x, const void* y, const void* weight, const void* g,
                 void* gx, void* gy, void* gw, void* workspace, size_t workspace_bytes, int64_t rows,
                 LunaStream stream) {
  return guard_call([&] {
    if (!cplan) fail("luna_uvw_bwd: null plan");
    if (rows < 0 || rows > 0x7fffffffLL) fail("luna_uvw_bwd: bad row count");
    if (!x || !y || !weight || !g) fail("luna_uvw_bwd: null tensor");
    UvwPlan& plan = const_cast<LunaUvwPlan*>(cplan)->plan;
    hipStream_t s = (hipStream_t)stream;
    int B = (int)rows;
    if ((gx || gy) && rows > 0) {
      if (!gx || !gy) fail("luna_uvw_bwd: gx and gy are produced together");
      hipModule_t module = module_for(plan, "bxy");
      void* args[] = {&x, &y, &weight, &g, &gx, &gy, &B};
      launch("uvw_bwd_xy", function_for(module, "luna_uvw_bwd_xy"), dim3((unsigned)((rows + kRows - 1) / kRows)),
             dim3(256), s, args);
    }
    if (gw) {
      const int64_t chunks = chunks_for(rows);
      const size_t need = (size_t)chunks * (size_t)plan.spec.wnum * sizeof(float);
      if (rows > 0 && (!workspace || workspace_bytes < need)) fail("luna_uvw_bwd: workspace too small");
      hipModule_t module = module_for(plan, "bw");
      if (rows > 0) {
        for (int p = 0; p < (int)plan.spec.paths.size(); ++p) {
          void* args[] = {&x, &y, &g, &workspace, &B};
          launch("uvw_bwd_w", function_for(module, "luna_uvw_bwd_w" + std::to_string(p)), dim3((unsigned)chunks),
                 dim3(256), s, args);
        }
      }
      int n = (int)chunks;
      void* args[] = {&workspace, &gw, &n};
      launch("uvw_bwd_w_reduce", function_for(module, "luna_uvw_bwd_w_reduce"),
             dim3((unsigned)((plan.spec.wnum + 255) / 256)), dim3(256), s, args);
    }
  });
}

}  // extern "C"
