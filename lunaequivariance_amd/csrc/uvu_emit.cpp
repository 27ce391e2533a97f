// HIP source emitter for the UVU convolution kernels of one path set.
//
// Every Clebsch-Gordan coefficient becomes a literal in straight-line code, so
// a wave holds all partial products and output accumulators of its group in
// VGPRs while edge attributes and graph indices, which are uniform across the
// wave, come through scalar loads.  One lane owns one channel u of a
// 64-channel chunk.
//
// Forward (dst-owned, as the reference's ordered forward kernel,
// src/lunatp/uvu_conv/kernels/forward.py:398-427):
//   out[t, ob + u*d3 + k] = sum_{e in row t} env[e] * w[e, wo + u*ws]
//                           * sum_{(i,j,k)} c_ijk x[src[e], xb + u*d1 + i] y[e, yb + j]
// Backward (src-owned, as src/lunatp/uvu_conv/kernels/backward.py:183-333):
//   q_ij = sum_k c_ijk G_k with G = env[e] * g[dst[e]] (+ gl0 for scalar paths)
//   gw[e, wo + u*ws] = sum_ij x_i y_j q_ij
//   gx[s, xb + u*d1 + i] = sum_e w sum_j y_j q_ij
//   gy[e, yb + j] = sum_u w sum_i x_i q_ij      (partials per wave, then reduced)
//   genv[e] = sum_u sum_k w g_k t_k, t_k = sum c x_i y_j
#include <cstdio>
#include <map>
#include <set>
#include <sstream>

#include "uvu_plan.h"

namespace luna {

namespace {

struct Code {
  std::ostringstream s;
  template <typename... A>
  void line(const char* fmt, A... args) {
    char buffer[1024];
    std::snprintf(buffer, sizeof(buffer), fmt, args...);
    s << buffer << '\n';
  }
  void raw(const std::string& text) { s << text; }
};

std::string literal(double c, int bits) {
  char buffer[64];
  if (bits == 64) {
    std::snprintf(buffer, sizeof(buffer), "%.17e", c);
  } else {
    std::snprintf(buffer, sizeof(buffer), "%.9ef", (double)(float)c);
  }
  return buffer;
}

std::string prelude(const Spec& spec) {
  std::ostringstream s;
  const bool fp64 = spec.dtype_bits == 64;
  s << "typedef " << (fp64 ? "double" : "float") << " real;\n";
  s << "typedef long long i64;\n";
  s << "#define FMA(a, b, c) " << (fp64 ? "__builtin_fma" : "__builtin_fmaf") << "((a), (b), (c))\n";
  s << "#define IN1 " << spec.in1 << "LL\n";
  s << "#define IN2 " << spec.in2 << "LL\n";
  s << "#define OUTD " << spec.out << "LL\n";
  s << "#define WNUM " << spec.wnum << "LL\n";
  s << "#define L0DIM " << spec.l0_dim << "LL\n";
  s << R"(
__device__ __forceinline__ real wave_sum(real v) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) v += __shfl_xor(v, m, 64);
  return v;
}
)";
  return s.str();
}

// Distinct edge-attribute indices and (i, y) products used by a group.
struct GroupUse {
  std::set<int> ys;                       // absolute y indices
  std::set<std::pair<int, int>> products; // (i, absolute y)
};

GroupUse group_use(const Spec& spec, const Group& g) {
  GroupUse use;
  for (int p : g.paths) {
    const Path& q = spec.paths[p];
    for (const Term& t : q.terms) {
      use.ys.insert(q.y_off + t.j);
      use.products.insert({t.i, q.y_off + t.j});
    }
  }
  return use;
}

void emit_forward_group(Code& c, const Spec& spec, const Group& g, bool env, bool l0) {
  const int bits = spec.dtype_bits;
  GroupUse use = group_use(spec, g);
  c.line("    const int u = (slot - %d) * 64 + lane;", g.slot_base);
  c.line("    const bool active = u < %d;", g.channels);
  c.line("    const int uc = active ? u : %d;", g.channels - 1);
  for (size_t b = 0; b < g.blocks.size(); ++b)
    for (int k = 0; k < g.blocks[b].d3; ++k) c.line("    real A%zu_%d = 0;", b, k);
  c.line("    for (int e = beg; e < end; ++e) {");
  c.line("      const int s = src[e];");
  c.line("      const real* xr = x + (i64)s * IN1 + (%d + uc * %d);", g.x_off, g.d1);
  for (int i = 0; i < g.d1; ++i) c.line("      const real x%d = xr[%d];", i, i);
  c.line("      const real* yr = y + (i64)e * IN2;");
  for (int yi : use.ys) c.line("      const real y%d = yr[%d];", yi, yi);
  c.line("      const real* wr = w + (i64)e * WNUM;");
  if (env) c.line("      const real ev = env[e];");
  for (const auto& pr : use.products)
    c.line("      const real p%d_%d = x%d * y%d;", pr.first, pr.second, pr.first, pr.second);
  // l0 columns are summed over the paths (edge copies) sharing them.
  std::map<int, std::vector<int>> l0_cols;
  for (size_t n = 0; n < g.paths.size(); ++n) {
    const Path& q = spec.paths[g.paths[n]];
    if (l0 && q.l0_col >= 0) l0_cols[q.l0_col].push_back((int)n);
  }
  for (const auto& col : l0_cols) c.line("      real L%d = 0;", col.first);
  for (size_t n = 0; n < g.paths.size(); ++n) {
    const Path& q = spec.paths[g.paths[n]];
    const int b = g.path_block[n];
    c.line("      {");
    c.line("        const real wraw = wr[%d + uc * %d];", q.w_off, q.w_stride);
    c.line("        const real wv = %s;", env ? "wraw * ev" : "wraw");
    std::map<int, std::vector<const Term*>> by_k;
    for (const Term& t : q.terms) by_k[t.k].push_back(&t);
    for (const auto& kv : by_k) {
      const int k = kv.first;
      bool first = true;
      for (const Term* t : kv.second) {
        std::string coef = literal(t->c, bits);
        if (first) {
          c.line("        real t%d = %s * p%d_%d;", k, coef.c_str(), t->i, q.y_off + t->j);
          first = false;
        } else {
          c.line("        t%d = FMA(%s, p%d_%d, t%d);", k, coef.c_str(), t->i, q.y_off + t->j, k);
        }
      }
      c.line("        A%d_%d = FMA(wv, t%d, A%d_%d);", b, k, k, b, k);
    }
    if (l0 && q.l0_col >= 0) {
      if (by_k.count(0))
        c.line("        L%d = FMA(wraw, t0, L%d);", q.l0_col, q.l0_col);
    }
    c.line("      }");
  }
  for (const auto& col : l0_cols)
    c.line("      if (l0 && active) l0[(i64)e * L0DIM + %d + u] = L%d;", col.first, col.first);
  c.line("    }");
  c.line("    if (active) {");
  for (size_t b = 0; b < g.blocks.size(); ++b) {
    const AccBlock& blk = g.blocks[b];
    c.line("      real* o%zu = out + (i64)t * OUTD + (%d + u * %d);", b, blk.out_off, blk.d3);
    for (int k = 0; k < blk.d3; ++k) {
      if (blk.accumulate)
        c.line("      o%zu[%d] += A%zu_%d;", b, k, b, k);
      else
        c.line("      o%zu[%d] = A%zu_%d;", b, k, b, k);
    }
  }
  c.line("    }");
}

void emit_backward_group(Code& c, const Spec& spec, const Group& g, bool env, bool gl0) {
  const int bits = spec.dtype_bits;
  GroupUse use = group_use(spec, g);
  const int pw = spec.in2 + (env ? 1 : 0);
  c.line("    const int u = (slot - %d) * 64 + lane;", g.slot_base);
  c.line("    const bool active = u < %d;", g.channels);
  c.line("    const int uc = active ? u : %d;", g.channels - 1);
  c.line("    const real* xr = x + (i64)s * IN1 + (%d + uc * %d);", g.x_off, g.d1);
  for (int i = 0; i < g.d1; ++i) c.line("    const real x%d = xr[%d];", i, i);
  for (int i = 0; i < g.d1; ++i) c.line("    real GX%d = 0;", i);
  c.line("    for (int pos = beg; pos < end; ++pos) {");
  c.line("      const int e = ebs[pos];");
  c.line("      const int d = dst[e];");
  c.line("      const real* yr = y + (i64)e * IN2;");
  for (int yi : use.ys) c.line("      const real y%d = yr[%d];", yi, yi);
  c.line("      const real* wr = w + (i64)e * WNUM;");
  if (env) c.line("      const real ev = env[e];");
  for (size_t b = 0; b < g.blocks.size(); ++b) {
    const AccBlock& blk = g.blocks[b];
    c.line("      const real* g%zu = g + (i64)d * OUTD + (%d + uc * %d);", b, blk.out_off, blk.d3);
    for (int k = 0; k < blk.d3; ++k) {
      c.line("      const real G%zu_%d = g%zu[%d];", b, k, b, k);
      c.line("      const real H%zu_%d = %s;", b, k, env ? ("ev * G" + std::to_string(b) + "_" + std::to_string(k)).c_str()
                                                       : ("G" + std::to_string(b) + "_" + std::to_string(k)).c_str());
    }
  }
  for (int yi : use.ys) c.line("      real GY%d = 0;", yi);
  if (env) {
    c.line("      real GE = 0;");
    for (const auto& pr : use.products)
      c.line("      const real p%d_%d = x%d * y%d;", pr.first, pr.second, pr.first, pr.second);
  }
  for (size_t n = 0; n < g.paths.size(); ++n) {
    const Path& q = spec.paths[g.paths[n]];
    const int b = g.path_block[n];
    c.line("      {");
    c.line("        const real wv = active ? wr[%d + uc * %d] : (real)0;", q.w_off, q.w_stride);
    const bool scalar_seed = gl0 && q.l0_col >= 0;
    if (scalar_seed) c.line("        const real S0 = H%d_0 + gl0[(i64)e * L0DIM + %d + uc];", b, q.l0_col);
    // q_ij for every (i, j) pair of the path.
    std::map<std::pair<int, int>, std::vector<const Term*>> by_ij;
    for (const Term& t : q.terms) by_ij[{t.i, t.j}].push_back(&t);
    std::set<int> is, js;
    for (const auto& kv : by_ij) {
      is.insert(kv.first.first);
      js.insert(kv.first.second);
    }
    for (int j : js) c.line("        real b%d = 0;", j);
    for (int i : is) c.line("        real a%d = 0;", i);
    for (const auto& kv : by_ij) {
      const int i = kv.first.first, j = kv.first.second;
      bool first = true;
      for (const Term* t : kv.second) {
        std::string coef = literal(t->c, bits);
        std::string seed = (scalar_seed && t->k == 0) ? std::string("S0")
                                                      : "H" + std::to_string(b) + "_" + std::to_string(t->k);
        if (first) {
          c.line("        real q%d_%d = %s * %s;", i, j, coef.c_str(), seed.c_str());
          first = false;
        } else {
          c.line("        q%d_%d = FMA(%s, %s, q%d_%d);", i, j, coef.c_str(), seed.c_str(), i, j);
        }
      }
      c.line("        b%d = FMA(x%d, q%d_%d, b%d);", j, i, i, j, j);
      c.line("        a%d = FMA(y%d, q%d_%d, a%d);", i, q.y_off + j, i, j, i);
    }
    // gw = sum_j y_j b_j
    bool first = true;
    for (int j : js) {
      if (first) {
        c.line("        real gwv = y%d * b%d;", q.y_off + j, j);
        first = false;
      } else {
        c.line("        gwv = FMA(y%d, b%d, gwv);", q.y_off + j, j);
      }
    }
    if (first) c.line("        real gwv = 0;");
    c.line("        if (gw && active) gw[(i64)e * WNUM + %d + u * %d] = gwv;", q.w_off, q.w_stride);
    for (int j : js) c.line("        GY%d = FMA(wv, b%d, GY%d);", q.y_off + j, j, q.y_off + j);
    for (int i : is) c.line("        GX%d = FMA(wv, a%d, GX%d);", i, i, i);
    if (env) {
      // genv: sum_k g_k t_k with t_k = sum c x_i y_j (raw output seed, no gl0).
      std::map<int, std::vector<const Term*>> by_k;
      for (const Term& t : q.terms) by_k[t.k].push_back(&t);
      c.line("        real tg = 0;");
      for (const auto& kv : by_k) {
        const int k = kv.first;
        bool f2 = true;
        for (const Term* t : kv.second) {
          std::string coef = literal(t->c, bits);
          if (f2) {
            c.line("        real t%d = %s * p%d_%d;", k, coef.c_str(), t->i, q.y_off + t->j);
            f2 = false;
          } else {
            c.line("        t%d = FMA(%s, p%d_%d, t%d);", k, coef.c_str(), t->i, q.y_off + t->j, k);
          }
        }
        c.line("        tg = FMA(G%d_%d, t%d, tg);", b, k, k);
      }
      c.line("        GE = FMA(wv, tg, GE);");
    }
    c.line("      }");
  }
  // Reduce the edge-attribute partials over the wave's channels.
  c.line("      real* pr = part + ((i64)(%d + (slot - %d)) * E + e) * %d;", g.gy_slot_base, g.slot_base, pw);
  for (int yi : use.ys) {
    c.line("      GY%d = wave_sum(GY%d);", yi, yi);
    c.line("      if (lane == 0 && part) pr[%d] = GY%d;", yi, yi);
  }
  if (env) {
    c.line("      GE = wave_sum(GE);");
    c.line("      if (lane == 0 && part) pr[%d] = GE;", spec.in2);
  }
  c.line("    }");
  c.line("    if (gx && active) {");
  c.line("      real* gxr = gx + (i64)s * IN1 + (%d + u * %d);", g.x_off, g.d1);
  for (int i = 0; i < g.d1; ++i) {
    if (g.gx_accumulate)
      c.line("      gxr[%d] += GX%d;", i, i);
    else
      c.line("      gxr[%d] = GX%d;", i, i);
  }
  c.line("    }");
}

}  // namespace

std::string emit_forward(const Plan& plan, bool env, bool l0) {
  const Spec& spec = plan.spec;
  Code c;
  c.raw(prelude(spec));
  for (int phase = 0; phase < plan.fwd_phases; ++phase) {
    c.line("extern \"C\" __global__ void __launch_bounds__(64) luna_uvu_fwd_p%d(", phase);
    c.line("    const real* __restrict__ x, const real* __restrict__ y, const real* __restrict__ w,");
    c.line("    const real* __restrict__ env, const int* __restrict__ src, const int* __restrict__ rowptr,");
    c.line("    const int* __restrict__ order, real* __restrict__ out, real* __restrict__ l0) {");
    c.line("  const int lane = threadIdx.x;");
    c.line("  const int t = order[blockIdx.x];");
    c.line("  const int beg = rowptr[t];");
    c.line("  const int end = rowptr[t + 1];");
    c.line("  const int slot = blockIdx.y;");
    bool first = true;
    for (const Group& g : plan.fwd_groups) {
      if (g.phase != phase) continue;
      c.line("  %sif (slot < %d) {", first ? "" : "else ", g.slot_base + g.chunks);
      first = false;
      emit_forward_group(c, spec, g, env, l0);
      c.line("  }");
    }
    c.line("}");
  }
  return c.s.str();
}

std::string emit_backward(const Plan& plan, bool env, bool gl0) {
  const Spec& spec = plan.spec;
  const int pw = spec.in2 + (env ? 1 : 0);
  Code c;
  c.raw(prelude(spec));
  for (int phase = 0; phase < plan.bwd_phases; ++phase) {
    c.line("extern \"C\" __global__ void __launch_bounds__(64) luna_uvu_bwd_p%d(", phase);
    c.line("    const real* __restrict__ x, const real* __restrict__ y, const real* __restrict__ w,");
    c.line("    const real* __restrict__ env, const real* __restrict__ g, const real* __restrict__ gl0,");
    c.line("    const int* __restrict__ dst, const int* __restrict__ srow, const int* __restrict__ ebs,");
    c.line("    const int* __restrict__ sorder, real* __restrict__ gx, real* __restrict__ gw,");
    c.line("    real* __restrict__ part, i64 E) {");
    c.line("  const int lane = threadIdx.x;");
    c.line("  const int s = sorder[blockIdx.x];");
    c.line("  const int beg = srow[s];");
    c.line("  const int end = srow[s + 1];");
    c.line("  const int slot = blockIdx.y;");
    bool first = true;
    for (const Group& g : plan.bwd_groups) {
      if (g.phase != phase) continue;
      c.line("  %sif (slot < %d) {", first ? "" : "else ", g.slot_base + g.chunks);
      first = false;
      emit_backward_group(c, spec, g, env, gl0);
      c.line("  }");
    }
    c.line("}");
  }
  // Reduction of the per-wave partials into gy (and genv).  Table: for each
  // partial column, the slots that wrote it.
  std::vector<std::vector<int>> writers(pw);
  for (const Group& g : plan.bwd_groups) {
    GroupUse use = group_use(spec, g);
    for (int chunk = 0; chunk < g.chunks; ++chunk) {
      for (int yi : use.ys) writers[yi].push_back(g.gy_slot_base + chunk);
      if (env) writers[spec.in2].push_back(g.gy_slot_base + chunk);
    }
  }
  std::vector<int> begin(pw + 1, 0), ids;
  for (int col = 0; col < pw; ++col) {
    begin[col] = (int)ids.size();
    for (int s : writers[col]) ids.push_back(s);
  }
  begin[pw] = (int)ids.size();
  c.s << "__constant__ int reduce_begin[" << pw + 1 << "] = {";
  for (int v : begin) c.s << v << ",";
  c.s << "};\n__constant__ int reduce_slot[" << (ids.empty() ? 1 : ids.size()) << "] = {";
  for (int v : ids) c.s << v << ",";
  if (ids.empty()) c.s << "0";
  c.s << "};\n";
  c.line("extern \"C\" __global__ void __launch_bounds__(256) luna_uvu_bwd_reduce(");
  c.line("    const real* __restrict__ part, real* __restrict__ gy, real* __restrict__ genv, i64 E) {");
  c.line("  const i64 idx = (i64)blockIdx.x * 256 + threadIdx.x;");
  c.line("  if (idx >= E * %d) return;", pw);
  c.line("  const i64 e = idx / %d;", pw);
  c.line("  const int col = (int)(idx - e * %d);", pw);
  c.line("  real acc = 0;");
  c.line("  for (int n = reduce_begin[col]; n < reduce_begin[col + 1]; ++n)");
  c.line("    acc += part[(i64)reduce_slot[n] * E * %d + idx];", pw);
  c.line("  if (col < %d) { if (gy) gy[e * IN2 + col] = acc; }", spec.in2);
  if (env) c.line("  else if (genv) genv[e] = acc;");
  c.line("}");
  return c.s.str();
}

}  // namespace luna
