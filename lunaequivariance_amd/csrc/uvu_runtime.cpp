// C-ABI entry points: plan lifetime, hipRTC compilation with an on-disk
// code-object cache, per-device module loading, and the launchers.
#include <hip/hip_runtime.h>
#include <hip/hiprtc.h>

#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <fstream>
#include <sstream>
#include <stdexcept>

#include "../../include/lunaeq_amd.h"
#include "uvu_plan.h"

namespace luna {

namespace {

thread_local std::string g_last_error;

struct Failure : std::runtime_error {
  using std::runtime_error::runtime_error;
};

uint64_t fnv1a(const std::string& text, uint64_t h = 1469598103934665603ULL) {
  for (unsigned char ch : text) {
    h ^= ch;
    h *= 1099511628211ULL;
  }
  return h;
}

// Options for every emitted module.  Packed FP32 instructions are disabled.
const char* kOptions[] = {
    "--offload-arch=gfx950", "-O3", "-ffp-contract=fast", "-Xclang", "-target-feature",
    "-Xclang", "-packed-fp32-ops", "-std=c++17",
};
constexpr int kNumOptions = sizeof(kOptions) / sizeof(kOptions[0]);

void check_hip(hipError_t status, const char* what) {
  if (status != hipSuccess) fail(std::string(what) + ": " + hipGetErrorString(status));
}

}  // namespace

void fail(const std::string& message) { throw Failure(message); }

std::vector<char> compile_hip(const std::string& source, const std::string& cache_dir,
                              const std::string& tag) {
  std::string key_text = source;
  for (int n = 0; n < kNumOptions; ++n) key_text += kOptions[n];
  key_text += "luna-uvu-1";
  char key[32];
  std::snprintf(key, sizeof(key), "%016llx", (unsigned long long)fnv1a(key_text));
  if (const char* dump = std::getenv("LUNAEQ_AMD_DUMP")) {
    std::ofstream out(std::string(dump) + "/" + tag + "_" + key + ".hip");
    out << source;
  }
  std::string path;
  if (!cache_dir.empty()) {
    path = cache_dir + "/" + tag + "_" + key + ".co";
    std::ifstream in(path, std::ios::binary);
    if (in) {
      std::vector<char> data((std::istreambuf_iterator<char>(in)), std::istreambuf_iterator<char>());
      if (!data.empty()) return data;
    }
  }
  hiprtcProgram program;
  if (hiprtcCreateProgram(&program, source.c_str(), (tag + ".hip").c_str(), 0, nullptr, nullptr) !=
      HIPRTC_SUCCESS)
    fail("hiprtcCreateProgram failed");
  hiprtcResult status = hiprtcCompileProgram(program, kNumOptions, kOptions);
  if (status != HIPRTC_SUCCESS) {
    size_t size = 0;
    hiprtcGetProgramLogSize(program, &size);
    std::string log(size, '\0');
    if (size) hiprtcGetProgramLog(program, &log[0]);
    hiprtcDestroyProgram(&program);
    fail("hipRTC compilation of " + tag + " failed: " + log.substr(0, 4000));
  }
  size_t size = 0;
  hiprtcGetCodeSize(program, &size);
  std::vector<char> data(size);
  hiprtcGetCode(program, data.data());
  hiprtcDestroyProgram(&program);
  if (!path.empty()) {
    mkdir(cache_dir.c_str(), 0755);
    // Write to a private name, then rename: concurrent builders never see a partial file.
    std::string tmp = path + ".tmp" + std::to_string(getpid());
    {
      std::ofstream out(tmp, std::ios::binary);
      out.write(data.data(), (std::streamsize)data.size());
    }
    std::rename(tmp.c_str(), path.c_str());
  }
  return data;
}

namespace {

std::string source_for(const Plan& plan, const std::string& variant) {
  // Variant names: fwd<env><l0> and bwd<env><gl0><gw><msg><part>, each flag '0' or '1'.
  auto flag = [&](size_t i) { return variant.size() > i && variant[i] == '1'; };
  if (variant.compare(0, 3, "fwd") == 0) return emit_forward(plan, flag(3), flag(4));
  return emit_backward(plan, flag(3), flag(4), flag(5), flag(6), flag(7));
}

const std::vector<char>& code_for(Plan& plan, const std::string& variant) {
  std::lock_guard<std::mutex> guard(plan.lock);
  auto it = plan.code.find(variant);
  if (it != plan.code.end()) return it->second;
  std::vector<char> data = compile_hip(source_for(plan, variant), plan.cache_dir, "uvu_" + variant);
  return plan.code.emplace(variant, std::move(data)).first->second;
}

hipModule_t module_for(Plan& plan, const std::string& variant) {
  int device = 0;
  check_hip(hipGetDevice(&device), "hipGetDevice");
  const std::vector<char>& data = code_for(plan, variant);
  std::lock_guard<std::mutex> guard(plan.lock);
  auto key = std::make_pair(variant, device);
  auto it = plan.modules.find(key);
  if (it != plan.modules.end()) return (hipModule_t)it->second;
  hipModule_t module;
  check_hip(hipModuleLoadData(&module, data.data()), "hipModuleLoadData");
  plan.modules[key] = module;
  return module;
}

hipFunction_t function_for(hipModule_t module, const std::string& name) {
  hipFunction_t function;
  check_hip(hipModuleGetFunction(&function, module, name.c_str()), ("hipModuleGetFunction " + name).c_str());
  return function;
}

// Optional per-launch timing with HIP events recorded on the launch stream.
struct ProfileRecord {
  std::string name;
  hipEvent_t start, stop;
};
std::mutex g_profile_lock;
bool g_profile_on = false;
std::vector<ProfileRecord> g_profile;

void launch(const std::string& name, hipFunction_t f, dim3 grid, dim3 block, hipStream_t stream,
            void** args) {
  ProfileRecord record{name, nullptr, nullptr};
  bool timed;
  {
    std::lock_guard<std::mutex> guard(g_profile_lock);
    timed = g_profile_on;
  }
  if (timed) {
    check_hip(hipEventCreate(&record.start), "hipEventCreate");
    check_hip(hipEventCreate(&record.stop), "hipEventCreate");
    check_hip(hipEventRecord(record.start, stream), "hipEventRecord");
  }
  check_hip(hipModuleLaunchKernel(f, grid.x, grid.y, grid.z, block.x, block.y, block.z, 0, stream, args,
                                  nullptr),
            "hipModuleLaunchKernel");
  check_hip(hipGetLastError(), "kernel launch");
  if (timed) {
    check_hip(hipEventRecord(record.stop, stream), "hipEventRecord");
    std::lock_guard<std::mutex> guard(g_profile_lock);
    g_profile.push_back(record);
  }
}

template <typename F>
int guarded(F body) {
  try {
    body();
    g_last_error.clear();
    return 0;
  } catch (const std::exception& error) {
    g_last_error = error.what();
    return 1;
  } catch (...) {
    g_last_error = "unknown error";
    return 1;
  }
}

}  // namespace
}  // namespace luna

using namespace luna;

struct LunaUvuPlan {
  Plan plan;
};

extern "C" {

const char* luna_last_error(void) { return g_last_error.c_str(); }

const char* luna_version(void) { return "lunaeq_amd 0.1 gfx950"; }

int luna_device_count(void) {
  int count = 0;
  if (hipGetDeviceCount(&count) != hipSuccess) return 0;
  return count;
}

int luna_uvu_plan_create(const char* spec, const char* cache_dir, LunaUvuPlan** out) {
  return guarded([&] {
    if (!spec || !out) fail("luna_uvu_plan_create: null argument");
    auto holder = std::make_unique<LunaUvuPlan>();
    holder->plan.spec = parse_spec(spec);
    holder->plan.cache_dir = cache_dir ? cache_dir : "";
    build_schedule(holder->plan);
    *out = holder.release();
  });
}

int luna_uvu_plan_destroy(LunaUvuPlan* plan) {
  return guarded([&] {
    if (!plan) return;
    for (auto& kv : plan->plan.modules) {
      int current = 0;
      (void)hipGetDevice(&current);
      (void)hipSetDevice(kv.first.second);
      (void)hipModuleUnload((hipModule_t)kv.second);
      (void)hipSetDevice(current);
    }
    delete plan;
  });
}

int luna_uvu_plan_info(const LunaUvuPlan* plan, LunaUvuPlanInfo* info) {
  return guarded([&] {
    if (!plan || !info) fail("luna_uvu_plan_info: null argument");
    const Plan& p = plan->plan;
    info->dtype_bits = p.spec.dtype_bits;
    info->in1_dim = p.spec.in1;
    info->in2_dim = p.spec.in2;
    info->out_dim = p.spec.out;
    info->weight_numel = p.spec.wnum;
    info->l0_dim = p.spec.l0_dim;
    info->num_paths = (int32_t)p.spec.paths.size();
    info->fwd_needs_zero = p.fwd_needs_zero;
    info->bwd_gx_needs_zero = p.bwd_gx_needs_zero;
    info->num_fwd_launches = p.fwd_phases;
    info->gy_parts = p.gy_parts;
  });
}

int luna_uvu_plan_precompile(LunaUvuPlan* plan) {
  return guarded([&] {
    if (!plan) fail("luna_uvu_plan_precompile: null plan");
    for (const char* v : {"fwd00", "bwd00111"}) code_for(plan->plan, v);
  });
}

int luna_uvu_conv_fwd(const LunaUvuPlan* cplan, const void* x, const void* y, const void* w,
                      const void* env, const int32_t* src, const int32_t* dst_rowptr,
                      const int32_t* node_order, void* out, void* l0, int64_t num_nodes,
                      int64_t num_edges, LunaStream stream) {
  return guarded([&] {
    if (!cplan) fail("luna_uvu_conv_fwd: null plan");
    Plan& plan = const_cast<LunaUvuPlan*>(cplan)->plan;
    if (num_nodes < 0 || num_edges < 0) fail("negative problem size");
    if (num_nodes > 0x7fffffffLL || num_edges > 0x7fffffffLL) fail("graph exceeds int32 indexing");
    if (num_nodes == 0) return;
    if (!x || !out || !dst_rowptr || !node_order) fail("luna_uvu_conv_fwd: null tensor");
    if (num_edges > 0 && (!y || !w || !src)) fail("luna_uvu_conv_fwd: null edge tensor");
    if (l0 && plan.spec.l0_dim == 0) l0 = nullptr;
    std::string variant = std::string("fwd") + (env ? '1' : '0') + (l0 ? '1' : '0');
    hipModule_t module = module_for(plan, variant);
    for (int phase = 0; phase < plan.fwd_phases; ++phase) {
      hipFunction_t f = function_for(module, "luna_uvu_fwd_p" + std::to_string(phase));
      void* args[] = {&x, &y, &w, &env, &src, &dst_rowptr, &node_order, &out, &l0};
      launch("uvu_fwd_p" + std::to_string(phase), f,
             dim3((unsigned)num_nodes, (unsigned)plan.phase_slots[phase]), dim3(64), (hipStream_t)stream,
             args);
    }
  });
}

namespace {

// Workspace layout: gy/genv partials, then the per-edge gx messages.
size_t align256(size_t n) { return (n + 255) & ~(size_t)255; }
size_t part_bytes(const Plan& p, int64_t num_edges) {
  return align256((size_t)p.gy_parts * (size_t)num_edges * (size_t)(p.spec.in2 + 1) * (p.spec.dtype_bits / 8));
}
size_t msg_bytes(const Plan& p, int64_t num_edges) {
  return align256((size_t)num_edges * (size_t)p.spec.in1 * (p.spec.dtype_bits / 8));
}

}  // namespace

int luna_uvu_conv_bwd_workspace(const LunaUvuPlan* plan, int64_t num_nodes, int64_t num_edges,
                                size_t* bytes) {
  return guarded([&] {
    if (!plan || !bytes) fail("luna_uvu_conv_bwd_workspace: null argument");
    if (num_nodes < 0 || num_edges < 0) fail("negative problem size");
    *bytes = part_bytes(plan->plan, num_edges) + msg_bytes(plan->plan, num_edges);
  });
}

int luna_uvu_conv_bwd(const LunaUvuPlan* cplan, const void* x, const void* y, const void* w,
                      const void* env, const void* g, const void* gl0, const int32_t* src,
                      const int32_t* dst_rowptr, const int32_t* node_order, const int32_t* src_rowptr,
                      const int32_t* edge_ids_by_src, void* gx, void* gy, void* gw, void* genv,
                      void* workspace, size_t workspace_bytes, int64_t num_nodes, int64_t num_edges,
                      LunaStream stream) {
  return guarded([&] {
    if (!cplan) fail("luna_uvu_conv_bwd: null plan");
    Plan& plan = const_cast<LunaUvuPlan*>(cplan)->plan;
    if (num_nodes < 0 || num_edges < 0) fail("negative problem size");
    if (num_nodes > 0x7fffffffLL || num_edges > 0x7fffffffLL) fail("graph exceeds int32 indexing");
    if (num_nodes == 0) return;
    if (!x || !g || !dst_rowptr || !node_order || !src_rowptr) fail("luna_uvu_conv_bwd: null tensor");
    if (num_edges > 0 && (!y || !w || !src || !edge_ids_by_src)) fail("luna_uvu_conv_bwd: null edge tensor");
    if (gl0 && plan.spec.l0_dim == 0) gl0 = nullptr;
    if (!env) genv = nullptr;
    int64_t E = num_edges;
    const bool want_parts = (gy || genv) && E > 0;
    const bool want_msg = gx && E > 0;
    const size_t pbytes = part_bytes(plan, E), mbytes = msg_bytes(plan, E);
    if ((want_parts || want_msg) && (!workspace || workspace_bytes < pbytes + mbytes))
      fail("luna_uvu_conv_bwd: workspace too small");
    void* part = want_parts ? workspace : nullptr;
    void* msg = want_msg ? (void*)((char*)workspace + pbytes) : nullptr;
    std::string variant = std::string("bwd") + (env ? '1' : '0') + (gl0 ? '1' : '0') + (gw ? '1' : '0') +
                          (want_msg ? '1' : '0') + (want_parts ? '1' : '0');
    hipModule_t module = module_for(plan, variant);
    hipStream_t s = (hipStream_t)stream;
    if (want_msg && plan.bwd_gx_needs_zero) {
      int64_t n = E * (int64_t)plan.spec.in1;
      void* args[] = {&msg, &n};
      launch("uvu_fill", function_for(module, "luna_uvu_fill"), dim3((unsigned)((n + 255) / 256)),
             dim3(256), s, args);
    }
    if (E > 0 && (gw || want_parts || want_msg)) {
      for (int phase = 0; phase < plan.bwd_phases; ++phase) {
        hipFunction_t f = function_for(module, "luna_uvu_bwd_p" + std::to_string(phase));
        void* args[] = {&x, &y, &w, &env, &g, &gl0, &src, &dst_rowptr, &node_order, &gw, &msg, &part, &E};
        launch("uvu_bwd_p" + std::to_string(phase), f,
               dim3((unsigned)num_nodes, (unsigned)plan.bwd_phase_slots[phase]), dim3(64), s, args);
      }
    }
    if (want_parts) {
      void* args[] = {&part, &gy, &genv, &E};
      launch("uvu_bwd_reduce", function_for(module, "luna_uvu_bwd_reduce"), dim3((unsigned)((E + 255) / 256)),
             dim3(256), s, args);
    }
    if (gx) {
      // With no edges the gather still writes zeros (every source row is empty).
      void* args[] = {&msg, &src_rowptr, &edge_ids_by_src, &gx};
      const int vec = gather_vector_width(plan);
      const int64_t per_block = 256LL * vec;
      launch("uvu_bwd_gather", function_for(module, "luna_uvu_bwd_gather"),
             dim3((unsigned)num_nodes, (unsigned)((plan.spec.in1 + per_block - 1) / per_block)), dim3(256), s,
             args);
    }
  });
}

int luna_profile_enable(int on) {
  return guarded([&] {
    std::lock_guard<std::mutex> guard(g_profile_lock);
    g_profile_on = on != 0;
  });
}

int luna_profile_collect(char* buffer, size_t capacity, size_t* needed) {
  return guarded([&] {
    std::vector<ProfileRecord> records;
    {
      std::lock_guard<std::mutex> guard(g_profile_lock);
      records.swap(g_profile);
    }
    std::map<std::string, std::vector<float>> times;
    for (auto& r : records) {
      check_hip(hipEventSynchronize(r.stop), "hipEventSynchronize");
      float ms = 0.f;
      check_hip(hipEventElapsedTime(&ms, r.start, r.stop), "hipEventElapsedTime");
      times[r.name].push_back(ms);
      (void)hipEventDestroy(r.start);
      (void)hipEventDestroy(r.stop);
    }
    std::ostringstream text;
    for (auto& kv : times) {
      double total = 0, lo = 1e30, hi = 0;
      for (float t : kv.second) {
        total += t;
        lo = std::min(lo, (double)t);
        hi = std::max(hi, (double)t);
      }
      text << kv.first << ' ' << kv.second.size() << ' ' << total << ' ' << lo << ' ' << hi << '\n';
    }
    std::string out = text.str();
    if (needed) *needed = out.size() + 1;
    if (buffer && capacity) {
      size_t n = std::min(capacity - 1, out.size());
      std::memcpy(buffer, out.data(), n);
      buffer[n] = '\0';
    }
  });
}

}  // extern "C"
