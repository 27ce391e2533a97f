// Shared runtime of the C-ABI library: error reporting, hipRTC compilation
// through the on-disk code-object cache, per-device module cache and timed
// launches.  Internal; the public interface is include/lunaeq_amd.h.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <exception>
#include <functional>
#include <map>
#include <mutex>
#include <string>
#include <vector>

namespace luna {

[[noreturn]] void fail(const std::string& message);
void check_hip(hipError_t status, const char* what);

// Compile HIP source for gfx950 with hipRTC, through the on-disk cache.
std::vector<char> compile_hip(const std::string& source, const std::string& cache_dir, const std::string& tag);

// Compiled code objects per variant and loaded modules per (variant, device).
struct ModuleCache {
  std::string cache_dir;
  std::string tag;  // file-name prefix in the code-object cache
  std::mutex lock;
  std::map<std::string, std::vector<char>> code;
  std::map<std::pair<std::string, int>, hipModule_t> modules;
  ~ModuleCache();
  const std::vector<char>& code_for(const std::string& variant, const std::function<std::string()>& source);
  hipModule_t module_for(const std::string& variant, const std::function<std::string()>& source);
};

hipFunction_t function_for(hipModule_t module, const std::string& name);

// Launch on `stream`; while profiling is enabled the launch is bracketed by
// HIP events recorded under `name`.
void launch(const std::string& name, hipFunction_t f, dim3 grid, dim3 block, hipStream_t stream, void** args,
            unsigned shared_bytes = 0);

// A second stream of the current device (created once, default priority,
// non-blocking), for work that may run beside the caller's stream.
hipStream_t side_stream();

// Runs `side` on side_stream() and `main` on `stream` concurrently: the side
// stream starts after everything already queued on `stream`, and `stream`
// continues only after the side work (events fork and join them, so a HIP
// graph captured on `stream` records both branches).
void fork_join(hipStream_t stream, const std::function<void(hipStream_t)>& side, const std::function<void()>& main);

// Runs body(); returns 0, or 1 with the message kept for luna_last_error().
int guard_call(const std::function<void()>& body);

}  // namespace luna
