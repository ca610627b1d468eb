// ytm_jit.hip -- training kernels specialised per model at run time (hipRTC).
//
// The reference compiles its kernel source once per model with the hyperparameters and
// sizes pasted in as #defines (src/cutm/base.py:129-159, 244-256).  The same idea here:
// the training header (ytm_train.h) is compiled again by hipRTC with the resolved
// geometry as a `constexpr Geom`, so every size, loop bound and threshold is a compile-time
// constant.  The built-in kernels read the geometry from their kernel arguments; the two
// compile from the same device code and draw the same random numbers, so results are
// identical whichever runs.  Compiled modules are cached per process and device.
#include <hip/hip_runtime.h>
#include <hip/hiprtc.h>

#include <cinttypes>
#include <cstdio>
#include <cstdlib>
#include <functional>
#include <map>
#include <mutex>
#include <string>
#include <tuple>
#include <vector>

#include "ytm_internal.h"

namespace ytm {
namespace {

#include "gen_jit_sources.inc"  // kJitHeaderNames[], kJitHeaderSources[], kJitHeaderCount

void append_value(std::string* s, int64_t v) { *s += std::to_string(v) + "ll"; }
void append_value(std::string* s, int v) { *s += std::to_string(v); }
void append_value(std::string* s, uint32_t v) { *s += std::to_string(v) + "u"; }
void append_value(std::string* s, double v) {
  char buf[64];
  std::snprintf(buf, sizeof(buf), "%a", v);  // exact binary value
  *s += buf;
}

const char* kernel_name(TrainKind kind) {
  switch (kind) {
    case TrainKind::kResident: return "ytm_jit_train_resident";
    case TrainKind::kStream: return "ytm_jit_train_stream";
    case TrainKind::kGlobalVanilla: return "ytm_jit_train_global_vanilla";
    default: return "ytm_jit_train_global_conv";
  }
}

std::string kernel_source(const Geom& g, TrainKind kind, bool inject) {
  // draw counting (YTM_TRAIN_PROFILE=4) only in the kernels of counting runs
  const char* prof = std::getenv("YTM_TRAIN_PROFILE");
  std::string s = std::string("#define YTM_COUNT_DRAWS ") + (prof && std::atoi(prof) == 4 ? "1" : "0") + "\n";
  s += "#include \"ytm_train.h\"\nnamespace ytm {\nstatic constexpr Geom kJitGeom = {\n";
#define YTM_GEOM_PRINT(type, name) \
  s += "  /* " #name " */ ";       \
  append_value(&s, (type)g.name);  \
  s += ",\n";
  YTM_GEOM_FIELDS(YTM_GEOM_PRINT)
#undef YTM_GEOM_PRINT
  s += "};\n}  // namespace ytm\n";
  const char* inj = inject ? "true" : "false";
  s += "extern \"C\" __global__ __launch_bounds__(" + std::to_string(g.threads) + ") void ";
  s += kernel_name(kind);
  s += "(ytm::TrainArgs a) {\n  ";
  switch (kind) {
    case TrainKind::kResident:
      s += std::string("ytm::train_resident_body<") + inj + ">(a, ytm::kJitGeom);\n";
      break;
    case TrainKind::kStream:
      s += "ytm::train_stream_body(a, ytm::kJitGeom);\n";
      break;
    case TrainKind::kGlobalVanilla:
      s += std::string("ytm::train_global_body<true, ") + inj + ">(a, ytm::kJitGeom);\n";
      break;
    default:
      s += std::string("ytm::train_global_body<false, ") + inj + ">(a, ytm::kJitGeom);\n";
  }
  s += "}\n";
  return s;
}

struct Cache {
  std::mutex mu;
  std::map<std::pair<int, std::string>, hipFunction_t> fns;  // (device, source) -> kernel
  std::map<std::string, std::vector<char>> code;              // source -> code object
  std::vector<std::pair<int, hipModule_t>> modules;           // (device, module) loaded
};

Cache& cache() {
  // never destroyed (no static destructor runs at exit); jit_unload_all() unloads the
  // modules, which ytm_shutdown() calls before the process ends
  static Cache* c = new Cache();
  return *c;
}

}  // namespace

bool jit_enabled() {
  const char* e = std::getenv("YTM_JIT");
  return !(e && std::atoi(e) == 0);
}

bool jit_compile(const Geom& g, TrainKind kind, bool inject, std::vector<char>* code, std::string* why) {
  const std::string src = kernel_source(g, kind, inject);
  {
    std::lock_guard<std::mutex> lk(cache().mu);
    auto it = cache().code.find(src);
    if (it != cache().code.end()) {
      *code = it->second;
      return true;
    }
  }
  hiprtcProgram prog;
  hiprtcResult r = hiprtcCreateProgram(&prog, src.c_str(), "ytm_jit_train.hip", kJitHeaderCount, kJitHeaderSources,
                                       kJitHeaderNames);
  if (r != HIPRTC_SUCCESS) {
    if (why) *why = std::string("hiprtcCreateProgram: ") + hiprtcGetErrorString(r);
    return false;
  }
  // Same code generation rules as the built-in kernels: no contraction of the float and
  // double arithmetic that decides updates, no packed-fp32 VALU forms.
  const char* opts[] = {"--offload-arch=gfx950", "-O3", "-std=c++17", "-ffp-contract=off",
                        "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"};
  r = hiprtcCompileProgram(prog, (int)(sizeof(opts) / sizeof(opts[0])), opts);
  if (r != HIPRTC_SUCCESS) {
    size_t n = 0;
    std::string log;
    if (hiprtcGetProgramLogSize(prog, &n) == HIPRTC_SUCCESS && n > 1) {
      log.resize(n);
      hiprtcGetProgramLog(prog, &log[0]);
    }
    if (why) *why = std::string("hiprtcCompileProgram: ") + hiprtcGetErrorString(r) + "\n" + log;
    hiprtcDestroyProgram(&prog);
    return false;
  }
  size_t n = 0;
  r = hiprtcGetCodeSize(prog, &n);
  if (r == HIPRTC_SUCCESS) {
    code->resize(n);
    r = hiprtcGetCode(prog, code->data());
  }
  hiprtcDestroyProgram(&prog);
  if (r != HIPRTC_SUCCESS) {
    if (why) *why = std::string("hiprtcGetCode: ") + hiprtcGetErrorString(r);
    return false;
  }
  // YTM_JIT_DUMP=<directory>: keep each code object (and its source) for inspection.
  if (const char* dir = std::getenv("YTM_JIT_DUMP")) {
    const std::string base = std::string(dir) + "/" + kernel_name(kind) + (inject ? "_inject" : "") + "_" +
                             std::to_string(std::hash<std::string>()(src));
    if (FILE* f = std::fopen((base + ".co").c_str(), "wb")) {
      std::fwrite(code->data(), 1, code->size(), f);
      std::fclose(f);
    }
    if (FILE* f = std::fopen((base + ".hip").c_str(), "w")) {
      std::fputs(src.c_str(), f);
      std::fclose(f);
    }
  }
  std::lock_guard<std::mutex> lk(cache().mu);
  cache().code.emplace(src, *code);
  return true;
}

hipFunction_t jit_train_kernel(const Geom& g, TrainKind kind, bool inject, std::string* why) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) {
    if (why) *why = "hipGetDevice failed";
    return nullptr;
  }
  const std::string src = kernel_source(g, kind, inject);
  {
    std::lock_guard<std::mutex> lk(cache().mu);
    auto it = cache().fns.find({dev, src});
    if (it != cache().fns.end()) return it->second;
  }
  std::vector<char> code;
  if (!jit_compile(g, kind, inject, &code, why)) return nullptr;
  hipModule_t mod = nullptr;
  hipError_t e = hipModuleLoadData(&mod, code.data());
  if (e != hipSuccess) {
    if (why) *why = std::string("hipModuleLoadData: ") + hipGetErrorString(e);
    return nullptr;
  }
  hipFunction_t fn = nullptr;
  e = hipModuleGetFunction(&fn, mod, kernel_name(kind));
  if (e != hipSuccess) {
    if (why) *why = std::string("hipModuleGetFunction: ") + hipGetErrorString(e);
    (void)hipModuleUnload(mod);
    return nullptr;
  }
  std::lock_guard<std::mutex> lk(cache().mu);
  auto ins = cache().fns.emplace(std::make_pair(dev, src), fn);
  if (!ins.second) {  // another thread loaded the same kernel meanwhile: keep one module
    (void)hipModuleUnload(mod);
    return ins.first->second;
  }
  cache().modules.emplace_back(dev, mod);
  return fn;
}

int jit_unload_all() {
  std::lock_guard<std::mutex> lk(cache().mu);
  if (cache().modules.empty()) return 0;  // no HIP call at all (also on hosts without a GPU)
  int prev = 0;
  const bool have_prev = hipGetDevice(&prev) == hipSuccess;
  int failed = 0;
  for (const auto& dm : cache().modules) {
    if (hipSetDevice(dm.first) != hipSuccess || hipDeviceSynchronize() != hipSuccess ||
        hipModuleUnload(dm.second) != hipSuccess)
      ++failed;
  }
  cache().modules.clear();
  cache().fns.clear();
  if (have_prev) (void)hipSetDevice(prev);
  return failed;
}

hipError_t jit_occupancy(hipFunction_t fn, int threads, size_t lds_bytes, int* blocks_per_cu) {
  return hipModuleOccupancyMaxActiveBlocksPerMultiprocessor(blocks_per_cu, fn, threads, lds_bytes);
}

hipError_t launch_train_jit(hipFunction_t fn, const TrainArgs& a, int grid, int threads, size_t lds_bytes,
                            hipStream_t s) {
  TrainArgs copy = a;
  void* args[] = {&copy};
  return hipModuleLaunchCooperativeKernel(fn, (unsigned)grid, 1, 1, (unsigned)threads, 1, 1, (unsigned)lds_bytes, s,
                                          args);
}

}  // namespace ytm
