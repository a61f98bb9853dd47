// C-ABI implementation (include/nablatensor_rocm.h) over the HIP runtime and
// hipRTC. Replaces the reference's FFM runtime surface (nablatensor-engine-rocm/
// .../backend/rocm/HipRuntime.java:79-446, HipCompute.java:26-125) and the
// device executable (nablatensor-core/.../engine/DeviceAadExecutable.java:43-222).
#include "nablatensor_rocm.h"

#include <amd_comgr/amd_comgr.h>
#include <dlfcn.h>
#include <hip/hip_runtime.h>
#include <hip/hiprtc.h>
#include <sys/stat.h>
#include <utime.h>

#include <algorithm>
#include <chrono>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <fstream>
#include <map>
#include <memory>
#include <mutex>
#include <sstream>
#include <string>
#include <vector>

#include "lower.hpp"
#include "nt_testing.h"
#include "nt_exec.hpp"
#include "skeleton_src.inc"

namespace ntr {

namespace {
thread_local std::string g_err;
}  // namespace

int fail(int code, const std::string& msg) {
  g_err = msg;
  return code;
}

int hip_fail(hipError_t e, const char* what) {
  std::ostringstream s;
  s << what << " failed: " << hipGetErrorString(e) << " (code " << static_cast<int>(e) << ")";
  return fail(static_cast<int>(e), s.str());
}

const char* last_error() { return g_err.c_str(); }

}  // namespace ntr

using ntr::fail;
using ntr::hip_fail;
using ntr::Lowered;
using ntr::MarketVariant;

namespace {

const char* kArch = "gfx950";

// ---- code-object cache ---------------------------------------------------------

uint64_t fnv1a(const std::string& s, uint64_t h = 1469598103934665603ull) {
  for (unsigned char ch : s) {
    h ^= ch;
    h *= 1099511628211ull;
  }
  return h;
}

std::string cache_dir() {
  const char* env = std::getenv("NABLATENSOR_ROCM_CACHE");
  if (env && std::strcmp(env, "off") == 0) return "";
  if (env && *env) return env;
  Dl_info info;
  if (dladdr(reinterpret_cast<void*>(&cache_dir), &info) && info.dli_fname) {
    std::string path(info.dli_fname);
    size_t slash = path.rfind('/');
    if (slash != std::string::npos) return path.substr(0, slash) + "/_kcache";
  }
  return "";
}

bool read_file(const std::string& path, std::vector<char>& out) {
  std::ifstream f(path, std::ios::binary);
  if (!f) return false;
  out.assign(std::istreambuf_iterator<char>(f), std::istreambuf_iterator<char>());
  return !out.empty();
}

void write_file_atomic(const std::string& path, const std::vector<char>& data) {
  const std::string tmp = path + ".tmp" + std::to_string(reinterpret_cast<uintptr_t>(&data));
  {
    std::ofstream f(tmp, std::ios::binary);
    if (!f) return;
    f.write(data.data(), static_cast<std::streamsize>(data.size()));
  }
  std::rename(tmp.c_str(), path.c_str());
}

// Target features the generated source asks to turn off, from its
// "// nt-compile: -feature ..." line.
std::vector<std::string> source_features(const std::string& src) {
  std::vector<std::string> out;
  const std::string tag = "// nt-compile:";
  const size_t at = src.find(tag);
  if (at == std::string::npos) return out;
  std::istringstream line(src.substr(at + tag.size(), src.find('\n', at) - at - tag.size()));
  std::string f;
  while (line >> f) {
    if (f.size() > 1 && f[0] == '-') out.push_back(f);
  }
  return out;
}

// Byte alignment of every loop's first instruction (clang's -falign-loops).
// The replay kernels are one hot loop that issues a VALU instruction on most
// cycles, and where that loop starts relative to the instruction cache lines
// is worth up to 8 % (the barrier fp32 kernel: the same instructions ran 4.02
// or 4.34 ms per 2x10^7 paths depending on the loop's offset within its 64-byte
// line). NABLATENSOR_ROCM_ALIGN_LOOPS sets it (a power of two; 0 leaves
// placement to the compiler).
int loop_alignment() {
  const char* env = std::getenv("NABLATENSOR_ROCM_ALIGN_LOOPS");
  if (!env || !*env) return 64;
  const int v = std::atoi(env);
  return (v > 0 && (v & (v - 1)) == 0 && v <= 4096) ? v : 0;
}

std::vector<std::string> compile_options(const std::string& src, bool dump) {
  std::vector<std::string> o = {std::string("--offload-arch=") + kArch, "-O3", "-std=c++17",
                                "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"};
  if (const int align = loop_alignment()) o.push_back("-falign-loops=" + std::to_string(align));
  for (const auto& f : source_features(src)) {
    o.insert(o.end(), {"-Xclang", "-target-feature", "-Xclang", f});
  }
  if (dump) o.push_back("-DNT_DUMP_PATHS=1");
  return o;
}

// Text appended to every program this thread compiles (nt_testing.h): lets a
// test make hipRTC fail on a real lowering and check the error path. Empty in
// every other use.
thread_local std::string t_test_source_suffix;

int compile_hiprtc(const std::string& lowered, bool dump, std::vector<char>& code, double& seconds) {
  const std::string& src = t_test_source_suffix.empty() ? lowered : lowered + t_test_source_suffix;
  const auto t0 = std::chrono::steady_clock::now();
  const std::vector<std::string> opts = compile_options(src, dump);
  int major = 0, minor = 0;
  hiprtcVersion(&major, &minor);
  std::string key = src + "\n#opts";
  for (auto& o : opts) key += " " + o;
  key += "\n#hiprtc " + std::to_string(major) + "." + std::to_string(minor) + "\n";
  key += NT_SKELETON_SRC;
  key += NT_MATH_TABLES_SRC;
  char hex[32];
  std::snprintf(hex, sizeof hex, "%016llx", static_cast<unsigned long long>(fnv1a(key)));
  const std::string dir = cache_dir();
  const std::string path = dir.empty() ? "" : dir + "/" + hex + ".co";
  if (!path.empty() && read_file(path, code)) {
    (void)utime(path.c_str(), nullptr);  // marks the entry as in use (build() prunes entries it did not touch)
    seconds = std::chrono::duration<double>(std::chrono::steady_clock::now() - t0).count();
    return NT_OK;
  }
  hiprtcProgram prog;
  const char* hdr_src[] = {NT_SKELETON_SRC, NT_MATH_TABLES_SRC};
  const char* hdr_name[] = {"nt_skeleton.h", "nt_math_tables.h"};
  hiprtcResult r = hiprtcCreateProgram(&prog, src.c_str(), "nt_replay.hip", 2, hdr_src, hdr_name);
  if (r != HIPRTC_SUCCESS) return fail(static_cast<int>(r), std::string("hiprtcCreateProgram failed: ") + hiprtcGetErrorString(r));
  std::vector<const char*> copts;
  for (auto& o : opts) copts.push_back(o.c_str());
  r = hiprtcCompileProgram(prog, static_cast<int>(copts.size()), copts.data());
  if (r != HIPRTC_SUCCESS) {
    size_t n = 0;
    hiprtcGetProgramLogSize(prog, &n);
    std::string log(n, '\0');
    if (n) hiprtcGetProgramLog(prog, &log[0]);
    hiprtcDestroyProgram(&prog);
    return fail(NT_E_COMPILE, "hipRTC compile failed: " + std::string(hiprtcGetErrorString(r)) + "\n" + log);
  }
  size_t size = 0;
  hiprtcGetCodeSize(prog, &size);
  code.resize(size);
  hiprtcGetCode(prog, code.data());
  hiprtcDestroyProgram(&prog);
  if (!path.empty()) {
    mkdir(dir.c_str(), 0755);
    write_file_atomic(path, code);
  }
  seconds = std::chrono::duration<double>(std::chrono::steady_clock::now() - t0).count();
  return NT_OK;
}

// ---- code-object metadata (register and scratch evidence, no device needed) ----

bool meta_string(amd_comgr_metadata_node_t node, std::string& out) {
  size_t n = 0;
  if (amd_comgr_get_metadata_string(node, &n, nullptr) != AMD_COMGR_STATUS_SUCCESS) return false;
  out.assign(n, '\0');
  if (amd_comgr_get_metadata_string(node, &n, &out[0]) != AMD_COMGR_STATUS_SUCCESS) return false;
  while (!out.empty() && out.back() == '\0') out.pop_back();
  return true;
}

int meta_int(amd_comgr_metadata_node_t map, const char* key) {
  amd_comgr_metadata_node_t v;
  if (amd_comgr_metadata_lookup(map, key, &v) != AMD_COMGR_STATUS_SUCCESS) return -1;
  std::string s;
  bool ok = meta_string(v, s);
  amd_comgr_destroy_metadata(v);
  return ok ? std::atoi(s.c_str()) : -1;
}

void kernel_resources(const std::vector<char>& code, const char* kernel, nt_exec_info& info) {
  info.vgprs = info.sgprs = info.agprs = info.scratch_bytes = info.lds_bytes = -1;
  amd_comgr_data_t data;
  if (amd_comgr_create_data(AMD_COMGR_DATA_KIND_EXECUTABLE, &data) != AMD_COMGR_STATUS_SUCCESS) return;
  amd_comgr_set_data(data, code.size(), code.data());
  amd_comgr_metadata_node_t meta;
  if (amd_comgr_get_data_metadata(data, &meta) == AMD_COMGR_STATUS_SUCCESS) {
    amd_comgr_metadata_node_t kernels;
    if (amd_comgr_metadata_lookup(meta, "amdhsa.kernels", &kernels) == AMD_COMGR_STATUS_SUCCESS) {
      size_t count = 0;
      amd_comgr_get_metadata_list_size(kernels, &count);
      for (size_t k = 0; k < count; ++k) {
        amd_comgr_metadata_node_t km;
        if (amd_comgr_index_list_metadata(kernels, k, &km) != AMD_COMGR_STATUS_SUCCESS) continue;
        amd_comgr_metadata_node_t nm;
        std::string name;
        if (amd_comgr_metadata_lookup(km, ".name", &nm) == AMD_COMGR_STATUS_SUCCESS) {
          meta_string(nm, name);
          amd_comgr_destroy_metadata(nm);
        }
        if (name == kernel) {
          info.vgprs = meta_int(km, ".vgpr_count");
          info.sgprs = meta_int(km, ".sgpr_count");
          info.agprs = meta_int(km, ".agpr_count");
          info.scratch_bytes = meta_int(km, ".private_segment_fixed_size");
          info.lds_bytes = meta_int(km, ".group_segment_fixed_size");
        }
        amd_comgr_destroy_metadata(km);
      }
      amd_comgr_destroy_metadata(kernels);
    }
    amd_comgr_destroy_metadata(meta);
  }
  amd_comgr_release_data(data);
}

// ---- lowering shared by nt_lower / nt_compile_check / nt_exec_create ------------

int lower(const nt_tape* tape, const nt_options* opt, Lowered& out) {
  std::string err;
  int rc = ntl::build_ir(tape, out.ir, err);
  if (rc != NT_OK) return fail(rc, err);
  rc = ntl::make_plan(out.ir, opt, out.plan, err);
  if (rc != NT_OK) return fail(rc, err);
  out.source = ntl::emit_source(out.ir, out.plan);
  return NT_OK;
}

void fill_static_info(const Lowered& l, nt_exec_info& info) {
  int active = 0;
  for (uint8_t a : l.ir.active) active += a;
  info.n_nodes = l.ir.n;
  info.n_active = active;
  info.n_inputs = l.ir.n_in;
  info.n_channels = l.plan.n_channels;
  const auto& L = l.plan.loop;
  info.loop_start = L.found ? L.start : 0;
  info.loop_period = L.found ? L.period : 0;
  info.loop_iters = L.found ? L.iters : 0;
  info.loop_carries = static_cast<int32_t>(l.plan.carries.size());
  info.seg_len = l.plan.seg;
  info.n_segments = l.plan.nseg_full + (l.plan.tail ? 1 : 0);
  info.checkpoint = (L.found || !l.plan.lbound.empty()) ? l.plan.ckpt : 0;
  info.tape_slots = l.plan.tape_slots;
  info.mode = l.plan.mode;
  info.block = l.plan.block;
}

int copy_out(const std::string& s, char* buf, int64_t* len) {
  if (!len) return fail(NT_E_INVALID, "len is null");
  const int64_t need = static_cast<int64_t>(s.size()) + 1;
  if (buf && *len >= need) std::memcpy(buf, s.c_str(), static_cast<size_t>(need));
  const bool fits = buf && *len >= need;
  *len = need;
  return (buf && !fits) ? fail(NT_E_INVALID, "buffer too small") : NT_OK;
}

// A kernel that spills keeps part of each lane's state in scratch memory
// (HBM behind the caches), which the engine's design excludes: the tape is
// declined, as the reference's engines decline in compile() so that engine
// selection falls back to another engine (AadEngine.java:50-59), unless the
// caller opted in with allow_spill.
int decline_spill(const nt_exec_info& info, const nt_options* opt) {
  if (info.scratch_bytes <= 0 || (opt && opt->allow_spill)) return NT_OK;
  char buf[320];
  std::snprintf(buf, sizeof buf,
                "the rocm engine declines this tape: its %s replay kernel (%d nodes, %s) would spill %d bytes per "
                "lane to scratch memory at %d VGPRs; set nt_options.allow_spill to run it anyway",
                info.mode == NT_MODE_TANGENT ? "tangent-mode" : "reverse-sweep", info.n_nodes,
                info.loop_period    ? "step loop rolled"
                : info.n_segments ? "no step loop found, straight line cut into checkpointed segments"
                                  : "no step loop found, straight line",
                info.scratch_bytes,
                info.vgprs);
  return fail(NT_E_UNSUPPORTED, buf);
}

// Compiles the lowered replay kernel. A kernel at one wave per SIMD cannot
// hide the latency of its own dependent fp64 instructions (the VALU issues on
// about half the cycles); one that needs at most 16 VGPRs more than two waves
// allow (256) is compiled again with launch bounds asking for two, and that
// code is kept when it fits without scratch (the 16-asset worst-of in fp64:
// 270 VGPRs, one wave, 9.07 ms; 254 VGPRs, two waves, 7.12 ms). An explicit
// nt_options.waves is left as asked.
int compile_replay(const nt_tape* tape, const nt_options* options, Lowered& low, std::vector<char>& code,
                   nt_exec_info& info) {
  double secs = 0;
  int rc = compile_hiprtc(low.source, false, code, secs);
  if (rc != NT_OK) return rc;
  fill_static_info(low, info);
  kernel_resources(code, "nt_replay", info);
  info.compile_seconds = secs;
  const bool asked = options && options->waves > 0;
  if (asked || info.vgprs <= 256 || info.vgprs > 256 + 16) return NT_OK;
  nt_options o = options ? *options : nt_options{};
  o.waves = 2;
  Lowered low2;
  std::vector<char> code2;
  double secs2 = 0;
  if (lower(tape, &o, low2) != NT_OK || compile_hiprtc(low2.source, false, code2, secs2) != NT_OK) {
    (void)fail(NT_OK, std::string());  // the first compile stands; drop the retry's message
    return NT_OK;
  }
  nt_exec_info info2{};
  fill_static_info(low2, info2);
  kernel_resources(code2, "nt_replay", info2);
  info.compile_seconds += secs2;
  if (info2.scratch_bytes != 0 || info2.vgprs < 0 || info2.vgprs > 256) return NT_OK;
  info2.compile_seconds = info.compile_seconds;
  low = std::move(low2);
  code = std::move(code2);
  info = info2;
  return NT_OK;
}

// A kernel the module may or may not hold (the exception kernel): null when absent.
hipFunction_t optional_function(hipModule_t mod, const char* name) {
  hipFunction_t fn = nullptr;
  if (hipModuleGetFunction(&fn, mod, name) != hipSuccess) {
    (void)hipGetLastError();
    return nullptr;
  }
  return fn;
}

int device_index(int& dev) {
  int count = 0;
  if (nt_probe(&count) != NT_OK || count == 0) {
    return fail(NT_E_NO_DEVICE, "no ROCm/HIP gfx950 device available for the AAD replay kernel");
  }
  NT_HIP(hipGetDevice(&dev), "hipGetDevice");
  return NT_OK;
}

}  // namespace

nt_exec::~nt_exec() {
  if (stream) (void)hipStreamSynchronize(stream);
  for (auto& e : ev) {
    if (e) (void)hipEventDestroy(e);
  }
  if (stream) (void)hipStreamDestroy(stream);
  if (d_scratch) (void)hipFree(d_scratch);
  if (d_flags) (void)hipFree(d_flags);
  if (h_sums) (void)hipHostFree(h_sums);
  if (h_deferred) (void)hipHostFree(h_deferred);
  if (d_partials) (void)hipFree(d_partials);
  if (d_inputs) (void)hipFree(d_inputs);
  for (auto& kv : markets) {
    MarketVariant& v = kv.second;
    if (v.d_partials) (void)hipFree(v.d_partials);
    if (v.d_inputs) (void)hipFree(v.d_inputs);
    if (v.mod) (void)hipModuleUnload(v.mod);
  }
  if (d_set_inputs) (void)hipFree(d_set_inputs);
  if (mod_dump) (void)hipModuleUnload(mod_dump);
  if (mod) (void)hipModuleUnload(mod);
}

namespace ntr {

// A path whose work is short (estimated VALU instructions per path below
// kShortPath: a European, a few-step tape) does not amortise a block's start,
// its launch and its copy of the math tables into LDS, over the one or two
// paths per lane that a full resident grid gives a 10^6-path dispatch: such a
// dispatch gets about kLanePaths paths per lane instead, in a whole number of
// blocks per compute unit (a CU holding one block more than the others sets
// the kernel's time). Measured on the European call, 10^6 paths: 2048 blocks
// 17.4 us, 768 blocks 13.1 us (fp64); 13.4 and 10.4 us (fp32).
//
// A long path is VALU-bound, and a resident grid that strides over all the
// paths ends in a tail: the lanes whose last round has a path run it while
// the rest of the chip idles, and a SIMD left with one wave issues far below
// its rate. More blocks than the device holds let the dispatcher hand each
// freed slot the next block, so a long path gets the fewest whole blocks per
// compute unit that leave at most kLongLanePaths paths per lane, up to
// kOversubscribe times the resident grid. A reverse sweep that keeps its tape
// in device memory sizes that tape per lane of the largest grid, so it gets
// the larger grid only while the tape stays within kTapeBudget, and only with
// two or more waves per SIMD resident: at one wave per SIMD its tape traffic,
// not the tail, sets the time (local-volatility tape, 388 VGPRs: 8.89 ms
// resident, 9.33 ms on 8 resident grids).
// Whole blocks per CU matter as much as the count: a grid of q CUs' worth
// plus r blocks leaves r CUs one block longer than the rest. Measured on one
// MI355X (bench.py --max-blocks, two runs per grid, kernel HIP-event means),
// at the resident grid, at 16 blocks per CU (4,096) and at 4,112 blocks:
// Asian fp64 2M 0.894 / 0.839 / 0.866 ms; Asian fp32 2M 0.299 ms resident,
// 0.292 ms at 4,096, 0.314 ms at 2,176; weekday Asian fp64 2M 1.093 /
// 1.012 ms, 1.043 ms at 4,224; worst-of fp32 10^6 2.694 ms resident, 2.525 ms
// at 8 blocks per CU, 3.339 ms at 576 blocks; barrier fp64 20M 14.40 / 13.10
// ms at 40 blocks per CU; Heston-Asian 10M 25.56 / 24.48 ms at 24.
constexpr double kShortPath = 1000;
constexpr uint64_t kLanePaths = 4;
constexpr uint64_t kLongLanePaths = 2;
constexpr int kOversubscribe = 8;
constexpr uint64_t kTapeBudget = 1ull << 30;

// The largest grid a dispatch of this executable launches (partials, lane
// flags and tape are sized for it).
int grid_cap_for(const nt_exec* x, int per_cu, int cus) {
  const int resident = std::max(1, per_cu * cus);
  if (x->low.plan.path_cost < kShortPath || cus <= 0) return resident;
  const uint64_t tape_block = tape_bytes_per_lane(x) * static_cast<uint64_t>(x->low.plan.block);
  if (tape_block == 0) return kOversubscribe * resident;
  if (per_cu * x->low.plan.block < 2 * 256) return resident;  // fewer than two waves per SIMD
  const uint64_t by_tape = kTapeBudget / tape_block / static_cast<uint64_t>(cus) * static_cast<uint64_t>(cus);
  return static_cast<int>(std::min<uint64_t>(static_cast<uint64_t>(kOversubscribe) * resident,
                                             std::max<uint64_t>(resident, by_tape)));
}

int grid_for(const nt_exec* x, uint64_t paths) {
  const uint64_t block = static_cast<uint64_t>(x->low.plan.block);
  const uint64_t need = (paths + block - 1) / block;
  if (x->fixed_grid) return std::max(1, static_cast<int>(std::min<uint64_t>(need, static_cast<uint64_t>(x->grid_cap))));
  const uint64_t resident = static_cast<uint64_t>(x->resident);
  int grid = std::max(1, static_cast<int>(std::min(need, resident)));
  if (x->cus <= 0) return grid;
  const uint64_t cus = static_cast<uint64_t>(x->cus);
  if (x->low.plan.path_cost < kShortPath) {
    const uint64_t per_cu = paths / (block * kLanePaths) / cus;
    if (per_cu >= 1 && per_cu * cus < static_cast<uint64_t>(grid)) grid = static_cast<int>(per_cu * cus);
  } else if (need > resident) {
    const uint64_t per_cu = (need + kLongLanePaths * cus - 1) / (kLongLanePaths * cus);
    grid = static_cast<int>(std::min(std::max(per_cu * cus, resident), static_cast<uint64_t>(x->grid_cap)));
  }
  return grid;
}

size_t tape_bytes_per_lane(const nt_exec* x) {
  const size_t elem = x->low.plan.precision == NT_FP32 ? sizeof(float) : sizeof(double);
  return static_cast<size_t>(x->low.plan.tape_slots) * elem;
}

size_t flags_bytes_for(uint64_t lanes, int markets) {
  return (1 + static_cast<size_t>((lanes + 63) / 64) * static_cast<size_t>(std::max(1, markets))) * sizeof(uint64_t);
}

int partial_rows(int grid) { return 16 * ((grid + 7) / 8); }

int partial_slow_offset(int grid) { return 8 * ((grid + 7) / 8); }

int launch_kernel_on(nt_exec* x, hipStream_t stream, hipFunction_t fn, hipFunction_t fn_slow, const double* d_inputs,
                     double* d_partials, int nch, void* d_tape, uint64_t* d_flags, uint64_t paths, uint64_t offset,
                     uint64_t seed, double* out_v, double* out_g, int grid, hipEvent_t between) {
  const int block = x->low.plan.block;
  void* args[] = {&d_inputs, &paths, &offset, &seed, &d_partials, &d_tape, &out_v, &out_g, &d_flags};
  NT_HIP(hipModuleLaunchKernel(fn, static_cast<unsigned>(grid), 1, 1, static_cast<unsigned>(block), 1, 1, 0, stream,
                               args, nullptr),
         "hipModuleLaunchKernel(nt_replay)");
  if (between) NT_HIP(hipEventRecord(between, stream), "hipEventRecord");
  if (!fn_slow) return NT_OK;
  return launch_slow_on(x, stream, fn_slow, d_inputs, d_partials, nch, d_tape, d_flags, paths, offset, seed, out_v,
                        out_g, grid);
}

int launch_slow_on(nt_exec* x, hipStream_t stream, hipFunction_t fn_slow, const double* d_inputs, double* d_partials,
                   int nch, void* d_tape, uint64_t* d_flags, uint64_t paths, uint64_t offset, uint64_t seed,
                   double* out_v, double* out_g, int grid) {
  const int block = x->low.plan.block;
  double* slow_rows = d_partials + partial_slow_offset(grid);  // the exception kernel's region of each column
  void* sargs[] = {&d_inputs, &paths, &offset, &seed, &slow_rows, &d_tape, &out_v, &out_g, &d_flags};
  NT_HIP(hipModuleLaunchKernel(fn_slow, static_cast<unsigned>(grid), 1, 1, static_cast<unsigned>(block), 1, 1, 0,
                               stream, sargs, nullptr),
         "hipModuleLaunchKernel(nt_replay_slow)");
  return NT_OK;
}

int launch_finish_on(hipStream_t stream, hipFunction_t fn, const double* d_partials, int grid, int slow_grid, int nch,
                     double* out, uint64_t* d_flags, uint32_t* deferred) {
  unsigned blocks = static_cast<unsigned>(grid), slow_blocks = static_cast<unsigned>(slow_grid);
  unsigned nchu = static_cast<unsigned>(nch);
  const unsigned threads = 64u * static_cast<unsigned>(std::min(std::max(nch, 1), 16));
  void* args[] = {&d_partials, &blocks, &slow_blocks, &nchu, &out, &d_flags, &deferred};
  NT_HIP(hipModuleLaunchKernel(fn, 1, 1, 1, threads, 1, 1, 0, stream, args, nullptr),
         "hipModuleLaunchKernel(nt_finish)");
  return NT_OK;
}

}  // namespace ntr

extern "C" {

int nt_abi_version(void) { return NT_ABI_VERSION; }

void nt_testing_append_source(const char* text) { t_test_source_suffix = text ? text : ""; }

const char* nt_last_error(void) { return ntr::last_error(); }

int nt_probe(int32_t* count) {
  if (!count) return fail(NT_E_INVALID, "count is null");
  *count = 0;
  int n = 0;
  if (hipGetDeviceCount(&n) != hipSuccess) {
    (void)hipGetLastError();
    return NT_OK;
  }
  int usable = 0;
  for (int d = 0; d < n; ++d) {
    hipDeviceProp_t prop;
    if (hipGetDeviceProperties(&prop, d) != hipSuccess) continue;
    if (std::strncmp(prop.gcnArchName, kArch, std::strlen(kArch)) == 0) ++usable;
  }
  *count = usable;
  return NT_OK;
}

int nt_device_name(char* name, int32_t name_len, char* arch, int32_t arch_len) {
  int dev = 0;
  int rc = device_index(dev);
  if (rc != NT_OK) return rc;
  hipDeviceProp_t prop;
  NT_HIP(hipGetDeviceProperties(&prop, dev), "hipGetDeviceProperties");
  if (name && name_len > 0) std::snprintf(name, static_cast<size_t>(name_len), "%s", prop.name);
  if (arch && arch_len > 0) std::snprintf(arch, static_cast<size_t>(arch_len), "%s", prop.gcnArchName);
  return NT_OK;
}

int nt_lower(const nt_tape* tape, const nt_options* options, char* source, int64_t* len) {
  Lowered l;
  int rc = lower(tape, options, l);
  if (rc != NT_OK) return rc;
  return copy_out(l.source, source, len);
}

int nt_compile_check(const nt_tape* tape, const nt_options* options, nt_exec_info* info) {
  Lowered l;
  int rc = lower(tape, options, l);
  if (rc != NT_OK) return rc;
  std::vector<char> code;
  nt_exec_info res{};
  rc = compile_replay(tape, options, l, code, res);
  if (rc != NT_OK) return rc;
  if (info) *info = res;
  return decline_spill(res, options);
}

static int ensure_flags(nt_exec* x, int grid, int markets);

int nt_exec_create(const nt_tape* tape, const nt_options* options, nt_exec** out) {
  if (!out) return fail(NT_E_INVALID, "out is null");
  *out = nullptr;
  std::unique_ptr<nt_exec> x(new nt_exec());
  if (options) x->opts = *options;
  if (x->opts.markets > 1) return fail(NT_E_INVALID, "markets is a lowering option; price several input sets with nt_exec_replay_many");
  int rc = lower(tape, options, x->low);
  if (rc != NT_OK) return rc;
  rc = device_index(x->dev);
  if (rc != NT_OK) return rc;
  rc = compile_replay(tape, options, x->low, x->code, x->info);
  if (rc != NT_OK) return rc;
  rc = decline_spill(x->info, options);
  if (rc != NT_OK) return rc;
  NT_HIP(hipModuleLoadData(&x->mod, x->code.data()), "hipModuleLoadData");
  NT_HIP(hipModuleGetFunction(&x->fn, x->mod, "nt_replay"), "hipModuleGetFunction(nt_replay)");
  NT_HIP(hipModuleGetFunction(&x->fn_finish, x->mod, "nt_finish"), "hipModuleGetFunction(nt_finish)");
  x->fn_slow = optional_function(x->mod, "nt_replay_slow");
  int per_cu = 0, cus = 0;
  NT_HIP(hipModuleOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, x->fn, x->low.plan.block, 0),
         "hipModuleOccupancyMaxActiveBlocksPerMultiprocessor");
  NT_HIP(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, x->dev), "hipDeviceGetAttribute");
  const nt_options o = options ? *options : nt_options{};
  x->resident = std::max(1, per_cu * cus);
  x->cus = cus;
  x->grid_cap = ntr::grid_cap_for(x.get(), per_cu, cus);
  if (o.max_blocks > 0) {
    x->grid_cap = o.max_blocks;
    x->fixed_grid = true;
  }
  x->info.grid_cap = x->grid_cap;
  NT_HIP(hipStreamCreateWithFlags(&x->stream, hipStreamNonBlocking), "hipStreamCreateWithFlags");
  // ev[0] and ev[1] are timing points only (before and after the replay
  // kernel); without a system-scope fence at each (hipEventDisableSystemFence)
  // a dispatch's launch-to-result latency drops by about 3 us (the European
  // call's 33.5 us dispatch). ev[2], the last point before the host waits and
  // reads the sums from pinned memory, keeps the default fence.
  NT_HIP(hipEventCreateWithFlags(&x->ev[0], hipEventDisableSystemFence), "hipEventCreateWithFlags");
  NT_HIP(hipEventCreateWithFlags(&x->ev[1], hipEventDisableSystemFence), "hipEventCreateWithFlags");
  NT_HIP(hipEventCreate(&x->ev[2]), "hipEventCreate");
  const int nch = x->low.plan.n_channels;
  NT_HIP(hipMalloc(&x->d_inputs, sizeof(double) * std::max(1, x->low.ir.n_in)), "hipMalloc(inputs)");
  NT_HIP(hipMalloc(&x->d_partials,
                   sizeof(double) * static_cast<size_t>(ntr::partial_rows(x->grid_cap)) * nch),
         "hipMalloc(partials)");
  NT_HIP(hipHostMalloc(reinterpret_cast<void**>(&x->h_sums), sizeof(double) * nch, hipHostMallocDefault),
         "hipHostMalloc(sums)");
  NT_HIP(hipHostMalloc(reinterpret_cast<void**>(&x->h_deferred), sizeof(uint32_t), hipHostMallocDefault),
         "hipHostMalloc(deferred)");
  x->h_cap = static_cast<size_t>(nch);
  const size_t scratch = ntr::tape_bytes_per_lane(x.get()) * x->grid_cap * x->low.plan.block;
  if (scratch > 0) NT_HIP(hipMalloc(&x->d_scratch, scratch), "hipMalloc(scratch)");
  x->scratch_bytes = scratch;
  rc = ensure_flags(x.get(), x->grid_cap, 1);  // every single-set dispatch fits these
  if (rc != NT_OK) return rc;
  // the allocation-free entry point's array on this device, looked up and
  // its flags cleared here rather than in a call that may be under capture
  rc = ntr::noalloc_prepare(x->dev);
  if (rc != NT_OK) return rc;
  // inputs default to zero until bound; the reference starts from the recorded values (Java side)
  x->inputs.assign(static_cast<size_t>(x->low.ir.n_in), 0.0);
  for (int j = 0; j < x->low.ir.n_in; ++j) x->inputs[j] = x->low.ir.c[x->low.ir.input_node[j]];
  *out = x.release();
  return NT_OK;
}

int nt_exec_set_inputs(nt_exec* x, const double* inputs, int32_t n) {
  if (!x) return fail(NT_E_CLOSED, "executable is closed");
  if (n != x->low.ir.n_in || (n > 0 && !inputs)) return fail(NT_E_INVALID, "expected one value per tape input");
  x->inputs.assign(inputs, inputs + n);
  x->dirty = true;
  return NT_OK;
}

using ntr::grid_for;

// Grows the flags to a dispatch on `grid` blocks pricing `markets` sets: a
// size set by the grid (at most the executable's grid cap), not by the paths, so it
// grows at most a few times per executable. The stream is drained first (the
// old flags may still be in use) and the new ones are zeroed whole: every
// dispatch leaves the count and the bitmap at zero after that.
static int ensure_flags(nt_exec* x, int grid, int markets) {
  const uint64_t lanes = static_cast<uint64_t>(grid) * static_cast<uint64_t>(x->low.plan.block);
  const size_t need = ntr::flags_bytes_for(lanes, markets);
  if (need <= x->flags_bytes) return NT_OK;
  NT_HIP(hipStreamSynchronize(x->stream), "hipStreamSynchronize");
  const size_t bytes = std::max(need, x->flags_bytes + x->flags_bytes / 2);
  if (x->d_flags) (void)hipFree(x->d_flags);
  x->d_flags = nullptr;
  x->flags_bytes = 0;
  NT_HIP(hipMalloc(reinterpret_cast<void**>(&x->d_flags), bytes), "hipMalloc(flags)");
  x->flags_bytes = bytes;
  NT_HIP(hipMemsetAsync(x->d_flags, 0, bytes, x->stream), "hipMemsetAsync(flags)");
  return NT_OK;
}

// Replay kernel and, when it has one, exception kernel over `paths` on
// `grid` blocks each.
static int launch_kernel(nt_exec* x, hipFunction_t fn, hipFunction_t fn_slow, double* d_inputs, double* d_partials,
                         int nch, int markets, uint64_t paths, uint64_t offset, uint64_t seed, double* out_v,
                         double* out_g, int& grid, hipEvent_t between = nullptr) {
  grid = grid_for(x, paths);
  int rc = ensure_flags(x, grid, markets);
  if (rc != NT_OK) return rc;
  return ntr::launch_kernel_on(x, x->stream, fn, fn_slow, d_inputs, d_partials, nch, x->d_scratch, x->d_flags, paths,
                               offset, seed, out_v, out_g, grid, between);
}

static int launch_replay(nt_exec* x, hipFunction_t fn, hipFunction_t fn_slow, uint64_t paths, uint64_t offset,
                         uint64_t seed, double* out_v, double* out_g, int& grid, hipEvent_t between = nullptr) {
  if (x->dirty) {
    if (!x->inputs.empty()) {
      NT_HIP(hipMemcpyAsync(x->d_inputs, x->inputs.data(), sizeof(double) * x->inputs.size(), hipMemcpyHostToDevice,
                            x->stream),
             "hipMemcpyAsync(inputs)");
    }
    x->dirty = false;
  }
  return launch_kernel(x, fn, fn_slow, x->d_inputs, x->d_partials, x->low.plan.n_channels, 1, paths, offset, seed,
                       out_v, out_g, grid, between);
}

// Finishing pass over the partials of one dispatch on `grid` blocks: `nch`
// sums written to host memory `out` (pinned, read after the stream drains).
static int launch_finish(nt_exec* x, hipFunction_t fn, hipFunction_t fn_slow, double* d_partials, int grid, int nch,
                         double* out) {
  return ntr::launch_finish_on(x->stream, fn, d_partials, grid, fn_slow ? grid : 0, nch, out,
                               fn_slow ? x->d_flags : nullptr);
}

int nt_exec_replay(nt_exec* x, uint64_t paths, uint64_t offset, uint64_t seed, double* sums, int32_t n_sums,
                   double* timing) {
  if (!x) return fail(NT_E_CLOSED, "executable is closed");
  if (paths == 0) return fail(NT_E_INVALID, "paths must be positive");
  const int nch = x->low.plan.n_channels;
  if (!sums || n_sums != nch) return fail(NT_E_INVALID, "sums must hold n_outputs * (2 + n_inputs) doubles");
  const auto t0 = std::chrono::steady_clock::now();
  NT_HIP(hipSetDevice(x->dev), "hipSetDevice");
  NT_HIP(hipEventRecord(x->ev[0], x->stream), "hipEventRecord");
  int grid = 0;
  // The exception kernel runs only when the replay kernel left paths to it:
  // the finishing pass, launched right after the replay kernel, reports that
  // (a rare event) instead of finishing, and the exception kernel and the
  // pass follow once the stream has drained. Sums, rows and their order are
  // those of the three kernels launched back to back.
  int rc = launch_replay(x, x->fn, nullptr, paths, offset, seed, nullptr, nullptr, grid, x->ev[1]);
  if (rc != NT_OK) return rc;
  if (x->fn_slow) {
    *x->h_deferred = 0;
    rc = ntr::launch_finish_on(x->stream, x->fn_finish, x->d_partials, grid, grid, nch, x->h_sums, x->d_flags,
                               x->h_deferred);
  } else {
    rc = launch_finish(x, x->fn_finish, nullptr, x->d_partials, grid, nch, x->h_sums);
  }
  if (rc != NT_OK) return rc;
  NT_HIP(hipEventRecord(x->ev[2], x->stream), "hipEventRecord");
  NT_HIP(hipStreamSynchronize(x->stream), "hipStreamSynchronize");
  if (x->fn_slow && *x->h_deferred != 0) {
    rc = ntr::launch_slow_on(x, x->stream, x->fn_slow, x->d_inputs, x->d_partials, nch, x->d_scratch, x->d_flags,
                             paths, offset, seed, nullptr, nullptr, grid);
    if (rc != NT_OK) return rc;
    rc = launch_finish(x, x->fn_finish, x->fn_slow, x->d_partials, grid, nch, x->h_sums);
    if (rc != NT_OK) return rc;
    NT_HIP(hipEventRecord(x->ev[2], x->stream), "hipEventRecord");
    NT_HIP(hipStreamSynchronize(x->stream), "hipStreamSynchronize");
  }
  std::memcpy(sums, x->h_sums, sizeof(double) * nch);
  if (timing) {
    float all = 0, rep = 0;
    NT_HIP(hipEventElapsedTime(&all, x->ev[0], x->ev[2]), "hipEventElapsedTime");
    NT_HIP(hipEventElapsedTime(&rep, x->ev[0], x->ev[1]), "hipEventElapsedTime");
    timing[0] = all;
    timing[1] = std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - t0).count();
    timing[2] = rep;
  }
  return NT_OK;
}

static int market_variant(nt_exec* x, int markets, MarketVariant*& out) {
  auto it = x->markets.find(markets);
  if (it != x->markets.end()) {
    out = &it->second;
    return NT_OK;
  }
  nt_options o = x->opts;
  o.markets = markets;
  o.mode = NT_MODE_TANGENT;
  std::string err;
  ntl::Plan plan;
  int rc = ntl::make_plan(x->low.ir, &o, plan, err);
  if (rc != NT_OK) return fail(rc, err);
  const std::string src = ntl::emit_source(x->low.ir, plan);
  std::vector<char> code;
  double secs = 0;
  rc = compile_hiprtc(src, false, code, secs);
  if (rc != NT_OK) return rc;
  MarketVariant v;
  nt_exec_info res{};
  kernel_resources(code, "nt_replay", res);
  v.vgprs = res.vgprs;
  v.scratch = res.scratch_bytes;
  NT_HIP(hipModuleLoadData(&v.mod, code.data()), "hipModuleLoadData(markets)");
  const int nin = x->low.ir.n_in;
  const size_t nch = static_cast<size_t>(x->low.plan.n_channels) * markets;
  hipError_t e = hipModuleGetFunction(&v.fn, v.mod, "nt_replay");
  if (e == hipSuccess) e = hipModuleGetFunction(&v.fn_finish, v.mod, "nt_finish");
  if (e == hipSuccess) v.fn_slow = optional_function(v.mod, "nt_replay_slow");
  if (e == hipSuccess) e = hipMalloc(&v.d_inputs, sizeof(double) * std::max<size_t>(1, static_cast<size_t>(nin) * markets));
  if (e == hipSuccess) {
    const size_t rows = static_cast<size_t>(ntr::partial_rows(x->grid_cap));
    e = hipMalloc(&v.d_partials, sizeof(double) * rows * nch);
  }
  if (e != hipSuccess) {
    if (v.d_partials) (void)hipFree(v.d_partials);
    if (v.d_inputs) (void)hipFree(v.d_inputs);
    (void)hipModuleUnload(v.mod);
    return hip_fail(e, "loading the multi-market kernel");
  }
  out = &(x->markets[markets] = v);
  return NT_OK;
}

// Input sets per multi-market kernel: the most whose kernel keeps two waves
// per SIMD (at most 256 VGPRs) without spilling. Each set adds its own copy of
// the step's state, tangents and loop invariants to the registers, so beyond
// that point occupancy or scratch costs more than the shared draws save.
static int choose_market_chunk(nt_exec* x, int& chunk) {
  if (x->market_chunk > 0) {
    chunk = x->market_chunk;
    return NT_OK;
  }
  MarketVariant* v1 = nullptr;
  MarketVariant* v2 = nullptr;
  int rc = market_variant(x, 1, v1);
  if (rc != NT_OK) return rc;
  if (v1->scratch > 0 && !x->opts.allow_spill) {
    return fail(NT_E_UNSUPPORTED, "the tangent-mode kernel that prices input sets together would spill to scratch "
                                  "memory; set nt_options.allow_spill to run it anyway");
  }
  rc = market_variant(x, 2, v2);
  if (rc != NT_OK) return rc;
  const int per = std::max(1, v2->vgprs - v1->vgprs);
  int c = std::max(1, std::min(8, 1 + (256 - v1->vgprs) / per));
  if (v2->vgprs > 256 || v2->scratch > 0) c = 1;
  while (c > 2) {
    MarketVariant* v = nullptr;
    rc = market_variant(x, c, v);
    if (rc != NT_OK) return rc;
    if (v->vgprs <= 256 && v->scratch == 0) break;
    --c;
  }
  x->market_chunk = c;
  chunk = c;
  return NT_OK;
}

int nt_exec_replay_many(nt_exec* x, const double* input_sets, int32_t markets, uint64_t paths, uint64_t offset,
                        uint64_t seed, double* sums, int32_t n_sums, double* timing) {
  if (!x) return fail(NT_E_CLOSED, "executable is closed");
  if (paths == 0) return fail(NT_E_INVALID, "paths must be positive");
  if (markets < 1 || markets > 64) return fail(NT_E_INVALID, "markets must be between 1 and 64");
  const int nin = x->low.ir.n_in;
  const int nch = x->low.plan.n_channels;
  if (nin > 0 && !input_sets) return fail(NT_E_INVALID, "input_sets is null");
  if (!sums || n_sums != nch * markets) {
    return fail(NT_E_INVALID, "sums must hold markets * n_outputs * (2 + n_inputs) doubles");
  }
  const auto t0 = std::chrono::steady_clock::now();
  NT_HIP(hipSetDevice(x->dev), "hipSetDevice");
  const bool shared = x->low.plan.mode == NT_MODE_TANGENT;
  const size_t need = static_cast<size_t>(nch) * markets;
  if (x->h_cap < need) {
    // Every launch below writes its own rows; the stream is idle between calls, so the old rows are free.
    NT_HIP(hipStreamSynchronize(x->stream), "hipStreamSynchronize");
    double* grown = nullptr;
    NT_HIP(hipHostMalloc(reinterpret_cast<void**>(&grown), sizeof(double) * need, hipHostMallocDefault),
           "hipHostMalloc(sums)");
    (void)hipHostFree(x->h_sums);
    x->h_sums = grown;
    x->h_cap = need;
  }
  NT_HIP(hipEventRecord(x->ev[0], x->stream), "hipEventRecord");
  int grid = 0;
  if (shared) {
    int chunk = 1;
    int rc = choose_market_chunk(x, chunk);
    if (rc != NT_OK) return rc;
    NT_HIP(hipEventRecord(x->ev[0], x->stream), "hipEventRecord");  // after any first-use compiles
    for (int m0 = 0; m0 < markets; m0 += chunk) {
      const int k = std::min(chunk, markets - m0);
      MarketVariant* v = nullptr;
      rc = market_variant(x, k, v);
      if (rc != NT_OK) return rc;
      if (nin > 0) {
        NT_HIP(hipMemcpyAsync(v->d_inputs, input_sets + static_cast<size_t>(m0) * nin, sizeof(double) * nin * k,
                              hipMemcpyHostToDevice, x->stream),
               "hipMemcpyAsync(input sets)");
      }
      rc = launch_kernel(x, v->fn, v->fn_slow, v->d_inputs, v->d_partials, nch * k, k, paths, offset, seed, nullptr,
                         nullptr, grid);
      if (rc != NT_OK) return rc;
      rc = launch_finish(x, v->fn_finish, v->fn_slow, v->d_partials, grid, nch * k,
                         x->h_sums + static_cast<size_t>(m0) * nch);
      if (rc != NT_OK) return rc;
    }
    NT_HIP(hipEventRecord(x->ev[2], x->stream), "hipEventRecord");
  } else {
    // The reverse sweep keeps one set's state per lane: replay the sets in turn.
    if (!x->d_set_inputs) NT_HIP(hipMalloc(&x->d_set_inputs, sizeof(double) * std::max(1, nin)), "hipMalloc(set inputs)");
    for (int m = 0; m < markets; ++m) {
      if (nin > 0) {
        NT_HIP(hipMemcpyAsync(x->d_set_inputs, input_sets + static_cast<size_t>(m) * nin, sizeof(double) * nin,
                              hipMemcpyHostToDevice, x->stream),
               "hipMemcpyAsync(input set)");
      }
      int rc = launch_kernel(x, x->fn, x->fn_slow, x->d_set_inputs, x->d_partials, nch, 1, paths, offset, seed, nullptr,
                             nullptr, grid);
      if (rc != NT_OK) return rc;
      rc = launch_finish(x, x->fn_finish, x->fn_slow, x->d_partials, grid, nch,
                         x->h_sums + static_cast<size_t>(m) * nch);
      if (rc != NT_OK) return rc;
    }
    NT_HIP(hipEventRecord(x->ev[2], x->stream), "hipEventRecord");
  }
  NT_HIP(hipStreamSynchronize(x->stream), "hipStreamSynchronize");
  std::memcpy(sums, x->h_sums, sizeof(double) * need);
  if (timing) {
    float ms = 0;
    NT_HIP(hipEventElapsedTime(&ms, x->ev[0], x->ev[2]), "hipEventElapsedTime");
    timing[0] = ms;
    timing[1] = std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - t0).count();
    timing[2] = ms;
  }
  return NT_OK;
}

int nt_exec_replay_paths(nt_exec* x, uint64_t paths, uint64_t offset, uint64_t seed, double* values, double* grads) {
  if (!x) return fail(NT_E_CLOSED, "executable is closed");
  if (paths == 0) return fail(NT_E_INVALID, "paths must be positive");
  if (!values) return fail(NT_E_INVALID, "values is null");
  const int nin = x->low.ir.n_in;
  if (nin > 0 && !grads) return fail(NT_E_INVALID, "grads is null");
  NT_HIP(hipSetDevice(x->dev), "hipSetDevice");
  if (!x->mod_dump) {
    std::vector<char> code;
    double secs = 0;
    int rc = compile_hiprtc(x->low.source, true, code, secs);
    if (rc != NT_OK) return rc;
    NT_HIP(hipModuleLoadData(&x->mod_dump, code.data()), "hipModuleLoadData(dump)");
    NT_HIP(hipModuleGetFunction(&x->fn_dump, x->mod_dump, "nt_replay"), "hipModuleGetFunction(dump)");
    x->fn_dump_slow = optional_function(x->mod_dump, "nt_replay_slow");
  }
  const uint64_t rows = paths * static_cast<uint64_t>(x->low.ir.outputs.size());
  double* d_v = nullptr;
  double* d_g = nullptr;
  NT_HIP(hipMalloc(&d_v, sizeof(double) * rows), "hipMalloc(values)");
  hipError_t e = hipMalloc(&d_g, sizeof(double) * rows * static_cast<uint64_t>(std::max(1, nin)));
  if (e != hipSuccess) {
    (void)hipFree(d_v);
    return hip_fail(e, "hipMalloc(grads)");
  }
  int grid = 0;
  int rc = launch_replay(x, x->fn_dump, x->fn_dump_slow, paths, offset, seed, d_v, d_g, grid);
  if (rc == NT_OK && x->fn_dump_slow) {
    // no finishing pass follows: the count of lanes with exception paths goes back to zero here
    e = hipMemsetAsync(x->d_flags, 0, sizeof(uint64_t), x->stream);
    if (e != hipSuccess) rc = hip_fail(e, "hipMemsetAsync(flags)");
  }
  if (rc == NT_OK) {
    e = hipMemcpyAsync(values, d_v, sizeof(double) * rows, hipMemcpyDeviceToHost, x->stream);
    if (e == hipSuccess && nin > 0) {
      e = hipMemcpyAsync(grads, d_g, sizeof(double) * rows * nin, hipMemcpyDeviceToHost, x->stream);
    }
    if (e == hipSuccess) e = hipStreamSynchronize(x->stream);
    if (e != hipSuccess) rc = hip_fail(e, "replay_paths copy-back");
  }
  (void)hipFree(d_v);
  (void)hipFree(d_g);
  return rc;
}

int nt_exec_info_get(const nt_exec* x, nt_exec_info* info) {
  if (!x) return fail(NT_E_CLOSED, "executable is closed");
  if (!info) return fail(NT_E_INVALID, "info is null");
  *info = x->info;
  return NT_OK;
}

int nt_exec_grid(const nt_exec* x, uint64_t paths, int32_t* grid, int32_t* block) {
  if (!x) return fail(NT_E_CLOSED, "executable is closed");
  if (!grid || !block) return fail(NT_E_INVALID, "grid or block is null");
  if (paths == 0) return fail(NT_E_INVALID, "paths must be positive");
  *grid = grid_for(x, paths);
  *block = x->low.plan.block;
  return NT_OK;
}

int nt_exec_source(const nt_exec* x, char* source, int64_t* len) {
  if (!x) return fail(NT_E_CLOSED, "executable is closed");
  return copy_out(x->low.source, source, len);
}

int nt_exec_destroy(nt_exec* x) {
  delete x;  // ~nt_exec releases the device resources
  return NT_OK;
}

}  // extern "C"
