// Codegen-target section of the C ABI (include/tilers_hip.h, section 3):
// the `hip` target's name/emit, the TargetRegistry with the built-in targets of
// this library ("debug" and "hip"), and the host toolchain step (hipcc).
//
// Reference seam: CodegenTarget (crates/tile_codegen/src/target.rs:57-65),
// TargetRegistry (registry.rs:19-68), DebugTarget (targets.rs:32-53),
// EmitterTarget (targets.rs:82-101).
#include <dlfcn.h>
#include <fcntl.h>
#include <spawn.h>
#include <sys/stat.h>
#include <sys/wait.h>
#include <unistd.h>

#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <fstream>
#include <sstream>
#include <string>
#include <vector>

#include "../../include/tilers_hip.h"
#include "target/emit.hpp"

extern char** environ;

namespace {

char* dup_str(const std::string& s) {
  char* p = static_cast<char*>(std::malloc(s.size() + 1));
  if (!p) return nullptr;
  std::memcpy(p, s.data(), s.size());
  p[s.size()] = '\0';
  return p;
}

std::string json_escape(const std::string& s) {
  std::string o;
  for (char c : s) {
    if (c == '"' || c == '\\') o.push_back('\\');
    o.push_back(c);
  }
  return o;
}

std::string meta_json(const std::vector<std::string>& names) {
  std::string m = "{\"has_cube_kernel\":false,\"kernel_names\":[";
  for (size_t i = 0; i < names.size(); ++i) m += (i ? ",\"" : "\"") + json_escape(names[i]) + "\"";
  return m + "]}";
}

void set_err(char** out_err, const std::string& msg) {
  if (out_err) *out_err = dup_str(msg);
}

bool is_blank(const std::string& s) {
  for (char c : s)
    if (!std::isspace(static_cast<unsigned char>(c))) return false;
  return true;
}

// DebugTarget::emit (targets.rs:41-52): echo the module in a comment banner.
int debug_emit(const char* mlir, size_t len, const th_emit_opts*, char** out_src,
               const char** out_ext, char** out_meta, char** out_err) {
  const std::string text(mlir ? mlir : "", mlir ? len : 0);
  if (is_blank(text)) {
    set_err(out_err, "empty MLIR module");
    return TH_KERNEL_ERROR;
  }
  size_t lines = 0;
  {
    std::stringstream ss(text);
    std::string l;
    while (std::getline(ss, l)) ++lines;
  }
  size_t funcs = 0;
  for (size_t p = text.find("func.func"); p != std::string::npos; p = text.find("func.func", p + 1))
    ++funcs;
  const std::string src = "// tile-rs debug target\n// " + std::to_string(lines) + " MLIR lines, " +
                          std::to_string(funcs) + " func.func op(s)\n" + text + "\n";
  *out_src = dup_str(src);
  *out_ext = "mlir.txt";
  *out_meta = dup_str(meta_json({}));
  return TH_OK;
}

struct Entry {
  std::string name;
  std::string ext;
  th_emit_fn fn;
};

}  // namespace

struct th_registry_s {
  std::vector<Entry> targets;
};

#ifndef TH_BUILD_STAMP
#define TH_BUILD_STAMP "unstamped"
#endif

extern "C" {

const char* th_target_name(void) { return "hip"; }

void th_string_free(char* s) { std::free(s); }

int th_emit(const char* mlir, size_t len, const th_emit_opts* opts, char** out_src,
            const char** out_ext, char** out_meta, char** out_err) {
  (void)opts;  // the hip target reads no hardware knobs (HardwareParams::ub_size is Ascend's)
  if (!out_src || !out_ext || !out_meta) {
    set_err(out_err, "th_emit: null output pointer");
    return TH_KERNEL_ERROR;
  }
  *out_src = nullptr;
  *out_meta = nullptr;
  *out_ext = "hip";
  const std::string text(mlir ? mlir : "", mlir ? len : 0);
  if (is_blank(text)) {
    set_err(out_err, "empty MLIR module");
    return TH_KERNEL_ERROR;
  }
  std::string src, err;
  std::vector<std::string> names;
  if (!th::target::convert_mlir_to_hip(text, &src, &names, &err)) {
    set_err(out_err, err);
    return TH_KERNEL_ERROR;
  }
  *out_src = dup_str(src);
  *out_meta = dup_str(meta_json(names));
  return TH_OK;
}

th_registry th_registry_new(void) { return new th_registry_s; }

th_registry th_registry_with_builtin(void) {
  auto* r = new th_registry_s;
  r->targets.push_back(Entry{"debug", "mlir.txt", debug_emit});
  r->targets.push_back(Entry{"hip", "hip", th_emit});
  return r;
}

void th_registry_free(th_registry r) { delete r; }

int th_registry_register(th_registry r, const char* name, const char* ext, th_emit_fn emit) {
  if (!r || !name || !emit) return TH_RUNTIME_ERROR;
  r->targets.push_back(Entry{name, ext ? ext : "", emit});
  return TH_OK;
}

size_t th_registry_len(th_registry r) { return r ? r->targets.size() : 0; }

size_t th_registry_names(th_registry r, const char** names, size_t cap) {
  if (!r) return 0;
  size_t n = 0;
  for (; n < r->targets.size() && n < cap; ++n) names[n] = r->targets[n].name.c_str();
  return n;
}

int th_registry_emit(th_registry r, const char* name, const char* mlir, size_t len,
                     const th_emit_opts* opts, char** out_src, const char** out_ext,
                     char** out_meta, char** out_err) {
  if (!r || !name) {
    set_err(out_err, "null registry or target name");
    return TH_RUNTIME_ERROR;
  }
  for (const Entry& e : r->targets) {
    if (e.name == name) {  // select(): the first registered target of that name
      const int rc = e.fn(mlir, len, opts, out_src, out_ext, out_meta, out_err);
      if (rc == TH_OK && out_ext && (!*out_ext || !**out_ext)) *out_ext = e.ext.c_str();
      return rc;
    }
  }
  std::string avail;
  for (size_t i = 0; i < r->targets.size(); ++i) avail += (i ? ", " : "") + r->targets[i].name;
  set_err(out_err, std::string("unknown target ") + name + "; available: " + avail);
  return TH_BACKEND_NOT_AVAILABLE;
}

// Host toolchain step: hipcc --genco for gfx950.  hipcc runs as a child process.
int th_compile(const char* src, size_t len, const char* out_path, const char* include_dir,
               char** out_err) {
  if (!src || !out_path) {
    set_err(out_err, "th_compile: null source or output path");
    return TH_KERNEL_ERROR;
  }
  std::string inc = include_dir ? include_dir : "";
  if (inc.empty()) {
    Dl_info info;
    if (dladdr(reinterpret_cast<void*>(&th_compile), &info) && info.dli_fname) {
      std::string lib = info.dli_fname;  // .../tilers_hip/lib/libtilers_hip.so
      const size_t cut = lib.rfind("/tilers_hip/lib/");
      if (cut != std::string::npos) inc = lib.substr(0, cut) + "/csrc";
    }
  }
  const char* rocm = std::getenv("ROCM_PATH");
  const std::string hipcc = std::string(rocm ? rocm : "/opt/rocm") + "/bin/hipcc";
  char dir_tmpl[] = "/tmp/tilers_hip_XXXXXX";
  const char* dir = mkdtemp(dir_tmpl);
  if (!dir) {
    set_err(out_err, "th_compile: cannot create a temporary directory");
    return TH_RUNTIME_ERROR;
  }
  const std::string src_path = std::string(dir) + "/kernel.hip";
  const std::string log_path = std::string(dir) + "/hipcc.log";
  {
    std::ofstream f(src_path, std::ios::binary);
    f.write(src, static_cast<std::streamsize>(len));
  }
  std::vector<std::string> argv_s = {hipcc,
                                     "--genco",
                                     "--offload-arch=gfx950",
                                     "-O3",
                                     "-std=c++17",
                                     "-Xclang",
                                     "-target-feature",
                                     "-Xclang",
                                     "-packed-fp32-ops",
                                     "-Wno-unused-command-line-argument",
                                     // the stamp of the sources this library was built from
                                     "-DTH_BUILD_STAMP=\"" TH_BUILD_STAMP "\"",
                                     "-I",
                                     inc,
                                     src_path,
                                     "-o",
                                     out_path};
  std::vector<char*> argv;
  for (auto& a : argv_s) argv.push_back(a.data());
  argv.push_back(nullptr);
  posix_spawn_file_actions_t fa;
  posix_spawn_file_actions_init(&fa);
  posix_spawn_file_actions_addopen(&fa, 1, log_path.c_str(), O_WRONLY | O_CREAT | O_TRUNC, 0644);
  posix_spawn_file_actions_adddup2(&fa, 1, 2);
  pid_t pid = 0;
  const int sp = posix_spawn(&pid, hipcc.c_str(), &fa, nullptr, argv.data(), environ);
  posix_spawn_file_actions_destroy(&fa);
  int status = 0;
  if (sp == 0) waitpid(pid, &status, 0);
  std::string log;
  {
    std::ifstream f(log_path);
    std::stringstream ss;
    ss << f.rdbuf();
    log = ss.str();
  }
  std::remove(src_path.c_str());
  std::remove(log_path.c_str());
  rmdir(dir);
  if (sp != 0) {
    set_err(out_err, "th_compile: cannot start " + hipcc);
    return TH_BACKEND_NOT_AVAILABLE;
  }
  if (!WIFEXITED(status) || WEXITSTATUS(status) != 0) {
    set_err(out_err, "hipcc failed:\n" + log);
    return TH_KERNEL_ERROR;
  }
  return TH_OK;
}

}  // extern "C"
