// The `hip` codegen target: MLIR text -> HIP C++ for gfx950.
//
// Mirrors the emitter contract of the reference (`convert_mlir_to_<t>(&str) ->
// Result<String, String>` wrapped by EmitterTarget, crates/tile_codegen/src/
// targets.rs:82-101): pure, deterministic, and an error for a module with no
// entry kernel (mlir_to_linalg.rs:82-84) or an op it cannot lower
// (mlir_to_linalg.rs:608-612).
//
// Lowering (the "hook" that maps tile ops to hand-written kernels):
//   load -> __tile_softmax_{f32,f16}            -> store : th::entry::softmax_rows
//   load -> __tile_rms_norm_f32                  -> store : th::entry::rms_norm_rows
//   load, load -> matmul -> silu, load -> mul    -> store : th::entry::gemm with the
//                                                           SiLU*Mul epilogue (the fusion the
//                                                           gpu target does, mlir_to_gpu.rs:536-634)
//   load, load -> __tile_matmul_{f16,f32}        -> store : th::entry::gemm (MFMA) / gemm_fma
//   load, load -> __tile_matmul_transposed_*     -> store : same, B stored N x K
//   load x3 -> __tile_attention_f32              -> store : th::entry::attention_tiles
//   load x3 -> __tile_attention_prefill_f32      -> store : th::entry::prefill
//   load x3 -> __tile_attention_gqa_{f32,f16}    -> store : th::entry::prefill (head-major)
//   load x3 -> __tile_attention_decode_f32       -> store : th::entry::decode
//   any DAG of elementwise tile ops              -> a plain HIP per-element kernel
// Per-tile pointer offsets follow the #[tile_kernel] prelude: logical tile t
// offsets each view by t * rows * cols (crates/tile_std_macros/src/lib.rs:242).
//
// Side channels the trait cannot carry:
//   - bf16: tile_std carries f16 and bf16 in one u16 type (tile_std/src/lib.rs:
//     182).  A u16 load/store is bf16 when its callee says so
//     (__tile_load_bf16, as mlir_to_pto.rs:5666-5690 reads it) or when the
//     kernel or pointer-argument name contains "bf16" (the name convention of
//     infer_dtype_from_name, mlir_to_pto.rs:5648-5654); otherwise f16.
//   - attention runtime scalars: appended as trailing uint32_t kernel
//     parameters after the buffers, in the Metal target's order
//     (mlir_to_msl.rs:1816-1823 decode, :1851-1859 prefill).
// Every emitted kernel also takes a hidden trailing `uint32_t th_tiles` (the
// logical tile count) and carries a launch descriptor `__th_desc_<name>`.
#include <cctype>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <iomanip>
#include <map>
#include <set>
#include <sstream>
#include <string>
#include <vector>

#include "launch_desc.hpp"
#include "target/emit.hpp"
#include "target/mlir_parse.hpp"

namespace th {
namespace target {
namespace {

enum Dt { F32 = 0, F16 = 1, BF16 = 2 };

const char* dt_name(int d) { return d == F32 ? "f32" : d == F16 ? "f16" : "bf16"; }
const char* dt_enum(int d) { return d == F32 ? "th::kF32" : d == F16 ? "th::kF16" : "th::kBF16"; }
const char* dt_ctype(int d) { return d == F32 ? "float" : "uint16_t"; }

struct PtrRef {
  int arg = -1;            // index into the kernel's GM pointer list
  long long offset = 0;    // element offset from the argument
  long long iv_stride = 0; // elements added per iteration of the lowered loop
};

// a * iv + b for the induction variable of a lowered loop
struct Affine {
  long long stride = 0, offset = 0;
};

// A counted tile loop `for iv in 0..n` whose views advance one tile per
// iteration (tile.rs:2196-2210): lowered by mapping iteration i to logical
// tile i, so the loop's tiles run in parallel over the grid.
struct Loop {
  bool present = false;
  long long trip = 0;    // constant trip count, or
  int trip_arg = -1;     // position of the scalar kernel argument holding it
  bool is_signed = false;  // signed compare: a negative bound runs no iteration
};

struct TileVal {
  std::string op;                  // "load" or the intrinsic name
  std::vector<std::string> ins;    // operand tiles
  std::vector<double> scalars;     // scalar operands (scale, clamp bounds, fill value)
  long long rows = 0, cols = 0;
  int dtype = F32;
  PtrRef src;                      // for loads
};

struct Store {
  PtrRef dst;
  std::string value;
  long long rows = 0, cols = 0;
  int dtype = F32;
};

struct Kernel {
  std::string name;
  std::vector<mlir::FuncArg> args;            // all args in order
  std::vector<mlir::FuncArg> gm;              // pointer args in order
  std::map<std::string, int> gm_index;        // arg name -> position
  std::map<std::string, double> consts;       // SSA -> numeric constant
  std::set<std::string> block_derived;        // SSA values computed from get_block_idx
  std::map<std::string, PtrRef> ptrs;         // SSA -> pointer (arg, offset)
  std::map<std::string, TileVal> tiles;       // SSA -> tile
  std::vector<Store> stores;
  bool bf16_hint = false;
  std::map<std::string, Affine> affine;       // SSA -> affine in the loop's induction variable
  Loop loop;
  int depth = 0;                              // pipelined_for(depth), 0 = no marker
  bool block_offset = false;                  // some view carries the per-tile offset
};

std::string ssa_token(const std::string& s) {
  size_t e = 0;
  while (e < s.size() && (std::isalnum(static_cast<unsigned char>(s[e])) || s[e] == '%' ||
                          s[e] == '_' || s[e] == '#'))
    ++e;
  return s.substr(0, e);
}

bool parse_number(const std::string& txt, double* v) {
  const std::string t = mlir::trim(txt);
  if (t == "true") { *v = 1; return true; }
  if (t == "false") { *v = 0; return true; }
  char* end = nullptr;
  const double d = std::strtod(t.c_str(), &end);
  if (end == t.c_str()) return false;
  *v = d;
  return true;
}

class Lowerer {
 public:
  Lowerer(const mlir::Func& f, std::string* err) : f_(f), err_(err) {}

  bool analyze(Kernel* k) {
    k->name = f_.name;
    k->args = f_.args;
    for (const auto& a : f_.args) {
      if (a.is_gm) {
        k->gm_index[a.name] = static_cast<int>(k->gm.size());
        k->ptrs[a.name] = PtrRef{static_cast<int>(k->gm.size()), 0};
        k->gm.push_back(a);
        if (a.name.find("bf16") != std::string::npos) k->bf16_hint = true;
      }
    }
    if (k->name.find("bf16") != std::string::npos) k->bf16_hint = true;
    for (const std::string& raw : f_.body_lines) {
      const std::string l = mlir::trim(raw);
      if (l.rfind("^bb", 0) == 0 || l.find(".br ") != std::string::npos ||
          l.find(".cond_br ") != std::string::npos)
        return loop_(k);
    }
    for (const std::string& raw : f_.body_lines) {
      const std::string line = mlir::trim(raw);
      if (line.empty() || line == "llvm.return" || line.rfind("llvm.return", 0) == 0) continue;
      if (!line_(k, line)) return false;
    }
    return true;
  }

 private:
  // ---- control flow: the counted tile loop ----
  struct Block {
    std::string label;                // "" for the entry block
    std::vector<std::string> params;  // block argument SSA names
    std::vector<std::string> lines;
  };

  static Block parse_label(const std::string& l) {
    Block b;
    const size_t paren = l.find('(');
    b.label = l.substr(0, paren == std::string::npos ? l.size() - 1 : paren);
    if (paren != std::string::npos) {
      const size_t close = l.rfind(')');
      std::stringstream ss(l.substr(paren + 1, close - paren - 1));
      std::string part;
      while (std::getline(ss, part, ',')) {
        part = mlir::trim(part);
        b.params.push_back(mlir::trim(part.substr(0, part.find(':'))));
      }
    }
    return b;
  }

  // SSA operands of a branch target `^bbN(%a, %b : i32, i32)` or `^bbN(%a : i32, %b : i32)`
  static std::string branch_target(const std::string& t, std::vector<std::string>* args) {
    const size_t paren = t.find('(');
    args->clear();
    if (paren != std::string::npos) {
      std::stringstream ss(t.substr(paren + 1, t.rfind(')') - paren - 1));
      std::string part;
      while (std::getline(ss, part, ',')) {
        part = mlir::trim(part);
        if (!part.empty() && part[0] == '%') args->push_back(ssa_token(part));
      }
    }
    return mlir::trim(t.substr(0, paren));
  }

  static bool parse_br(const std::string& l, std::string* target, std::vector<std::string>* args) {
    for (const char* op : {"llvm.br ", "cf.br "}) {
      if (l.rfind(op, 0) == 0) {
        *target = branch_target(mlir::trim(l.substr(std::strlen(op))), args);
        return true;
      }
    }
    return false;
  }

  // `llvm.cond_br %c, ^bbT, ^bbF` -> (cond, T, F); targets must take no arguments
  static bool parse_cond_br(const std::string& l, std::string* cond, std::string* t,
                            std::string* f) {
    std::string rest;
    for (const char* op : {"llvm.cond_br ", "cf.cond_br "})
      if (l.rfind(op, 0) == 0) rest = mlir::trim(l.substr(std::strlen(op)));
    if (rest.empty()) return false;
    std::vector<std::string> parts;
    int depth = 0;
    std::string cur;
    for (char c : rest) {
      if (c == '(' || c == '[') ++depth;
      if (c == ')' || c == ']') --depth;
      if (c == ',' && depth == 0) {
        parts.push_back(mlir::trim(cur));
        cur.clear();
      } else {
        cur += c;
      }
    }
    parts.push_back(mlir::trim(cur));
    if (parts.size() != 3) return false;
    std::vector<std::string> ta, fa;
    *cond = ssa_token(parts[0]);
    *t = branch_target(parts[1], &ta);
    *f = branch_target(parts[2], &fa);
    return ta.empty() && fa.empty();
  }

  bool loop_(Kernel* k) {
    std::vector<Block> blocks(1);
    for (const std::string& raw : f_.body_lines) {
      const std::string l = mlir::trim(raw);
      if (l.empty() || l.rfind("llvm.return", 0) == 0) continue;
      if (l.rfind("^bb", 0) == 0 && l.back() == ':') blocks.push_back(parse_label(l));
      else blocks.back().lines.push_back(l);
    }
    auto find = [&](const std::string& lab) -> const Block* {
      for (const Block& b : blocks)
        if (!lab.empty() && b.label == lab) return &b;
      return nullptr;
    };
    const std::string shape =
        "control flow: only a counted tile loop is lowered (entry -> header(iv) -> body -> "
        "header, exit on iv >= n)";
    const Block& entry = blocks[0];
    std::string hlab;
    std::vector<std::string> hargs;
    if (entry.lines.empty() || !parse_br(entry.lines.back(), &hlab, &hargs) || hargs.size() != 1)
      return fail(shape);
    const Block* H = find(hlab);
    if (!H || H->params.size() != 1 || H->lines.size() < 2) return fail(shape);
    const std::string iv = H->params[0];
    std::string cond, ta, fb;
    if (!parse_cond_br(H->lines.back(), &cond, &ta, &fb)) return fail(shape);
    // the compare that defines the condition
    std::string pred, x, y;
    for (const std::string& l : H->lines) {
      const auto r = mlir::result_ssa(l);
      const size_t p = l.find("llvm.icmp \"");
      if (r && *r == cond && p != std::string::npos) {
        const size_t q = l.find('"', p + 11);
        pred = l.substr(p + 11, q - p - 11);
        std::string ops = mlir::trim(l.substr(q + 1));
        ops = ops.substr(0, ops.find(" : "));
        x = mlir::trim(ops.substr(0, ops.find(',')));
        y = mlir::trim(ops.substr(ops.find(',') + 1));
      }
    }
    if (pred.empty()) return fail(shape);
    auto latches = [&](const Block* b) {
      std::string t;
      std::vector<std::string> a;
      return b && !b->lines.empty() && parse_br(b->lines.back(), &t, &a) && t == hlab &&
             a.size() == 1;
    };
    const Block* A = find(ta);
    const Block* B = find(fb);
    if (!A || !B || latches(A) == latches(B)) return fail(shape);
    const bool true_is_body = latches(A);
    const Block* body = true_is_body ? A : B;
    const Block* exitb = true_is_body ? B : A;
    std::string n_tok;
    bool ok = false;
    if (x == iv) {
      n_tok = y;
      ok = true_is_body ? (pred == "ult" || pred == "slt" || pred == "ne")
                        : (pred == "uge" || pred == "sge" || pred == "eq");
    } else if (y == iv) {
      n_tok = x;
      ok = true_is_body ? (pred == "ugt" || pred == "sgt" || pred == "ne")
                        : (pred == "ule" || pred == "sle" || pred == "eq");
    }
    if (!ok) return fail("control flow: the loop must run while iv < n: " + H->lines.back());
    k->loop.is_signed = pred[0] == 's';
    // entry block (constants, the pipelined_for marker)
    for (size_t i = 0; i + 1 < entry.lines.size(); ++i)
      if (!line_(k, entry.lines[i])) return false;
    double start = -1;
    if (!resolve(k, hargs[0], &start) || start != 0) return fail("control flow: the loop must start at 0");
    for (const std::string& l : H->lines) {
      if (l.find("llvm.icmp") != std::string::npos || l.find("cond_br") != std::string::npos) continue;
      if (!line_(k, l)) return false;
    }
    double nv = 0;
    if (resolve(k, n_tok, &nv)) {
      if (nv < 0 && !k->loop.is_signed) return fail("control flow: negative trip count");
      k->loop.trip = nv < 0 ? 0 : static_cast<long long>(nv);
      if (k->loop.trip > 0xffffffffll) return fail("control flow: trip count beyond 2^32 - 1");
    } else {
      for (size_t i = 0; i < f_.args.size(); ++i)
        if (f_.args[i].name == n_tok && !f_.args[i].is_gm) k->loop.trip_arg = static_cast<int>(i);
      if (k->loop.trip_arg < 0)
        return fail("control flow: the loop bound must be a constant or a scalar kernel argument");
      const std::string& ty = f_.args[k->loop.trip_arg].ty;
      if (ty.find("i32") == std::string::npos && ty.find("i64") == std::string::npos)
        return fail("control flow: the loop bound must be an i32 or i64 argument, not " + ty);
      if (k->loop.trip_arg + 1 > static_cast<int>(th::kScaleIndex))
        return fail("control flow: the loop bound must be one of the first 63 arguments");
    }
    if (!k->tiles.empty() || !k->stores.empty())
      return fail("control flow: tile operations outside the loop body are not lowered");
    // body: iv is affine; the latch increments it by one
    std::string next_t;
    std::vector<std::string> next_a;
    parse_br(body->lines.back(), &next_t, &next_a);
    bool stepped = false;
    k->affine[iv] = Affine{1, 0};
    for (size_t i = 0; i + 1 < body->lines.size(); ++i) {
      const std::string& l = body->lines[i];
      const auto r = mlir::result_ssa(l);
      if (r && *r == next_a[0] && l.find("llvm.add ") != std::string::npos) {
        std::string ops = mlir::trim(l.substr(l.find("llvm.add ") + 9));
        ops = ops.substr(0, ops.find(" : "));
        const std::string a0 = mlir::trim(ops.substr(0, ops.find(',')));
        const std::string a1 = mlir::trim(ops.substr(ops.find(',') + 1));
        double one = 0;
        stepped = (a0 == iv && resolve(k, a1, &one) && one == 1) ||
                  (a1 == iv && resolve(k, a0, &one) && one == 1);
        if (!stepped) return fail("control flow: the loop must step by 1: " + l);
        continue;
      }
      if (!line_(k, l)) return false;
    }
    if (!stepped) return fail("control flow: the loop must step its index by 1");
    for (const std::string& l : exitb->lines) {
      const auto c = mlir::callee(l);
      if (!c || *c != "__tile_pipelined_for_end")
        return fail("control flow: the loop exit may only end the pipelined_for marker: " + l);
    }
    for (const auto& kv : k->tiles) {
      const TileVal& t = kv.second;
      if (t.op == "load" && t.src.iv_stride != t.rows * t.cols)
        return fail("control flow: loop views must advance one tile (rows * cols) per iteration");
    }
    for (const Store& st : k->stores)
      if (st.dst.iv_stride != st.rows * st.cols)
        return fail("control flow: loop views must advance one tile (rows * cols) per iteration");
    if (k->stores.empty()) return fail("control flow: the loop body stores nothing");
    // The reference runs the body in order (tile.rs:2187-2210); here the iterations
    // run in parallel.  That is the same result only when no iteration reads what
    // another writes: a stored argument may be loaded only at the store's own view
    // (same offset, tile size and dtype: an in-place update), never shifted.
    for (const Store& st : k->stores)
      for (const auto& kv : k->tiles) {
        const TileVal& t = kv.second;
        if (t.op != "load" || t.src.arg != st.dst.arg) continue;
        if (t.src.offset != st.dst.offset || t.src.iv_stride != st.dst.iv_stride ||
            t.dtype != st.dtype || t.rows * t.cols != st.rows * st.cols)
          return fail("control flow: the loop loads argument " + k->gm[st.dst.arg].name +
                      " at another view than it stores it (a loop-carried dependence; "
                      "the iterations are run in parallel)");
      }
    // Every launched tile of such a kernel walks the same n tiles; a view that
    // also carried the per-tile offset would need that offset's stride, which
    // the folding cannot check.
    if (k->block_offset)
      return fail("control flow: loop views may not also carry the per-tile (block index) offset");
    k->loop.present = true;
    return true;
  }

 public:

 private:
  bool fail(const std::string& m) {
    *err_ = "mlir_to_hip: " + f_.name + ": " + m;
    return false;
  }

  bool resolve(const Kernel* k, const std::string& tok, double* v) const {
    auto it = k->consts.find(tok);
    if (it != k->consts.end()) {
      *v = it->second;
      return true;
    }
    return parse_number(tok, v);
  }

  int u16_dtype(const Kernel* k, const std::string& callee, const std::string& ptr) const {
    if (callee.find("bf16") != std::string::npos) return BF16;
    if (k->bf16_hint || ptr.find("bf16") != std::string::npos) return BF16;
    return F16;
  }

  bool line_(Kernel* k, const std::string& line) {
    const auto res = mlir::result_ssa(line);
    // ---- constants ----
    if (line.find("llvm.mlir.constant") != std::string::npos) {
      const size_t open = line.find('(');
      const size_t colon = line.find(':', open);
      double v = 0;
      if (res && open != std::string::npos && colon != std::string::npos &&
          parse_number(line.substr(open + 1, colon - open - 1), &v)) {
        k->consts[*res] = v;
        return true;
      }
      return fail("cannot parse constant: " + line);
    }
    // ---- integer casts / arithmetic on constants (GEP offsets) ----
    static const char* kUnary[] = {"llvm.bitcast ", "llvm.zext ", "llvm.sext ", "llvm.trunc ",
                                   "llvm.ptrtoint ", "llvm.inttoptr "};
    for (const char* op : kUnary) {
      const size_t p = line.find(op);
      if (p != std::string::npos && res) {
        const std::string src = ssa_token(mlir::trim(line.substr(p + std::strlen(op))));
        if (k->consts.count(src)) k->consts[*res] = k->consts[src];
        if (k->affine.count(src)) k->affine[*res] = k->affine[src];
        if (k->block_derived.count(src)) k->block_derived.insert(*res);
        if (k->ptrs.count(src)) k->ptrs[*res] = k->ptrs[src];
        return true;
      }
    }
    static const char* kBinary[] = {"llvm.mul ", "llvm.add ", "llvm.sub ", "llvm.shl "};
    for (const char* op : kBinary) {
      const size_t p = line.find(op);
      if (p != std::string::npos && res) {
        std::string rest = mlir::trim(line.substr(p + std::strlen(op)));
        const size_t c = rest.find(" : ");
        if (c != std::string::npos) rest = rest.substr(0, c);
        const size_t comma = rest.find(',');
        if (comma == std::string::npos) return fail("cannot parse: " + line);
        const std::string a = mlir::trim(rest.substr(0, comma));
        const std::string b = mlir::trim(rest.substr(comma + 1));
        if (k->block_derived.count(a) || k->block_derived.count(b)) {
          k->block_derived.insert(*res);
          return true;
        }
        if (k->affine.count(a) || k->affine.count(b)) {
          // affine in the loop index: (s*iv + o) op constant, or a sum of two
          const std::string o = op;
          Affine fa, fb;
          double ca = 0, cb = 0;
          const bool aa = k->affine.count(a), ab = k->affine.count(b);
          if (aa) fa = k->affine[a];
          else if (!resolve(k, a, &ca)) return fail("non-affine use of the loop index: " + line);
          if (ab) fb = k->affine[b];
          else if (!resolve(k, b, &cb)) return fail("non-affine use of the loop index: " + line);
          const long long ia = static_cast<long long>(ca), ib = static_cast<long long>(cb);
          Affine r;
          if (o == "llvm.add ") {
            r.stride = fa.stride + fb.stride;
            r.offset = (aa ? fa.offset : ia) + (ab ? fb.offset : ib);
          } else if (o == "llvm.sub ") {
            r.stride = fa.stride - fb.stride;
            r.offset = (aa ? fa.offset : ia) - (ab ? fb.offset : ib);
          } else if (o == "llvm.mul " && aa != ab) {
            const Affine& f = aa ? fa : fb;
            const long long c = aa ? ib : ia;
            r.stride = f.stride * c;
            r.offset = f.offset * c;
          } else if (o == "llvm.shl " && aa && !ab) {
            r.stride = fa.stride << ib;
            r.offset = fa.offset << ib;
          } else {
            return fail("non-affine use of the loop index: " + line);
          }
          k->affine[*res] = r;
          return true;
        }
        double x = 0, y = 0;
        if (resolve(k, a, &x) && resolve(k, b, &y)) {
          const std::string o = op;
          k->consts[*res] = o == "llvm.mul " ? x * y
                            : o == "llvm.add " ? x + y
                            : o == "llvm.sub " ? x - y
                                               : std::ldexp(x, static_cast<int>(y));
          return true;
        }
        return fail("non-constant integer arithmetic is not supported: " + line);
      }
    }
    // ---- pointer arithmetic ----
    if (line.find("llvm.getelementptr") != std::string::npos) {
      if (!res) return fail("getelementptr without result: " + line);
      size_t p = line.find("llvm.getelementptr") + std::strlen("llvm.getelementptr");
      std::string rest = mlir::trim(line.substr(p));
      if (rest.rfind("inbounds", 0) == 0) rest = mlir::trim(rest.substr(8));
      const size_t lb = rest.find('['), rb = rest.find(']');
      if (lb == std::string::npos || rb == std::string::npos) return fail("cannot parse: " + line);
      const std::string base = mlir::trim(rest.substr(0, lb));
      const std::string idx = mlir::trim(rest.substr(lb + 1, rb - lb - 1));
      auto bp = k->ptrs.find(base);
      if (bp == k->ptrs.end()) return fail("getelementptr on an unknown pointer: " + line);
      PtrRef r = bp->second;
      double off = 0;
      if (k->block_derived.count(idx)) {
        // the #[tile_kernel] per-tile offset: applied implicitly per logical tile
        k->block_offset = true;
      } else if (k->affine.count(idx)) {
        r.offset += k->affine[idx].offset;
        r.iv_stride += k->affine[idx].stride;
      } else if (resolve(k, idx, &off)) {
        r.offset += static_cast<long long>(off);
      } else {
        return fail("non-constant pointer offset: " + line);
      }
      k->ptrs[*res] = r;
      return true;
    }
    // ---- calls ----
    const auto cal = mlir::callee(line);
    if (!cal) return fail("unsupported operation (control flow and scalar memory ops are not lowered): " + line);
    const auto args = mlir::call_args(line);
    if (!args) return fail("cannot parse call arguments: " + line);
    const std::string& c = *cal;
    const std::vector<std::string>& a = *args;
    if (c == "get_block_idx" || c == "get_block_num") {
      if (res) k->block_derived.insert(*res);
      return true;
    }
    if (c == "__tile_pipelined_for_begin") {
      // pipelined_for(depth) (tile.rs:2183-2221): recorded for the loop's kernel
      double d = 0;
      if (!a.empty() && resolve(k, a[0], &d)) k->depth = static_cast<int>(d);
      return true;
    }
    if (c == "__tile_pipelined_for_end") return true;
    if (c.rfind("__tile_load_", 0) == 0) {
      if (a.size() < 3 || !res) return fail("load: expected (ptr, rows, cols): " + line);
      auto p = k->ptrs.find(a[0]);
      if (p == k->ptrs.end()) return fail("load from an unknown pointer: " + line);
      TileVal t;
      t.op = "load";
      t.src = p->second;
      double r = 0, cc = 0;
      if (!resolve(k, a[1], &r) || !resolve(k, a[2], &cc)) return fail("load: shape is not constant");
      t.rows = static_cast<long long>(r);
      t.cols = static_cast<long long>(cc);
      if (c == "__tile_load_f32") t.dtype = F32;
      else if (c == "__tile_load_f16" || c == "__tile_load_bf16") t.dtype = u16_dtype(k, c, a[0]);
      else return fail("unsupported load " + c);
      k->tiles[*res] = t;
      return true;
    }
    if (c.rfind("__tile_store_", 0) == 0) {
      if (a.size() < 4) return fail("store: expected (ptr, tile, rows, cols): " + line);
      auto p = k->ptrs.find(a[0]);
      if (p == k->ptrs.end()) return fail("store to an unknown pointer: " + line);
      Store s;
      s.dst = p->second;
      s.value = a[1];
      double r = 0, cc = 0;
      if (!resolve(k, a[2], &r) || !resolve(k, a[3], &cc)) return fail("store: shape is not constant");
      s.rows = static_cast<long long>(r);
      s.cols = static_cast<long long>(cc);
      if (c == "__tile_store_f32" || c == "__tile_store_u32") s.dtype = F32;
      else if (c == "__tile_store_f16" || c == "__tile_store_bf16") s.dtype = u16_dtype(k, c, a[0]);
      else return fail("unsupported store " + c);
      if (!k->tiles.count(s.value)) return fail("store of an unknown tile " + s.value);
      k->stores.push_back(s);
      return true;
    }
    if (c.rfind("__tile_", 0) == 0) {
      if (!res) return fail("tile op without result: " + line);
      TileVal t;
      t.op = c;
      return op_(k, line, c, a, *res, t);
    }
    return fail("unsupported call @" + c);
  }

  // Operand layouts of the supported tile ops (crates/tile_std/src/tile.rs).
  bool op_(Kernel* k, const std::string& line, const std::string& c,
           const std::vector<std::string>& a, const std::string& res, TileVal t) {
    auto tile = [&](const std::string& s) -> const TileVal* {
      auto it = k->tiles.find(s);
      return it == k->tiles.end() ? nullptr : &it->second;
    };
    auto num = [&](const std::string& s, double* v) { return resolve(k, s, v); };
    const std::string base = c.substr(7);  // after "__tile_"
    auto shape_from = [&](size_t ri, size_t ci) {
      double r = 0, cc = 0;
      if (!num(a[ri], &r) || !num(a[ci], &cc)) return false;
      t.rows = static_cast<long long>(r);
      t.cols = static_cast<long long>(cc);
      return true;
    };
    static const std::set<std::string> kBin = {"add_f32", "sub_f32", "mul_f32", "div_f32",
                                               "max_f32", "min_f32", "add_f16", "mul_f16"};
    static const std::set<std::string> kUn = {"exp_f32", "neg_f32", "silu_f32", "log_f32",
                                              "tanh_f32", "abs_f32", "sqrt_f32", "rsqrt_f32",
                                              "sigmoid_f32", "relu_f32",
                                              "causal_mask_f32", "exp_f16", "neg_f16", "silu_f16",
                                              "cast_f32_f16", "cast_f16_f32", "cast_f32_bf16",
                                              "cast_bf16_f32"};
    // row reductions and transpose: (dst, src, rows, cols), mlir_to_linalg.rs:1458-1660
    static const std::set<std::string> kRow = {"reduce_sum_f32", "reduce_max_f32", "absmax_f32",
                                               "argmax_f32", "transpose_f32"};
    if (base == "softmax_f32" || base == "softmax_f16") {
      if (a.size() < 4 || !tile(a[1]) || !shape_from(2, 3)) return fail("softmax arity: " + line);
      t.ins = {a[1]};
      t.dtype = tile(a[1])->dtype;
    } else if (base == "rms_norm_f32") {
      // (dst, src, eps, rows, cols), tile.rs:2063
      double eps = 0;
      if (a.size() < 5 || !tile(a[1]) || !num(a[2], &eps) || !shape_from(3, 4))
        return fail("rms_norm arity: " + line);
      t.ins = {a[1]};
      t.scalars = {eps};
      t.dtype = tile(a[1])->dtype;
    } else if (base == "matmul_f32" || base == "matmul_f16" || base == "matmul_transposed_f32" ||
               base == "matmul_transposed_f16") {
      if (a.size() < 6 || !tile(a[1]) || !tile(a[2])) return fail("matmul arity: " + line);
      double m = 0, kk = 0, n = 0;
      if (!num(a[3], &m) || !num(a[4], &kk) || !num(a[5], &n)) return fail("matmul shape: " + line);
      t.ins = {a[1], a[2]};
      t.rows = static_cast<long long>(m);
      t.cols = static_cast<long long>(n);
      t.scalars = {kk};
      t.dtype = tile(a[1])->dtype;
    } else if (base == "attention_f32") {
      if (a.size() < 6 || !tile(a[1]) || !tile(a[2]) || !tile(a[3]) || !shape_from(4, 5))
        return fail("attention arity: " + line);
      t.ins = {a[1], a[2], a[3]};
      t.dtype = tile(a[1])->dtype;
    } else if (base == "attention_prefill_f32" || base == "attention_decode_f32") {
      if (a.size() < 6 || !tile(a[1]) || !tile(a[2]) || !tile(a[3]) || !shape_from(4, 5))
        return fail(base + " arity: " + line);
      t.ins = {a[1], a[2], a[3]};
      t.dtype = tile(a[1])->dtype;
    } else if (base == "attention_gqa_f32" || base == "attention_gqa_f16") {
      // (dst, q, k, v, num_heads, num_kv_heads, seq_len, head_dim), all four sizes
      // compile-time constants (mlir_to_gpu.rs:1627-1647); result [NH * S][D]
      double nh = 0, nkv = 0, seq = 0, hd = 0;
      if (a.size() < 8 || !tile(a[1]) || !tile(a[2]) || !tile(a[3]) || !num(a[4], &nh) ||
          !num(a[5], &nkv) || !num(a[6], &seq) || !num(a[7], &hd))
        return fail(base + " arity: " + line);
      t.ins = {a[1], a[2], a[3]};
      t.rows = static_cast<long long>(nh * seq);
      t.cols = static_cast<long long>(hd);
      t.scalars = {nh, nkv, seq, hd};
      t.dtype = tile(a[1])->dtype;
    } else if (kBin.count(base)) {
      // (dst, a, b, rows, cols) as in the linalg bridge (mlir_to_linalg.rs:620-633), or
      // (a, b, rows, cols) as the gpu emitter's inputs also use
      if (a.size() == 4 && tile(a[0]) && tile(a[1]) && shape_from(2, 3)) {
        t.ins = {a[0], a[1]};
      } else {
        if (a.size() < 5 || !tile(a[1]) || !tile(a[2]) || !shape_from(3, 4))
          return fail(base + " arity: " + line);
        t.ins = {a[1], a[2]};
      }
      t.dtype = F32;
    } else if (kRow.count(base)) {
      if (a.size() < 4 || !tile(a[1]) || !shape_from(2, 3)) return fail(base + " arity: " + line);
      t.ins = {a[1]};
      t.dtype = F32;
    } else if (base == "matvec_f32") {
      // (dst, a, b, rows, cols): a rows x cols, b cols -> rows (mlir_to_linalg.rs:1395-1440)
      if (a.size() < 5 || !tile(a[1]) || !tile(a[2]) || !shape_from(3, 4))
        return fail("matvec arity: " + line);
      t.ins = {a[1], a[2]};
      t.dtype = F32;
    } else if (kUn.count(base)) {
      if (a.size() < 4 || !tile(a[1]) || !shape_from(2, 3)) return fail(base + " arity: " + line);
      t.ins = {a[1]};
      t.dtype = F32;
    } else if (base == "rope_f32" || base == "rope_f16") {
      // (dst, src, pos, rows, cols), tile.rs:232, :2425; pos is a constant as in
      // the gpu lowering (mlir_to_gpu.rs:1508-1557)
      double pos = 0;
      if (a.size() < 5 || !tile(a[1]) || !num(a[2], &pos) || !shape_from(3, 4))
        return fail(base + " arity: " + line);
      if (t.cols % 2 != 0) return fail(base + ": cols must be even: " + line);
      t.ins = {a[1]};
      t.scalars = {pos};
      t.dtype = F32;
    } else if (base == "scale_f32") {
      double s = 0;
      if (a.size() < 5 || !tile(a[1]) || !num(a[2], &s) || !shape_from(3, 4))
        return fail("scale arity: " + line);
      t.ins = {a[1]};
      t.scalars = {s};
    } else if (base == "clamp_f32") {
      double lo = 0, hi = 0;
      if (a.size() < 6 || !tile(a[1]) || !num(a[2], &lo) || !num(a[3], &hi) || !shape_from(4, 5))
        return fail("clamp arity: " + line);
      t.ins = {a[1]};
      t.scalars = {lo, hi};
    } else if (base == "fill_f32") {
      double v = 0;
      if (a.size() < 4 || !num(a[1], &v) || !shape_from(2, 3)) return fail("fill arity: " + line);
      t.scalars = {v};
    } else {
      return fail("unsupported intrinsic " + c);
    }
    k->tiles[res] = t;
    return true;
  }

  const mlir::Func& f_;
  std::string* err_;
};

// ---------------------------------------------------------------------------
// Code generation
// ---------------------------------------------------------------------------

std::string u(long long v) { return std::to_string(v) + "u"; }

// Exact C++ spelling of an f32 constant.
std::string fconst(double v) {
  std::ostringstream os;
  os << std::hexfloat << static_cast<float>(v) << "f";
  return os.str();
}

// scale_args / scale_div / wg_cap: grid factors from run-time scalar arguments
// (launch_desc.hpp); a lowered loop multiplies the workgroups per tile by its
// trip count.
void desc(std::ostringstream& os, const Kernel& k, unsigned threads, unsigned wg_per_tile,
          unsigned tiles_per_wg, unsigned scale_args = 0, unsigned scale_div = 0,
          unsigned wg_cap = 0, unsigned grid_per_cu = 0) {
  unsigned long long wpt = wg_per_tile ? wg_per_tile : 1;
  if (k.loop.present) {
    // the kernel runs n tiles for any launched tile count: size the grid for
    // ceil(n / tiles_per_wg) workgroups per launched tile (usually one)
    constexpr unsigned long long kCap = 1u << 16;
    const unsigned long long tpw = tiles_per_wg ? tiles_per_wg : 1;
    tiles_per_wg = 1;
    if (k.loop.trip_arg >= 0) {
      // callers with both slots in use reject run-time loop bounds before this point
      const unsigned slot = (scale_args & 0xffu) ? 8u : 0u;
      unsigned b = static_cast<unsigned>(k.loop.trip_arg + 1);
      if (k.args[k.loop.trip_arg].ty.find("i64") != std::string::npos) b |= th::kScaleWide;
      if (k.loop.is_signed) b |= th::kScaleSigned;
      scale_args |= b << slot;
      scale_div |= static_cast<unsigned>(tpw) << (2 * slot);
      wg_cap = wg_cap ? wg_cap : static_cast<unsigned>(kCap);
    } else {
      const unsigned long long n = k.loop.trip > 0 ? static_cast<unsigned long long>(k.loop.trip) : 1;
      wpt *= (n + tpw - 1) / tpw;
      if (wpt > kCap) wpt = kCap;
    }
  }
  os << "extern \"C\" __device__ th::LaunchDesc __th_desc_" << k.name << " = {th::kLaunchDescMagic, "
     << threads << "u, " << wpt << "u, " << (tiles_per_wg ? tiles_per_wg : 1) << "u, 0u, "
     << scale_args << "u, " << scale_div << "u, " << wg_cap << "u, " << grid_per_cu << "u};\n\n";
}

// C type of a scalar kernel argument
std::string scalar_ctype(const std::string& ty) {
  if (ty.find("f32") != std::string::npos) return "float";
  if (ty.find("f64") != std::string::npos) return "double";
  if (ty.find("i64") != std::string::npos) return "uint64_t";
  return "uint32_t";
}

// min_groups > 0 asks for that many resident workgroups per CU (it caps the
// registers per wave accordingly).
// Parameters follow the MLIR function's arguments (pointers p<i>, scalars s<pos>),
// then the trailing run-time scalars `extra`, then the hidden tile count.  A
// lowered loop folds its iterations into the tile count.
void signature(std::ostringstream& os, const Kernel& k, unsigned threads,
               const std::vector<std::string>& extra, unsigned min_groups = 0) {
  os << "extern \"C\" __global__ void __launch_bounds__(" << threads;
  if (min_groups) os << ", " << min_groups;
  os << ") " << k.name << "(";
  bool first = true;
  for (size_t i = 0; i < k.args.size(); ++i) {
    const mlir::FuncArg& a = k.args[i];
    os << (first ? "" : ", ");
    if (a.is_gm) os << "void* __restrict__ p" << k.gm_index.at(a.name);
    else os << scalar_ctype(a.ty) << " s" << i;
    first = false;
  }
  for (const std::string& e : extra) {
    os << (first ? "" : ", ") << "uint32_t " << e;
    first = false;
  }
  os << (first ? "" : ", ");
  if (!k.loop.present) {
    os << "uint32_t th_tiles) {\n";
    return;
  }
  os << "uint32_t th_tiles_in) {\n";
  os << "  // counted tile loop: iteration i is tile i.  Every launched tile walks the\n"
        "  // same iterations, so any number of launched tiles computes them once.\n";
  std::string n;
  if (k.loop.trip_arg < 0) {
    n = std::to_string(k.loop.trip) + "u";
  } else {
    // the bound as the loop compares it: a negative signed bound runs no iteration;
    // a 64-bit one is capped at 2^32 - 1 tiles
    const std::string a = "s" + std::to_string(k.loop.trip_arg);
    const bool wide = k.args[k.loop.trip_arg].ty.find("i64") != std::string::npos;
    const std::string cap = "(" + a + " > 0xffffffffull ? 0xffffffffu : static_cast<uint32_t>(" + a + "))";
    if (wide && k.loop.is_signed)
      n = "(static_cast<int64_t>(" + a + ") <= 0 ? 0u : " + cap + ")";
    else if (wide)
      n = cap;
    else if (k.loop.is_signed)
      n = "(static_cast<int32_t>(" + a + ") <= 0 ? 0u : " + a + ")";
    else
      n = a;
  }
  os << "  const uint32_t th_tiles = th_tiles_in ? " << n << " : 0u;\n";
  for (size_t i = 0; i < k.args.size(); ++i)
    if (!k.args[i].is_gm && static_cast<int>(i) != k.loop.trip_arg) os << "  (void)s" << i << ";\n";
}

bool is_elementwise(const std::string& op) {
  for (const char* hot : {"softmax", "rms_norm", "matmul", "attention", "reduce_", "absmax",
                          "argmax", "transpose", "matvec"})
    if (op.find(hot) != std::string::npos) return false;
  return op != "load";
}

// Pointer expressions of a loaded view / the stored view (per-tile offsets are
// added by the entry from th_tiles).
std::string view_ptr(const TileVal& t, const char* ctype) {
  return "(reinterpret_cast<const " + std::string(ctype) + "*>(p" + std::to_string(t.src.arg) +
         ")" + (t.src.offset ? " + " + std::to_string(t.src.offset) + "ll" : "") + ")";
}
std::string store_ptr(const Store& st, const char* ctype) {
  return "(reinterpret_cast<" + std::string(ctype) + "*>(p" + std::to_string(st.dst.arg) + ")" +
         (st.dst.offset ? " + " + std::to_string(st.dst.offset) + "ll" : "") + ")";
}

// GEMM body for the matmul tile `mm` stored by `st`; epi names the epilogue
// (th::gemm::kEpiStore, or kEpiSiluMul with the UP view `up`).
bool matmul_entry(const Kernel& k, const TileVal& mm, const Store& st, const char* epi,
                  const TileVal* up, std::ostringstream& os, std::string* err) {
  const bool bt = mm.op.find("transposed") != std::string::npos;
  const TileVal& a = k.tiles.at(mm.ins[0]);
  const TileVal& b = k.tiles.at(mm.ins[1]);
  const long long M = mm.rows, N = mm.cols, K = static_cast<long long>(mm.scalars[0]);
  if (a.rows * a.cols != M * K || b.rows * b.cols != K * N || st.rows * st.cols != M * N) {
    *err = "mlir_to_hip: " + k.name + ": matmul operand shapes do not match m/k/n";
    return false;
  }
  if (a.dtype != b.dtype) {
    *err = "mlir_to_hip: " + k.name + ": matmul operands have different dtypes";
    return false;
  }
  const int in = a.dtype, out = st.dtype;
  const bool mfma = in != F32 && K % 8 == 0 && (bt || N % 8 == 0) && a.src.offset % 8 == 0 &&
                    b.src.offset % 8 == 0;
  // 32-deep K steps (and N % 8 for the 16-byte epilogue): the LDS-DMA pipeline
  // (its entry checks the run-time 16-byte alignment the offsets cannot show).
  const int osz = out == F32 ? 4 : 2;
  const bool dma = mfma && K % 32 == 0 && N % 8 == 0 && (st.dst.offset * osz) % 16 == 0 &&
                   (!up || (up->src.offset * osz) % 16 == 0);
  // whole 256 x 256 tiles, plain store or SiLU*Mul into 16-bit C: the generated-assembly
  // program (the shapes th::gasm::fits accepts: K in groups of four 32-deep steps, at
  // least two, and per-lane byte offsets within 32 bits)
  const bool gasm = dma && (!up || out != F32) && M > 0 && N > 0 && M % 256 == 0 && N % 256 == 0 &&
                    K % 128 == 0 && K >= 256 && 512LL * K < (1LL << 31) &&
                    136LL * N * osz < (1LL << 31) && 64LL * N < (1LL << 31);
  os << "matmul " << M << "x" << K << "x" << N << (bt ? " (B transposed)" : "") << " " << dt_name(in)
     << " -> " << dt_name(out) << (up ? " with silu*mul epilogue" : "")
     << (gasm ? " -> th::entry::gemm_asm (MFMA, generated assembly)"
             : dma ? " -> th::entry::gemm_dma (MFMA, LDS-DMA)"
             : mfma ? " -> th::entry::gemm (MFMA)"
             : in == F32 ? " -> th::entry::gemm_f32 (fp32 MFMA)" : " -> th::entry::gemm_fma")
     << "\n";
  const unsigned threads = gasm ? 256 : dma ? 512 : 256;
  signature(os, k, threads, {}, gasm ? 1 : 0);
  const std::string tmpl = std::string(dt_enum(in)) + ", " + dt_enum(out) + ", " +
                           (bt ? "true" : "false") + ", " + epi;
  // pipelined_for(depth >= 2): the LDS ring depth (4 or 5 stages; the staged
  // epilogue needs four stages of LDS)
  const int ns = k.depth >= 2 ? (k.depth > 5 ? 5 : (k.depth < 4 ? 4 : k.depth)) : 0;
  const std::string tmpl_dma = ns ? tmpl + ", " + std::to_string(ns) : tmpl;
  const std::string tail = up ? ", th_tiles, " + view_ptr(*up, dt_ctype(out)) + ");\n}\n"
                              : ", th_tiles);\n}\n";
  if (gasm) {
    os << "  th::entry::gemm_asm<" << dt_enum(in) << ", " << dt_enum(out) << ", "
       << (bt ? "true" : "false") << (up ? ", true" : "") << ">("
       << view_ptr(a, "uint16_t") << ", " << view_ptr(b, "uint16_t") << ", "
       << store_ptr(st, dt_ctype(out)) << ", " << u(M) << ", " << u(N) << ", " << u(K) << tail;
    desc(os, k, threads, static_cast<unsigned>((M / 256) * (N / 256)), 1);
  } else if (dma) {
    os << "  th::entry::gemm_dma<" << tmpl_dma << ">(" << view_ptr(a, "uint16_t") << ", "
       << view_ptr(b, "uint16_t") << ", " << store_ptr(st, dt_ctype(out)) << ", " << u(M) << ", "
       << u(N) << ", " << u(K) << tail;
    desc(os, k, threads, static_cast<unsigned>(((M + 255) / 256) * ((N + 255) / 256)), 1);
  } else if (mfma) {
    os << "  th::entry::gemm<" << tmpl << ">(" << view_ptr(a, "uint16_t") << ", "
       << view_ptr(b, "uint16_t") << ", " << store_ptr(st, dt_ctype(out)) << ", " << u(M) << ", "
       << u(N) << ", " << u(K) << tail;
    desc(os, k, 256, static_cast<unsigned>(((M + 255) / 256) * ((N + 255) / 256)), 1);
  } else if (in == F32) {
    // 16-byte pieces when every row start is 16-byte aligned (the base's alignment
    // is checked at run time by the entry)
    const bool vec = K % 4 == 0 && (bt || N % 4 == 0) && a.src.offset % 4 == 0 &&
                     b.src.offset % 4 == 0;
    os << "  th::entry::gemm_f32<" << dt_enum(out) << ", " << (bt ? "true" : "false") << ", "
       << (vec ? "true" : "false") << ", " << epi << ">(" << view_ptr(a, "float") << ", "
       << view_ptr(b, "float") << ", " << store_ptr(st, dt_ctype(out)) << ", " << u(M) << ", "
       << u(N) << ", " << u(K) << tail;
    desc(os, k, 256, static_cast<unsigned>(((M + 127) / 128) * ((N + 127) / 128)), 1);
  } else {
    os << "  th::entry::gemm_fma<" << tmpl << ">(" << view_ptr(a, dt_ctype(in)) << ", "
       << view_ptr(b, dt_ctype(in)) << ", " << store_ptr(st, dt_ctype(out)) << ", " << u(M)
       << ", " << u(N) << ", " << u(K) << tail;
    desc(os, k, 256, static_cast<unsigned>(((M + 63) / 64) * ((N + 63) / 64)), 1);
  }
  return true;
}

// store(mul(silu(matmul(load, load)), load)) with nothing else in the kernel: the
// GEMM with the SiLU*Mul epilogue.  Returns false when the kernel is not of that
// shape (and leaves *err empty); true when emitted, or on error with *err set.
bool emit_fused_swiglu(const Kernel& k, std::ostringstream& os, std::string* err) {
  if (k.stores.size() != 1) return false;
  const Store& st = k.stores[0];
  const TileVal& mul = k.tiles.at(st.value);
  if (mul.op != "__tile_mul_f32" && mul.op != "__tile_mul_f16") return false;
  const TileVal* silu = nullptr;
  const TileVal* up = nullptr;
  for (const std::string& in : mul.ins) {
    const TileVal& t = k.tiles.at(in);
    if (t.op == "__tile_silu_f32" || t.op == "__tile_silu_f16") silu = &t;
    else if (t.op == "load") up = &t;
  }
  if (!silu || !up) return false;
  const TileVal& mm = k.tiles.at(silu->ins[0]);
  if (mm.op.find("matmul") == std::string::npos) return false;
  for (const std::string& in : mm.ins)
    if (k.tiles.at(in).op != "load") return false;
  size_t others = 0;
  for (const auto& kv : k.tiles)
    if (kv.second.op != "load") ++others;
  if (others != 3) return false;  // exactly matmul, silu, mul
  if (up->dtype != st.dtype) {
    *err = "mlir_to_hip: " + k.name + ": fused silu*mul needs UP in the output dtype";
    return true;
  }
  if (up->rows * up->cols != mm.rows * mm.cols || st.rows * st.cols != mm.rows * mm.cols) {
    *err = "mlir_to_hip: " + k.name + ": fused silu*mul operand shapes do not match the matmul";
    return true;
  }
  os << "// kernel " << k.name << ": ";
  matmul_entry(k, mm, st, "th::gemm::kEpiSiluMul", up, os, err);
  return true;
}

// Emits kernels for one function; returns false with *err on unsupported shapes.
bool emit_kernel(const Kernel& k, std::ostringstream& os, std::string* err) {
  if (emit_fused_swiglu(k, os, err)) return err->empty();
  // Identify a hot-op chain: one store whose value is a hot op fed by loads.
  const TileVal* hot = nullptr;
  const Store* st = nullptr;
  if (k.stores.size() == 1) {
    const TileVal& v = k.tiles.at(k.stores[0].value);
    if (v.op != "load" && !is_elementwise(v.op)) {
      bool direct = true;
      for (const std::string& in : v.ins) direct = direct && k.tiles.at(in).op == "load";
      if (!direct) {
        *err = "mlir_to_hip: " + k.name + ": " + v.op + " operands must come straight from loads";
        return false;
      }
      hot = &v;
      st = &k.stores[0];
    }
  }
  for (const auto& kv : k.tiles) {
    if (&kv.second != hot && kv.second.op != "load" && !is_elementwise(kv.second.op)) {
      *err = "mlir_to_hip: " + k.name + ": " + kv.second.op +
             " must be the only op between loads and a single store";
      return false;
    }
  }
  os << "// kernel " << k.name << ": ";
  if (!hot) {
    // ---------------- elementwise fallback ----------------
    if (k.stores.empty()) {
      *err = "mlir_to_hip: " + k.name + ": kernel has no store";
      return false;
    }
    const long long R = k.stores[0].rows, C = k.stores[0].cols;
    for (const auto& kv : k.tiles)
      if (kv.second.rows * kv.second.cols != R * C) {
        *err = "mlir_to_hip: " + k.name + ": elementwise tiles must share one shape";
        return false;
      }
    for (const Store& s : k.stores)
      if (s.rows * s.cols != R * C) {
        *err = "mlir_to_hip: " + k.name + ": elementwise tiles must share one shape";
        return false;
      }
    os << "elementwise over " << R << "x" << C << " tiles (plain HIP)\n";
    signature(os, k, 256, {});
    os << "  const uint64_t th_n = static_cast<uint64_t>(th_tiles) * " << R * C << "ull;\n";
    os << "  for (uint64_t i = static_cast<uint64_t>(blockIdx.x) * 256u + threadIdx.x; i < th_n;"
          " i += static_cast<uint64_t>(gridDim.x) * 256u) {\n";
    os << "    const uint32_t row = static_cast<uint32_t>((i / " << C << "ull) % " << R
       << "ull), col = static_cast<uint32_t>(i % " << C << "ull);\n";
    os << "    (void)row; (void)col;\n";
    // topological emission: repeat until every tile value is defined
    std::map<std::string, std::string> var;
    int n = 0;
    bool progress = true;
    while (progress && var.size() < k.tiles.size()) {
      progress = false;
      for (const auto& kv : k.tiles) {
        if (var.count(kv.first)) continue;
        bool ready = true;
        for (const std::string& in : kv.second.ins) ready = ready && var.count(in);
        if (!ready) continue;
        const TileVal& t = kv.second;
        const std::string v = "v" + std::to_string(n++);
        const std::string o = t.op.size() > 7 ? t.op.substr(7) : t.op;
        auto in = [&](int i) { return var.at(t.ins[i]); };
        std::ostringstream e;
        // Element `ix` (an index expression) of a loaded view, widened to f32.
        auto load_at = [&](const TileVal& l, const std::string& ix) {
          const std::string p = "reinterpret_cast<const " + std::string(dt_ctype(l.dtype)) + "*>(p" +
                                std::to_string(l.src.arg) + ")";
          const std::string idx = std::to_string(l.src.offset) + "ll + static_cast<int64_t>(" + ix + ")";
          if (l.dtype == F32) return p + "[" + idx + "]";
          return "th::u16_to_f32<" + std::string(dt_enum(l.dtype)) + ">(" + p + "[" + idx + "])";
        };
        if (t.op == "load") {
          e << load_at(t, "i");
        } else if (o == "rope_f32" || o == "rope_f16") {
          // Interleaved pairs (x[2j], x[2j+1]) of a row rotate by pos * 10000^(-2j/cols);
          // the partner of element i is element i ^ 1 of the same loaded view (cols
          // is even, so pairs never straddle rows or tiles).
          const TileVal& src = k.tiles.at(t.ins[0]);
          if (src.op != "load") {
            *err = "mlir_to_hip: " + k.name + ": rope input must come straight from a load";
            return false;
          }
          const std::string r = "r" + std::to_string(n);
          os << "    const float " << r << "_f = 1.0f / powf(10000.0f, 2.0f * static_cast<float>(col >> 1) / "
             << fconst(static_cast<double>(C)) << ");\n";
          os << "    const float " << r << "_a = " << fconst(t.scalars[0]) << " * " << r << "_f;\n";
          os << "    const float " << r << "_c = cosf(" << r << "_a), " << r << "_s = sinf(" << r << "_a);\n";
          os << "    const float " << r << "_p = " << load_at(src, "i ^ 1ull") << ";\n";
          e << "((col & 1u) == 0u ? " << in(0) << " * " << r << "_c - " << r << "_p * " << r << "_s : " << r
            << "_p * " << r << "_s + " << in(0) << " * " << r << "_c)";
        } else if (o == "add_f32" || o == "add_f16") e << in(0) << " + " << in(1);
        else if (o == "sub_f32") e << in(0) << " - " << in(1);
        else if (o == "mul_f32" || o == "mul_f16") e << in(0) << " * " << in(1);
        else if (o == "div_f32") e << in(0) << " / " << in(1);
        // linalg.max / linalg.min / arith.maximumf / arith.minimumf: NaN-propagating
        else if (o == "max_f32") e << "th::maximumf(" << in(0) << ", " << in(1) << ")";
        else if (o == "min_f32") e << "th::minimumf(" << in(0) << ", " << in(1) << ")";
        else if (o == "log_f32") e << "logf(" << in(0) << ")";
        else if (o == "tanh_f32") e << "tanhf(" << in(0) << ")";
        else if (o == "abs_f32") e << "fabsf(" << in(0) << ")";
        else if (o == "sqrt_f32") e << "sqrtf(" << in(0) << ")";
        else if (o == "rsqrt_f32") e << "(1.0f / sqrtf(" << in(0) << "))";
        // sigmoid and relu as the linalg bridge's generic bodies (mlir_to_linalg.rs:765-789)
        else if (o == "sigmoid_f32") e << "(1.0f / (expf(-" << in(0) << ") + 1.0f))";
        else if (o == "relu_f32") e << "th::maximumf(" << in(0) << ", 0.0f)";
        else if (o == "exp_f32" || o == "exp_f16") e << "expf(" << in(0) << ")";
        else if (o == "neg_f32" || o == "neg_f16") e << "-" << in(0);
        else if (o == "silu_f32" || o == "silu_f16") e << in(0) << " / (1.0f + expf(-" << in(0) << "))";
        else if (o == "scale_f32") e << in(0) << " * " << fconst(t.scalars[0]);
        else if (o == "clamp_f32")
          e << "th::minimumf(th::maximumf(" << in(0) << ", " << fconst(t.scalars[0]) << "), "
            << fconst(t.scalars[1]) << ")";
        else if (o == "fill_f32") e << fconst(t.scalars[0]);
        else if (o == "causal_mask_f32") e << "(col <= row ? " << in(0) << " : -INFINITY)";
        else if (o == "cast_f32_f16") e << "th::f16_to_f32(th::f32_to_f16(" << in(0) << "))";
        else if (o == "cast_f32_bf16") e << "th::bf16_to_f32(th::f32_to_bf16(" << in(0) << "))";
        else if (o == "cast_f16_f32" || o == "cast_bf16_f32") e << in(0);
        else {
          *err = "mlir_to_hip: " + k.name + ": unsupported elementwise op " + t.op;
          return false;
        }
        os << "    const float " << v << " = " << e.str() << ";\n";
        var[kv.first] = v;
        progress = true;
      }
    }
    for (const Store& s : k.stores) {
      const std::string p = "reinterpret_cast<" + std::string(dt_ctype(s.dtype)) + "*>(p" +
                            std::to_string(s.dst.arg) + ")";
      const std::string idx = std::to_string(s.dst.offset) + "ll + static_cast<int64_t>(i)";
      if (s.dtype == F32) os << "    " << p << "[" << idx << "] = " << var.at(s.value) << ";\n";
      else
        os << "    " << p << "[" << idx << "] = th::f32_to_u16<" << dt_enum(s.dtype) << ">("
           << var.at(s.value) << ");\n";
    }
    os << "  }\n}\n";
    const long long per = (R * C + 255) / 256;
    desc(os, k, 256, static_cast<unsigned>(per > 1024 ? 1024 : per), 1);
    return true;
  }

  auto in_ptr = [&](int i, const char* ctype) {
    const TileVal& t = k.tiles.at(hot->ins[i]);
    return "(reinterpret_cast<const " + std::string(ctype) + "*>(p" + std::to_string(t.src.arg) +
           ")" + (t.src.offset ? " + " + std::to_string(t.src.offset) + "ll" : "") + ")";
  };
  auto out_ptr = [&](const char* ctype) {
    return "(reinterpret_cast<" + std::string(ctype) + "*>(p" + std::to_string(st->dst.arg) + ")" +
           (st->dst.offset ? " + " + std::to_string(st->dst.offset) + "ll" : "") + ")";
  };
  const std::string o = hot->op.substr(7);
  if (o == "softmax_f32" || o == "softmax_f16") {
    const TileVal& x = k.tiles.at(hot->ins[0]);
    const long long R = hot->rows, C = hot->cols;
    if (x.rows * x.cols != R * C || st->rows * st->cols != R * C || st->dtype != x.dtype) {
      *err = "mlir_to_hip: " + k.name + ": softmax shape/dtype mismatch between load and store";
      return false;
    }
    const int E = x.dtype == F32 ? 4 : 8;
    const long long nvec = C / E;
    int nv = 0;  // 0 = any-cols path
    const bool aligned = (C % E == 0) && (x.src.offset % E == 0) && (st->dst.offset % E == 0);
    if (aligned && nvec <= 64 * 16) nv = nvec <= 64 ? 1 : nvec <= 128 ? 2 : nvec <= 256 ? 4 : nvec <= 512 ? 8 : 16;
    const bool stream = k.depth != 1;   // pipelined_for(1): no next row in flight
    if (aligned && nvec > 64 * 16 && nvec <= 256 * 16) {
      // one workgroup per row, the row in registers
      const int wnv = nvec <= 256 * 8 ? 8 : 16;
      os << "row softmax " << R << "x" << C << " " << dt_name(x.dtype)
         << " per tile -> th::entry::softmax_rows_wg (one workgroup per row)\n";
      signature(os, k, 256, {});
      os << "  th::entry::softmax_rows_wg<" << dt_enum(x.dtype) << ", " << wnv << ">("
         << in_ptr(0, dt_ctype(x.dtype)) << ", " << out_ptr(dt_ctype(x.dtype)) << ", th_tiles * "
         << u(R) << ", " << u(C) << ");\n}\n";
      desc(os, k, 256, static_cast<unsigned>(R), 1);
      return true;
    }
    os << "row softmax " << R << "x" << C << " " << dt_name(x.dtype) << " per tile"
       << (k.loop.present ? " (counted loop" + std::string(k.depth ? ", pipelined_for(" + std::to_string(k.depth) + ")" : "") + ")" : "")
       << " -> th::entry::softmax_rows\n";
    signature(os, k, 256, {});
    os << "  th::entry::softmax_rows<" << dt_enum(x.dtype) << ", " << nv << (stream ? "" : ", false")
       << ">(" << in_ptr(0, dt_ctype(x.dtype)) << ", " << out_ptr(dt_ctype(x.dtype)) << ", th_tiles * "
       << u(R) << ", " << u(C) << ");\n}\n";
    // Rows per workgroup: 16 for the streaming loop (nv <= 4: each of the 4 waves
    // walks about 4 rows, next row in flight), 4 (one per wave) otherwise.
    const long long per_wg = (stream && nv > 0 && nv <= 4) ? 16 : 4;
    const unsigned tpw = R >= per_wg ? 1 : static_cast<unsigned>(per_wg / R);
    const unsigned wpt = R >= per_wg ? static_cast<unsigned>((R + per_wg - 1) / per_wg) : 1;
    desc(os, k, 256, wpt, tpw);
    return true;
  }
  if (o.rfind("matmul", 0) == 0) {
    matmul_entry(k, *hot, *st, "th::gemm::kEpiStore", nullptr, os, err);
    return err->empty();
  }
  if (o == "rms_norm_f32") {
    const TileVal& x = k.tiles.at(hot->ins[0]);
    const long long R = hot->rows, C = hot->cols;
    if (x.rows * x.cols != R * C || st->rows * st->cols != R * C || st->dtype != x.dtype) {
      *err = "mlir_to_hip: " + k.name + ": rms_norm shape/dtype mismatch between load and store";
      return false;
    }
    // 16-byte vectors per lane for the streaming loop (rows held in registers),
    // as for softmax; 0 = the two-pass any-cols path.
    const int E = x.dtype == F32 ? 4 : 8;
    const long long nvec = C / E;
    int nv = 0;
    const bool aligned = (C % E == 0) && (x.src.offset % E == 0) && (st->dst.offset % E == 0);
    if (aligned && nvec <= 64 * 16 && k.depth != 1)
      nv = nvec <= 64 ? 1 : nvec <= 128 ? 2 : nvec <= 256 ? 4 : nvec <= 512 ? 8 : 16;
    if (aligned && nvec > 64 * 16 && nvec <= 256 * 16) {
      // one workgroup per row, the row in registers
      const int wnv = nvec <= 256 * 8 ? 8 : 16;
      os << "row rms_norm " << R << "x" << C << " " << dt_name(x.dtype) << " eps "
         << hot->scalars[0] << " per tile -> th::entry::rms_norm_rows_wg (one workgroup per row)\n";
      signature(os, k, 256, {});
      os << "  th::entry::rms_norm_rows_wg<" << dt_enum(x.dtype) << ", " << wnv << ">("
         << in_ptr(0, dt_ctype(x.dtype)) << ", " << out_ptr(dt_ctype(x.dtype)) << ", th_tiles * "
         << u(R) << ", " << u(C) << ", " << fconst(hot->scalars[0]) << ");\n}\n";
      desc(os, k, 256, static_cast<unsigned>(R), 1);
      return true;
    }
    os << "row rms_norm " << R << "x" << C << " " << dt_name(x.dtype) << " eps "
       << hot->scalars[0] << " per tile -> th::entry::rms_norm_rows\n";
    signature(os, k, 256, {});
    os << "  th::entry::rms_norm_rows<" << dt_enum(x.dtype) << ", " << nv << ">("
       << in_ptr(0, dt_ctype(x.dtype)) << ", " << out_ptr(dt_ctype(x.dtype)) << ", th_tiles * "
       << u(R) << ", " << u(C) << ", " << fconst(hot->scalars[0]) << ");\n}\n";
    // rows per workgroup: 8 for the streaming loop (measured for 8192 x 4096 bf16:
    // 24.4 us at 8, 25.3 at 16, 27-28 at 10-12), 4 (one per wave) otherwise
    const long long per_wg = nv > 0 ? 8 : 4;
    const unsigned tpw = R >= per_wg ? 1 : static_cast<unsigned>(per_wg / R);
    const unsigned wpt = R >= per_wg ? static_cast<unsigned>((R + per_wg - 1) / per_wg) : 1;
    desc(os, k, 256, wpt, tpw);
    return true;
  }
  if (o == "reduce_sum_f32" || o == "reduce_max_f32" || o == "absmax_f32" || o == "argmax_f32") {
    const TileVal& x = k.tiles.at(hot->ins[0]);
    const long long R = hot->rows, C = hot->cols;
    if (x.rows * x.cols != R * C || x.dtype != F32) {
      *err = "mlir_to_hip: " + k.name + ": " + o + " input must be an f32 " + std::to_string(R) +
             "x" + std::to_string(C) + " tile";
      return false;
    }
    // one value per row; the stored view is rows x 1 (or declares the rows)
    if (st->rows * st->cols != R && st->rows != R) {
      *err = "mlir_to_hip: " + k.name + ": " + o + " stores one value per row";
      return false;
    }
    const char* op = o == "reduce_sum_f32" ? "th::entry::kRowSum"
                     : o == "reduce_max_f32" ? "th::entry::kRowMax"
                     : o == "absmax_f32" ? "th::entry::kRowAbsMax" : "th::entry::kRowArgMax";
    os << "row " << o.substr(0, o.size() - 4) << " " << R << "x" << C << " f32 per tile"
       << (o == "argmax_f32" ? " (i32 indices)" : "") << " -> th::entry::reduce_rows\n";
    signature(os, k, 256, {});
    os << "  th::entry::reduce_rows<" << op << ">(" << in_ptr(0, "float") << ", "
       << out_ptr("float") << ", th_tiles, " << u(R) << ", " << u(C) << ", "
       << st->rows * st->cols << "ull);\n}\n";
    const long long wpt = (R + 3) / 4;
    desc(os, k, 256, static_cast<unsigned>(wpt > 1024 ? 1024 : wpt), 1);
    return true;
  }
  if (o == "transpose_f32") {
    const TileVal& x = k.tiles.at(hot->ins[0]);
    const long long R = hot->rows, C = hot->cols;
    if (x.rows * x.cols != R * C || st->rows * st->cols != R * C || x.dtype != F32 ||
        st->dtype != F32) {
      *err = "mlir_to_hip: " + k.name + ": transpose needs f32 tiles of " + std::to_string(R * C) +
             " elements";
      return false;
    }
    os << "transpose " << R << "x" << C << " f32 per tile -> th::entry::transpose\n";
    signature(os, k, 256, {});
    os << "  th::entry::transpose(" << in_ptr(0, "float") << ", " << out_ptr("float")
       << ", th_tiles, " << u(R) << ", " << u(C) << ");\n}\n";
    const long long blocks = ((R + 31) / 32) * ((C + 31) / 32);
    desc(os, k, 256, static_cast<unsigned>(blocks > 1024 ? 1024 : blocks), 1);
    return true;
  }
  if (o == "matvec_f32") {
    const TileVal& a = k.tiles.at(hot->ins[0]);
    const TileVal& x = k.tiles.at(hot->ins[1]);
    const long long R = hot->rows, C = hot->cols;
    if (a.rows * a.cols != R * C || x.rows * x.cols != C || st->rows * st->cols != R ||
        a.dtype != F32 || x.dtype != F32 || st->dtype != F32) {
      *err = "mlir_to_hip: " + k.name + ": matvec needs f32 a (" + std::to_string(R) + "x" +
             std::to_string(C) + "), x (" + std::to_string(C) + ") and y (" + std::to_string(R) + ")";
      return false;
    }
    os << "matvec " << R << "x" << C << " f32 per tile -> th::entry::matvec\n";
    signature(os, k, 256, {});
    os << "  th::entry::matvec(" << in_ptr(0, "float") << ", " << in_ptr(1, "float") << ", "
       << out_ptr("float") << ", th_tiles, " << u(R) << ", " << u(C) << ", " << C << "ull, " << R
       << "ull);\n}\n";
    const long long wpt = (R + 3) / 4;
    desc(os, k, 256, static_cast<unsigned>(wpt > 1024 ? 1024 : wpt), 1);
    return true;
  }
  if (o == "attention_f32") {
    const TileVal& q = k.tiles.at(hot->ins[0]);
    const long long S = hot->rows, D = hot->cols;
    if (D > 256) {
      *err = "mlir_to_hip: " + k.name + ": attention head_dim > 256";
      return false;
    }
    os << "single-head attention S=" << S << " D=" << D << " " << dt_name(q.dtype)
       << " -> th::entry::attention_tiles\n";
    signature(os, k, 256, {});
    os << "  th::entry::attention_tiles<" << dt_enum(q.dtype) << ", 256>(" << in_ptr(0, dt_ctype(q.dtype))
       << ", " << in_ptr(1, dt_ctype(q.dtype)) << ", " << in_ptr(2, dt_ctype(q.dtype)) << ", "
       << out_ptr(dt_ctype(st->dtype)) << ", " << u(S) << ", " << u(D) << ", th_tiles);\n}\n";
    // f32 with head_dim 64/128: the MFMA flash kernel, one workgroup per 128 queries;
    // otherwise one per query
    const bool flash = q.dtype == F32 && (D == 64 || D == 128);
    desc(os, k, 256, static_cast<unsigned>(flash ? (S + 127) / 128 : S), 1);
    return true;
  }
  // The prefill and decode launch descriptors read their grid from two run-time
  // scalars, which fills both scale slots; a loop bound taken from an argument
  // would need a third.
  if ((o == "attention_prefill_f32" || o == "attention_decode_f32") && k.loop.present &&
      k.loop.trip_arg >= 0) {
    *err = "mlir_to_hip: " + k.name + ": control flow: a loop with a run-time bound around " + o +
           " is not lowered (its launch already scales with two run-time sizes)";
    return false;
  }
  if (o == "attention_prefill_f32") {
    const TileVal& q = k.tiles.at(hot->ins[0]);
    os << "causal GQA prefill " << dt_name(q.dtype) << " (runtime seq_len, start_pos, max_seq, head_dim, "
       << "num_heads, num_kv_heads) -> th::entry::prefill\n";
    // the library's kernel: one 512-thread workgroup per (head, 256-query block),
    // all of LDS, one workgroup per CU
    signature(os, k, 512, {"seq_len", "start_pos", "max_seq", "head_dim", "num_heads", "num_kv_heads"}, 1);
    const char* ct = dt_ctype(q.dtype);
    os << "  th::entry::prefill<" << dt_enum(q.dtype) << ">(" << in_ptr(0, ct) << ", " << in_ptr(1, ct)
       << ", " << in_ptr(2, ct) << ", " << out_ptr(ct)
       << ", th_tiles, seq_len, start_pos, max_seq, head_dim, num_heads, num_kv_heads);\n}\n";
    // Workgroups per tile (batch element) = num_heads x ceil(seq_len / 256), read from
    // the scalar arguments at launch.
    const unsigned a_seq = static_cast<unsigned>(k.args.size()) + 0;
    const unsigned a_nh = static_cast<unsigned>(k.args.size()) + 4;
    desc(os, k, 512, 1, 1, (a_seq + 1) | ((a_nh + 1) << 8), 256u | (1u << 16), 1u << 20);
    return true;
  }
  if (o == "attention_gqa_f32" || o == "attention_gqa_f16") {
    const TileVal& q = k.tiles.at(hot->ins[0]);
    const long long NH = static_cast<long long>(hot->scalars[0]);
    const long long NKV = static_cast<long long>(hot->scalars[1]);
    const long long S = static_cast<long long>(hot->scalars[2]);
    const long long HD = static_cast<long long>(hot->scalars[3]);
    if (NH <= 0 || NKV <= 0 || NH % NKV != 0 || S <= 0 || HD <= 0 || HD > 256 ||
        NH * S * HD > 0xffffffffll) {
      *err = "mlir_to_hip: " + k.name + ": " + o + " needs num_heads a multiple of num_kv_heads, " +
             "seq_len > 0 and 0 < head_dim <= 256";
      return false;
    }
    os << "causal GQA attention, head-major Q/O [" << NH << "][" << S << "][" << HD << "], K/V [" << NKV
       << "][" << S << "][" << HD << "] " << dt_name(q.dtype) << " -> th::entry::prefill (head-major)\n";
    signature(os, k, 512, {}, 1);
    const char* ct = dt_ctype(q.dtype);
    os << "  th::entry::prefill<" << dt_enum(q.dtype) << ", true>(" << in_ptr(0, ct) << ", "
       << in_ptr(1, ct) << ", " << in_ptr(2, ct) << ", " << out_ptr(ct) << ", th_tiles, " << u(S)
       << ", 0u, " << u(S) << ", " << u(HD) << ", " << u(NH) << ", " << u(NKV) << ");\n}\n";
    // 16-bit with head_dim 128 or 64: the library's kernel, one workgroup per (head,
    // 256-query block); otherwise one workgroup per (head, query)
    // (the asm kernel takes 16-bit head_dim 128 and 64, as entry::prefill dispatches)
    const bool fast = q.dtype != F32 && (HD == 128 || HD == 64);
    long long wpt = fast ? NH * ((S + 255) / 256) : NH * S;
    if (wpt > (1 << 20)) wpt = 1 << 20;
    desc(os, k, 512, static_cast<unsigned>(wpt), 1);
    return true;
  }
  if (o == "attention_decode_f32") {
    const TileVal& q = k.tiles.at(hot->ins[0]);
    os << "GQA decode " << dt_name(q.dtype) << " (runtime seq_len, max_seq, head_dim, num_heads, "
       << "num_kv_heads) -> th::entry::decode\n";
    // One workgroup per (batch, kv_head) walks all of its chunks, so two resident
    // workgroups per CU are needed to keep the K/V stream going (the unconstrained
    // build takes 264 registers per wave: one workgroup per CU).
    signature(os, k, 256, {"seq_len", "max_seq", "head_dim", "num_heads", "num_kv_heads"}, 2);
    const char* ct = dt_ctype(q.dtype);
    os << "  th::entry::decode<" << dt_enum(q.dtype) << ">(" << in_ptr(0, ct) << ", " << in_ptr(1, ct)
       << ", " << in_ptr(2, ct) << ", " << out_ptr(ct)
       << ", th_tiles, seq_len, max_seq, head_dim, num_heads, num_kv_heads);\n}\n";
    // Workgroups per tile (batch element) = num_kv_heads x ceil(seq_len / 512), one
    // per 512-position chunk, the whole grid capped at two per CU; the kernel splits
    // each (batch, kv_head)'s chunks over ceil(grid / items) workgroups and the last
    // of them merges the partials.
    const unsigned a_seq = static_cast<unsigned>(k.args.size()) + 0;
    const unsigned a_nkv = static_cast<unsigned>(k.args.size()) + 4;
    desc(os, k, 256, 1, 1, (a_nkv + 1) | ((a_seq + 1) << 8), 1u | (512u << 16), 1u << 20, 2);
    return true;
  }
  *err = "mlir_to_hip: " + k.name + ": unsupported intrinsic " + hot->op;
  return false;
}

}  // namespace

bool convert_mlir_to_hip(const std::string& mlir_text, std::string* out,
                         std::vector<std::string>* kernel_names, std::string* err) {
  mlir::Module mod;
  if (!mlir::parse_module(mlir_text, &mod, err)) return false;
  std::ostringstream os;
  os << "// Generated by tilers_hip `hip` target (gfx950) — DO NOT EDIT\n";
  os << "// Build: hipcc --genco --offload-arch=gfx950 -O3 -I <tile-rs_amd/csrc>\n";
  os << "#include \"kernels/tile_entry.hpp\"\n\n";
  int count = 0;
  for (const mlir::Func& f : mod.functions) {
    if (!f.is_entry || f.body_lines.empty() || mlir::is_builtin_helper(f.name)) continue;
    Kernel k;
    Lowerer low(f, err);
    if (!low.analyze(&k)) return false;
    if (!emit_kernel(k, os, err)) return false;
    if (kernel_names) kernel_names->push_back(k.name);
    ++count;
  }
  if (count == 0) {
    *err = "No entry-point kernel functions found in MLIR module";
    return false;
  }
  *out = os.str();
  return true;
}

}  // namespace target
}  // namespace th
