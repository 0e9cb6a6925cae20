// Std-only parser for the MLIR text that rustc_codegen_tile hands to every
// emitter.  Same contract as the reference parser
// (crates/rustc_codegen_tile/src/mlir_parse.rs):
//   - `llvm.func @name(%arg0: !llvm.ptr<1>, ...) attributes {hacc.entry} {` ... `}`
//     (pretty form, :133-160), and the generic form
//     `"llvm.func"() <{sym_name = "name", function_type = !llvm.func<...>}> ({`
//     `^bb0(...)` ... `}) {hacc.entry} : () -> ()` (:161-210);
//   - a function is an entry when its header (or generic closing line) carries
//     `hacc.entry`; arguments of type `ptr<1>` are global-memory pointers;
//   - generic body lines are normalized to the pretty form (:399-992) for the
//     ops the hip target consumes: llvm.call, llvm.mlir.constant,
//     llvm.getelementptr, llvm.return.
#pragma once

#include <optional>
#include <string>
#include <vector>

namespace th {
namespace mlir {

struct FuncArg {
  std::string name;  // "%arg0"
  std::string ty;    // "!llvm.ptr<1>"
  bool is_gm = false;
};

struct Func {
  std::string name;
  std::vector<FuncArg> args;
  bool is_entry = false;
  std::vector<std::string> body_lines;  // trimmed, pretty form
};

struct Module {
  std::vector<Func> functions;
};

// Parses `text`; never throws.  Unparseable function headers produce an error.
bool parse_module(const std::string& text, Module* out, std::string* err);

// `%r = ...` -> "%r".
std::optional<std::string> result_ssa(const std::string& line);
// Arguments of `op @callee(%a, %b) : ...` (text between '(' and ") :").
std::optional<std::vector<std::string>> call_args(const std::string& line);
// Callee of `llvm.call @name(`.
std::optional<std::string> callee(const std::string& line);
// True for the builtin helpers that are never kernels (mlir_parse.rs:1387-1397).
bool is_builtin_helper(const std::string& name);
// Pretty form of a generic-form body line; other lines are returned trimmed.
std::string normalize_generic(const std::string& line);
std::string trim(const std::string& s);

}  // namespace mlir
}  // namespace th
