// MLIR text parser for the hip target (contract: mlir_parse.hpp).
#include "target/mlir_parse.hpp"

#include <cctype>
#include <cstdlib>
#include <sstream>

namespace th {
namespace mlir {

std::string trim(const std::string& s) {
  size_t b = 0, e = s.size();
  while (b < e && std::isspace(static_cast<unsigned char>(s[b]))) ++b;
  while (e > b && std::isspace(static_cast<unsigned char>(s[e - 1]))) --e;
  return s.substr(b, e - b);
}

static int count(const std::string& s, char c) {
  int n = 0;
  for (char x : s) n += (x == c);
  return n;
}

std::optional<std::string> result_ssa(const std::string& line) {
  const std::string l = trim(line);
  if (l.empty() || l[0] != '%') return std::nullopt;
  const size_t eq = l.find(" = ");
  if (eq == std::string::npos) return std::nullopt;
  return trim(l.substr(0, eq));
}

std::optional<std::vector<std::string>> call_args(const std::string& line) {
  const size_t open = line.find('(');
  if (open == std::string::npos) return std::nullopt;
  const size_t close = line.find(") :", open + 1);
  if (close == std::string::npos) return std::nullopt;
  const std::string inner = line.substr(open + 1, close - open - 1);
  std::vector<std::string> out;
  if (trim(inner).empty()) return out;
  std::stringstream ss(inner);
  std::string part;
  while (std::getline(ss, part, ',')) out.push_back(trim(part));
  return out;
}

std::optional<std::string> callee(const std::string& line) {
  const size_t at = line.find("llvm.call @");
  if (at == std::string::npos) return std::nullopt;
  const size_t b = at + std::string("llvm.call @").size();
  size_t e = b;
  while (e < line.size() && line[e] != '(' && !std::isspace(static_cast<unsigned char>(line[e]))) ++e;
  return line.substr(b, e - b);
}

bool is_builtin_helper(const std::string& name) {
  return name == "get_block_idx" || name == "get_block_num" || name == "get_sub_block_idx" ||
         name == "get_sub_block_num" || name == "__rust_eh_personality" ||
         name.rfind("__tile_", 0) == 0 || name.rfind("__rust_", 0) == 0;
}

// Split on top-level commas (ignoring commas nested in <> or ()).
static std::vector<std::string> split_top(const std::string& s) {
  std::vector<std::string> out;
  int depth = 0;
  std::string cur;
  for (char c : s) {
    if (c == '<' || c == '(') ++depth;
    if (c == '>' || c == ')') --depth;
    if (c == ',' && depth == 0) {
      out.push_back(trim(cur));
      cur.clear();
    } else {
      cur.push_back(c);
    }
  }
  if (!trim(cur).empty()) out.push_back(trim(cur));
  return out;
}

static std::vector<FuncArg> parse_named_args(const std::string& inner) {
  std::vector<FuncArg> args;
  for (const std::string& part : split_top(inner)) {
    const size_t colon = part.find(':');
    if (colon == std::string::npos) continue;
    FuncArg a;
    a.name = trim(part.substr(0, colon));
    a.ty = trim(part.substr(colon + 1));
    a.is_gm = a.ty.find("ptr<1>") != std::string::npos;
    args.push_back(a);
  }
  return args;
}

// Text between the paren at `open` and its match.
static std::string paren_body(const std::string& s, size_t open) {
  int depth = 0;
  for (size_t i = open; i < s.size(); ++i) {
    if (s[i] == '(') ++depth;
    if (s[i] == ')' && --depth == 0) return s.substr(open + 1, i - open - 1);
  }
  return s.substr(open + 1);
}

static std::string property(const std::string& line, const std::string& key) {
  const std::string marker = key + " = ";
  const size_t p = line.find(marker);
  if (p == std::string::npos) return "";
  size_t b = p + marker.size();
  if (b < line.size() && line[b] == '"') {  // quoted string: up to the closing quote
    const size_t q = line.find('"', b + 1);
    return q == std::string::npos ? line.substr(b) : line.substr(b, q - b + 1);
  }
  size_t e = b;
  int depth = 0;
  while (e < line.size()) {
    const char c = line[e];
    if (c == '<' || c == '(' || c == '[' || c == '{') ++depth;
    if (c == '>' || c == ')' || c == ']' || c == '}') {
      if (depth == 0) break;
      --depth;
    }
    if (c == ',' && depth == 0) break;
    ++e;
  }
  return trim(line.substr(b, e - b));
}

std::string normalize_generic(const std::string& raw) {
  const std::string line = trim(raw);
  std::string lhs;
  std::string rest = line;
  if (!line.empty() && line[0] == '%') {
    const size_t eq = line.find(" = ");
    if (eq != std::string::npos) {
      lhs = line.substr(0, eq) + " = ";
      rest = line.substr(eq + 3);
    }
  }
  auto types_of = [&](const std::string& r) {
    const size_t c = r.rfind("}> : ");
    if (c != std::string::npos) return trim(r.substr(c + 4));
    const size_t c2 = r.rfind(" : ");
    return c2 == std::string::npos ? std::string() : trim(r.substr(c2 + 3));
  };
  if (rest.rfind("\"llvm.call\"", 0) == 0) {
    const size_t open = rest.find('(');
    const std::string args = paren_body(rest, open);
    std::string cal = property(rest, "callee");
    return lhs + "llvm.call " + cal + "(" + args + ") : " + types_of(rest);
  }
  if (rest.rfind("\"llvm.mlir.constant\"", 0) == 0) {
    const std::string v = property(rest, "value");
    const std::string ty = types_of(rest);
    const size_t arrow = ty.find("->");
    const std::string rty = arrow == std::string::npos ? ty : trim(ty.substr(arrow + 2));
    return lhs + "llvm.mlir.constant(" + v + ") : " + rty;
  }
  if (rest.rfind("\"llvm.getelementptr\"", 0) == 0) {
    const size_t open = rest.find('(');
    const std::vector<std::string> ops = split_top(paren_body(rest, open));
    const std::string elem = property(rest, "elem_type");
    std::string idx = ops.size() > 1 ? ops[1] : "";
    return lhs + "llvm.getelementptr " + (ops.empty() ? "" : ops[0]) + "[" + idx + "] : " +
           types_of(rest) + ", " + elem;
  }
  if (rest.rfind("\"llvm.return\"", 0) == 0) return "llvm.return";
  // control flow and integer arithmetic of a lowered loop (mlir_parse.rs:564-611)
  auto successors = [&](const std::string& r) {
    const size_t lb = r.find(")["), rb = r.find(']', lb == std::string::npos ? 0 : lb);
    if (lb == std::string::npos || rb == std::string::npos) return std::vector<std::string>();
    return split_top(r.substr(lb + 2, rb - lb - 2));
  };
  auto operand_types = [&](const std::string& r) {
    std::string t = types_of(r);
    const size_t arrow = t.find("->");
    if (arrow != std::string::npos) t = trim(t.substr(0, arrow));
    if (!t.empty() && t.front() == '(') t = paren_body(t, 0);
    return split_top(t);
  };
  if (rest.rfind("\"llvm.br\"", 0) == 0) {
    const std::vector<std::string> ops = split_top(paren_body(rest, rest.find('(')));
    const std::vector<std::string> succ = successors(rest);
    if (succ.empty()) return line;
    if (ops.empty() || ops[0].empty()) return "llvm.br " + succ[0];
    const std::vector<std::string> tys = operand_types(rest);
    std::string a = "llvm.br " + succ[0] + "(";
    for (size_t i = 0; i < ops.size(); ++i) a += (i ? ", " : "") + ops[i];
    a += " : ";
    for (size_t i = 0; i < tys.size(); ++i) a += (i ? ", " : "") + tys[i];
    return a + ")";
  }
  if (rest.rfind("\"llvm.cond_br\"", 0) == 0) {
    const std::vector<std::string> ops = split_top(paren_body(rest, rest.find('(')));
    const std::vector<std::string> succ = successors(rest);
    if (ops.empty() || succ.size() < 2) return line;
    return "llvm.cond_br " + ops[0] + ", " + succ[0] + ", " + succ[1];
  }
  static const char* kPred[] = {"eq", "ne", "slt", "sle", "sgt", "sge", "ult", "ule", "ugt", "uge"};
  if (rest.rfind("\"llvm.icmp\"", 0) == 0) {
    const std::vector<std::string> ops = split_top(paren_body(rest, rest.find('(')));
    const std::string pv = property(rest, "predicate");
    // `predicate = 9 : i64`, or the enum spelled out (`#llvm<icmp_predicate uge>`)
    int pi = std::isdigit(static_cast<unsigned char>(pv.empty() ? ' ' : pv[0]))
                 ? std::atoi(pv.c_str()) : -1;
    for (int i = 0; i < 10 && pi < 0; ++i) {
      const std::string nm = std::string(" ") + kPred[i] + ">";
      if (pv.find(nm) != std::string::npos) pi = i;
    }
    const std::vector<std::string> tys = operand_types(rest);
    if (ops.size() != 2 || pi < 0 || pi > 9) return line;
    return lhs + "llvm.icmp \"" + kPred[pi] + "\" " + ops[0] + ", " + ops[1] + " : " +
           (tys.empty() ? std::string("i32") : tys[0]);
  }
  for (const char* op : {"add", "sub", "mul", "shl"}) {
    const std::string g = std::string("\"llvm.") + op + "\"";
    if (rest.rfind(g, 0) == 0) {
      const std::vector<std::string> ops = split_top(paren_body(rest, rest.find('(')));
      const std::vector<std::string> tys = operand_types(rest);
      if (ops.size() != 2) return line;
      return lhs + "llvm." + op + " " + ops[0] + ", " + ops[1] + " : " +
             (tys.empty() ? std::string("i32") : tys[0]);
    }
  }
  // `%r = "llvm.zext"(%v) : (i32) -> i64` -> `%r = llvm.zext %v : i32 to i64`
  for (const char* op : {"zext", "sext", "trunc", "bitcast"}) {
    const std::string g = std::string("\"llvm.") + op + "\"";
    if (rest.rfind(g, 0) == 0) {
      const std::vector<std::string> ops = split_top(paren_body(rest, rest.find('(')));
      const std::string t = types_of(rest);
      const size_t arrow = t.find("->");
      const std::vector<std::string> tys = operand_types(rest);
      if (ops.size() != 1 || arrow == std::string::npos) return line;
      return lhs + "llvm." + op + " " + ops[0] + " : " + (tys.empty() ? std::string("i32") : tys[0]) +
             " to " + trim(t.substr(arrow + 2));
    }
  }
  return line;
}

static std::optional<std::string> pretty_name(const std::string& line) {
  const size_t at = line.find("llvm.func @");
  if (at == std::string::npos) return std::nullopt;
  size_t b = at + std::string("llvm.func @").size();
  size_t e = b;
  while (e < line.size() && line[e] != '(' && !std::isspace(static_cast<unsigned char>(line[e]))) ++e;
  if (e == b) return std::nullopt;
  return line.substr(b, e - b);
}

bool parse_module(const std::string& text, Module* out, std::string* err) {
  std::vector<std::string> lines;
  {
    std::stringstream ss(text);
    std::string l;
    while (std::getline(ss, l)) lines.push_back(l);
  }
  out->functions.clear();
  size_t i = 0;
  while (i < lines.size()) {
    const std::string line = trim(lines[i]);
    if (line.find("llvm.func @") != std::string::npos) {
      Func f;
      auto name = pretty_name(line);
      if (!name) {
        if (err) *err = "Cannot parse function name from: " + line;
        return false;
      }
      f.name = *name;
      const size_t open = line.find('(', line.find("llvm.func @"));
      if (open != std::string::npos) f.args = parse_named_args(paren_body(line, open));
      f.is_entry = line.find("hacc.entry") != std::string::npos;
      int depth = count(line, '{') - count(line, '}');
      ++i;
      while (i < lines.size() && depth > 0) {
        const std::string& bl = lines[i];
        depth += count(bl, '{') - count(bl, '}');
        if (depth > 0) {
          // block labels after the entry block are kept (control flow lowering)
          const std::string t = trim(bl);
          if (!t.empty() && t.rfind("^bb0", 0) != 0) f.body_lines.push_back(t);
        }
        ++i;
      }
      out->functions.push_back(std::move(f));
    } else if (line.rfind("\"llvm.func\"()", 0) == 0) {
      Func f;
      std::string sym = property(line, "sym_name");
      if (sym.size() >= 2 && sym.front() == '"') sym = sym.substr(1, sym.size() - 2);
      f.name = sym;
      // argument types from function_type = !llvm.func<void (ptr<1>, ...)>
      std::vector<FuncArg> type_args;
      {
        const std::string ft = property(line, "function_type");
        const size_t open = ft.find('(');
        if (open != std::string::npos) {
          int k = 0;
          for (const std::string& ty : split_top(paren_body(ft, open))) {
            FuncArg a;
            a.name = "%arg" + std::to_string(k++);
            a.ty = ty;
            a.is_gm = ty.find("ptr<1>") != std::string::npos;
            type_args.push_back(a);
          }
        }
      }
      std::vector<FuncArg> bb_args;
      int depth = count(line, '(') - count(line, ')');
      ++i;
      while (i < lines.size() && depth > 0) {
        const std::string bl = trim(lines[i]);
        depth += count(bl, '(') - count(bl, ')');
        if (depth <= 0) {
          f.is_entry = bl.find("hacc.entry") != std::string::npos;
        } else if (bl.rfind("^bb0(", 0) == 0) {
          bb_args = parse_named_args(paren_body(bl, bl.find('(')));
        } else if (!bl.empty() && bl.rfind("^bb0", 0) != 0) {
          f.body_lines.push_back(bl.rfind("^bb", 0) == 0 ? bl : normalize_generic(bl));
        }
        ++i;
      }
      f.args = bb_args.empty() ? type_args : bb_args;
      if (!f.name.empty()) out->functions.push_back(std::move(f));
    } else {
      ++i;
    }
  }
  return true;
}

}  // namespace mlir
}  // namespace th
