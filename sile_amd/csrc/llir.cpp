// Generic HIP code generation for sile's LLVM-like IR (LLIR).
//
// Input: a function in the printed LLIR form of the reference
// (crates/sile-llvm-ir/src/print.rs:6-57 `format_llvm_ir`, data model
// crates/sile-llvm-ir/src/ir.rs:1-279).  Output: HIP C++ with the per-program
// body `sile_llvm_ir_<name>` and a launch wrapper `sile_kernel_<name>`, compiled
// for gfx950 at run time with hiprtc, as the CPU backend compiles its
// generated C on every launch (crates/sile-backend/src/cpu/mod.rs:48-134).
//
// Semantics follow the CPU backend's C codegen
// (crates/sile-backend/src/cpu/codegen.rs, crates/sile-backend/src/emit.rs:112-177):
//   * every value is a local declared at the top; block parameters are locals
//     assigned on the branch into the block;
//   * bin / cmp / select / load / store / cast / gep lower to the C operators
//     (`&(base[i][j])` for a gep, plain assignment for a cast);
//   * block ids are the program's tile coordinates (gid0, gid1, gid2), thread
//     ids are 0 and barriers do nothing (the program's own code is one
//     thread's, also where its long loops are spread over a workgroup);
//   * exp is expf, atomic add is an atomic float add, vec.load / vec.reduce.add
//     are 4-wide loads and ((v0 + v1) + v2) + v3.
// Control flow is emitted as labels and gotos (the reference's structured
// for/if emitter produces the same execution order).  The launch wrapper
// derives the number of tiles and the pid -> (gid0, gid1) decode from the
// tile plan of the output parameter, as the CPU wrapper does
// (crates/sile-backend/src/cpu/codegen.rs:409-555); the plan itself is an
// input here (the reference computes it with `infer_tile_plan`,
// crates/sile-backend/src/emit.rs:241-296, which a HIP backend in that crate
// calls before handing the text over).  Programs are laid out one per lane,
// 64 per workgroup, or, when the function has long loops the lanes can split,
// one per workgroup (cooperative mode, below).
#include <hip/hip_runtime.h>
#include <hip/hiprtc.h>

#include <cctype>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <climits>
#include <functional>
#include <map>
#include <memory>
#include <set>
#include <sstream>
#include <string>
#include <vector>

#include "runtime_internal.h"

using sile_rt::fail;
using sile_rt::ok;

namespace {

// ---------------------------------------------------------------------------
// data model (the subset of ir.rs the printed form carries)
// ---------------------------------------------------------------------------
enum class TK { Void, I1, I32, I64, F16, F32, F64, Ptr, Vec, Arr };

struct Type {
  TK k = TK::Void;
  int addr = 0;                // Ptr: address space number
  std::shared_ptr<Type> elem;  // Ptr pointee (may be null: unknown), Vec / Arr element
  int64_t len = 0;             // Vec / Arr length
};

Type scalar(TK k) {
  Type t;
  t.k = k;
  return t;
}
Type ptr_to(const Type& pointee, int addr) {
  Type t;
  t.k = TK::Ptr;
  t.addr = addr;
  t.elem = std::make_shared<Type>(pointee);
  return t;
}

struct Operand {
  bool is_value = false;
  std::string name;  // value name (without %) or the constant's text
  enum { kInt, kFloat, kBool } ck = kInt;
};

struct Inst {
  std::string result;  // empty: no result
  Type ty;             // result type
  std::string op;      // alloca gep load store atomic memcpy bin cmp cast select call intr
  std::string sub;     // bin / cmp / cast mnemonic, intrinsic kind, callee
  int dim = 0;         // intrinsic dim / vector length
  std::vector<Operand> args;
  Type aux;            // gep source element type, alloca type
};

struct Term {
  std::string kind;  // br condbr switch ret
  Operand cond;
  std::string t, f;  // targets
  std::vector<Operand> targs, fargs;
  std::vector<std::pair<std::string, std::string>> cases;  // (literal, target)
};

struct Block {
  std::string name;
  std::vector<std::pair<std::string, Type>> params;
  std::vector<Inst> insts;
  Term term;
};

struct Param {
  std::string name;
  Type ty;
  int rank = -1, shape_offset = -1;  // ABI (rank < 0: none)
};

struct Function {
  std::string name;
  std::vector<Param> params;
  std::vector<Block> blocks;
};

struct ParseError {
  std::string msg;
};

[[noreturn]] void perr(int line, const std::string& msg) {
  throw ParseError{"LLIR line " + std::to_string(line) + ": " + msg};
}

std::string trim(const std::string& s) {
  size_t a = 0, b = s.size();
  while (a < b && isspace((unsigned char)s[a])) ++a;
  while (b > a && isspace((unsigned char)s[b - 1])) --b;
  return s.substr(a, b - a);
}

bool starts_with(const std::string& s, const std::string& p) {
  return s.compare(0, p.size(), p) == 0;
}

// Splits on commas that are not inside <...>, [...] or (...).
std::vector<std::string> split_top(const std::string& s, char sep = ',') {
  std::vector<std::string> out;
  int depth = 0;
  std::string cur;
  for (char c : s) {
    if (c == '<' || c == '[' || c == '(') ++depth;
    if (c == '>' || c == ']' || c == ')') --depth;
    if (c == sep && depth == 0) {
      out.push_back(trim(cur));
      cur.clear();
    } else {
      cur += c;
    }
  }
  if (!trim(cur).empty()) out.push_back(trim(cur));
  return out;
}

// ---- types: i1 i32 i64 f16 f32 f64 void ptr "ptr addrspace(N)" <N x T> [N x T]
struct Cursor {
  const std::string& s;
  size_t i;
  int line;
  void ws() {
    while (i < s.size() && isspace((unsigned char)s[i])) ++i;
  }
  bool eat(const std::string& p) {
    ws();
    if (s.compare(i, p.size(), p) == 0) {
      i += p.size();
      return true;
    }
    return false;
  }
  void expect(const std::string& p) {
    if (!eat(p)) perr(line, "expected '" + p + "' in: " + s);
  }
  std::string word() {  // [A-Za-z0-9_.$-]+
    ws();
    size_t a = i;
    while (i < s.size() && (isalnum((unsigned char)s[i]) || s[i] == '_' || s[i] == '.' ||
                            s[i] == '$' || s[i] == '-'))
      ++i;
    if (a == i) perr(line, "expected a word at column " + std::to_string(a) + " in: " + s);
    return s.substr(a, i - a);
  }
  int64_t integer() {
    ws();
    size_t a = i;
    if (i < s.size() && s[i] == '-') ++i;
    while (i < s.size() && isdigit((unsigned char)s[i])) ++i;
    if (a == i) perr(line, "expected an integer in: " + s);
    return std::stoll(s.substr(a, i - a));
  }
  Type type() {
    ws();
    if (eat("<")) {
      Type t;
      t.k = TK::Vec;
      t.len = integer();
      expect("x");
      t.elem = std::make_shared<Type>(type());
      expect(">");
      return t;
    }
    if (eat("[")) {
      Type t;
      t.k = TK::Arr;
      t.len = integer();
      expect("x");
      t.elem = std::make_shared<Type>(type());
      expect("]");
      return t;
    }
    const std::string w = word();
    if (w == "void") return scalar(TK::Void);
    if (w == "i1") return scalar(TK::I1);
    if (w == "i32") return scalar(TK::I32);
    if (w == "i64") return scalar(TK::I64);
    if (w == "f16") return scalar(TK::F16);
    if (w == "f32") return scalar(TK::F32);
    if (w == "f64") return scalar(TK::F64);
    if (w == "ptr") {
      Type t;
      t.k = TK::Ptr;
      size_t save = i;
      if (eat("addrspace(")) {
        t.addr = (int)integer();
        expect(")");
      } else {
        i = save;
      }
      return t;
    }
    perr(line, "unknown type '" + w + "' in: " + s);
  }
  Operand operand() {
    ws();
    Operand o;
    if (eat("%")) {
      o.is_value = true;
      o.name = word();
      return o;
    }
    const std::string w = word();
    o.name = w;
    if (w == "true" || w == "false") {
      o.ck = Operand::kBool;
    } else if (w.find_first_of(".eE") != std::string::npos || w == "inf" || w == "-inf" ||
               w == "NaN") {
      o.ck = Operand::kFloat;
    } else {
      o.ck = Operand::kInt;
    }
    return o;
  }
  // "TYPE operand"
  std::pair<Type, Operand> typed_operand() {
    Type t = type();
    Operand o = operand();
    return {t, o};
  }
  bool done() {
    ws();
    return i >= s.size();
  }
};

struct Parser {
  Function fn;
  std::map<std::string, Type> types;  // value name -> type

  const Type* type_of(const Operand& o) {
    if (!o.is_value) return nullptr;
    auto it = types.find(o.name);
    return it == types.end() ? nullptr : &it->second;
  }

  void define_value(const std::string& name, const Type& t, int line) {
    if (name.empty()) return;
    if (types.count(name)) perr(line, "value %" + name + " defined twice");
    types[name] = t;
  }

  static std::string strip_metadata(const std::string& body) {
    // a trailing " [parallel, unroll=4, ...]" (crates/sile-llvm-ir/src/print.rs:262-274)
    if (body.empty() || body.back() != ']') return body;
    const size_t open = body.rfind(" [");
    if (open == std::string::npos) return body;
    const std::string inner = body.substr(open + 2, body.size() - open - 3);
    static const char* kw[] = {"parallel", "reduction", "vectorize_width=", "unroll=",
                               "align=",   "noalias",   "readonly",         "writeonly"};
    for (const std::string& item : split_top(inner)) {
      bool known = false;
      for (const char* k : kw) known |= starts_with(item, k);
      if (!known) return body;  // part of the instruction (an array type)
    }
    return body.substr(0, open);
  }

  std::vector<Operand> arg_list(const std::string& s, int line) {
    std::vector<Operand> out;
    for (const std::string& a : split_top(s)) {
      Cursor c{a, 0, line};
      out.push_back(c.operand());
    }
    return out;
  }

  // " ; args(a, b)" style suffixes of a terminator
  std::map<std::string, std::vector<Operand>> branch_suffixes(std::string& text, int line) {
    std::map<std::string, std::vector<Operand>> out;
    size_t pos;
    while ((pos = text.rfind(" ; ")) != std::string::npos) {
      std::string suf = trim(text.substr(pos + 3));
      text = text.substr(0, pos);
      const size_t lp = suf.find('(');
      if (lp == std::string::npos || suf.back() != ')') perr(line, "bad branch arguments: " + suf);
      out[suf.substr(0, lp)] = arg_list(suf.substr(lp + 1, suf.size() - lp - 2), line);
    }
    return out;
  }

  Inst parse_inst(const std::string& raw, int line) {
    Inst in;
    std::string body = raw;
    if (starts_with(body, "%")) {
      const size_t eq = body.find(" = ");
      if (eq == std::string::npos) perr(line, "expected ' = ' in: " + raw);
      in.result = body.substr(1, eq - 1);
      body = body.substr(eq + 3);
    }
    body = strip_metadata(body);
    Cursor c{body, 0, line};
    const std::string op = c.word();
    if (op == "alloca") {
      in.op = "alloca";
      in.aux = c.type();
      c.expect(",");
      c.expect("addrspace(");
      const int as = (int)c.integer();
      c.expect(")");
      in.ty = ptr_to(in.aux, as);
    } else if (op == "getelementptr") {
      in.op = "gep";
      in.aux = c.type();
      c.expect(",");
      auto [bt, base] = c.typed_operand();
      in.args.push_back(base);
      while (c.eat(",")) {
        c.type();  // i64
        in.args.push_back(c.operand());
      }
      // result: the backends' C indexing `&base[i][j]...` of a pointer whose
      // array pointee is decayed (crates/sile-backend/src/emit.rs:164-176,
      // cpu/codegen.rs:601-664): the indices address the array's dimensions
      // in order (a tile [R x [C x f32]] takes [row, col]); a scalar pointee
      // takes one index, pointer arithmetic.  In the base's address space.
      Type pointee = in.aux;
      const size_t nidx = in.args.size() - 1;
      if (nidx == 0) perr(line, "gep without an index: " + raw);
      if (pointee.k == TK::Arr) {
        for (size_t k = 0; k < nidx; ++k) {
          if (pointee.k != TK::Arr) perr(line, "gep indexes past the array levels: " + raw);
          pointee = *pointee.elem;
        }
      } else if (nidx != 1) {
        perr(line, "gep on a scalar pointee takes one index: " + raw);
      }
      in.ty = ptr_to(pointee, bt.addr);
    } else if (op == "load") {
      in.op = "load";
      in.ty = c.type();
      c.expect(",");
      in.args.push_back(c.typed_operand().second);
    } else if (op == "store") {
      in.op = "store";
      c.type();
      in.args.push_back(c.operand());  // value
      c.expect(",");
      in.args.insert(in.args.begin(), c.typed_operand().second);  // [ptr, value]
    } else if (op == "atomicrmw") {
      in.op = "atomic";
      in.sub = c.word();  // fadd / add
      in.args.push_back(c.typed_operand().second);
      c.expect(",");
      auto [vt, v] = c.typed_operand();
      in.args.push_back(v);
      in.ty = vt;
    } else if (op == "fadd" || op == "fsub" || op == "fmul" || op == "fdiv" || op == "add" ||
               op == "sub" || op == "mul" || op == "sdiv" || op == "and" || op == "or") {
      in.op = "bin";
      in.sub = op;
      in.args.push_back(c.operand());
      c.expect(",");
      in.args.push_back(c.operand());
      const Type* t0 = type_of(in.args[0]);
      const Type* t1 = type_of(in.args[1]);
      if (t0) in.ty = *t0;
      else if (t1) in.ty = *t1;
      else in.ty = scalar(op[0] == 'f' ? TK::F32 : TK::I64);
    } else if (op == "icmp" || op == "fcmp") {
      in.op = "cmp";
      in.sub = c.word();
      in.args.push_back(c.operand());
      c.expect(",");
      in.args.push_back(c.operand());
      in.ty = scalar(TK::I1);
    } else if (op == "bitcast" || op == "sext" || op == "zext" || op == "trunc" ||
               op == "sitofp" || op == "fptosi") {
      in.op = "cast";
      in.sub = op;
      in.args.push_back(c.operand());
      c.expect("to");
      in.ty = c.type();
    } else if (op == "select") {
      in.op = "select";
      c.type();  // i1
      in.args.push_back(c.operand());
      c.expect(",");
      auto [tt, a] = c.typed_operand();
      c.expect(",");
      auto [ft, b] = c.typed_operand();
      in.args.push_back(a);
      in.args.push_back(b);
      const Type* ta = type_of(a);
      const Type* tb = type_of(b);
      in.ty = ta ? *ta : tb ? *tb : tt;
    } else if (op == "call") {
      Type rt = c.type();
      c.expect("@");
      const std::string callee = c.word();
      c.expect("(");
      const size_t close = body.rfind(')');
      if (close == std::string::npos || close < c.i) perr(line, "unterminated call: " + raw);
      std::vector<Operand> args;
      for (const std::string& a : split_top(body.substr(c.i, close - c.i))) {
        Cursor ac{a, 0, line};
        args.push_back(ac.typed_operand().second);
      }
      in.ty = rt;
      in.args = args;
      if (starts_with(callee, "llvm.nvvm.tid.") || starts_with(callee, "llvm.nvvm.ctaid.")) {
        in.op = "intr";
        in.sub = starts_with(callee, "llvm.nvvm.tid.") ? "tid" : "ctaid";
        const char d = callee.back();
        in.dim = d == 'y' ? 1 : d == 'z' ? 2 : 0;
        in.ty = scalar(TK::I64);
      } else if (callee == "llvm.nvvm.barrier0") {
        in.op = "intr";
        in.sub = "barrier";
      } else if (starts_with(callee, "llvm.exp.")) {
        in.op = "intr";
        in.sub = "exp";
      } else if (starts_with(callee, "llvm.vec.load.")) {
        in.op = "intr";
        in.sub = "vload";
        in.dim = std::stoi(callee.substr(strlen("llvm.vec.load.")));
      } else if (starts_with(callee, "llvm.vec.store.")) {
        in.op = "intr";
        in.sub = "vstore";
        in.dim = std::stoi(callee.substr(strlen("llvm.vec.store.")));
      } else if (callee == "llvm.vec.reduce.add") {
        in.op = "intr";
        in.sub = "vreduce";
      } else if (callee == "llvm.memcpy.inline") {
        in.op = "memcpy";
        if (in.args.size() < 3) perr(line, "memcpy needs dst, src, size: " + raw);
        in.args.resize(3);
      } else {
        in.op = "call";
        in.sub = callee;
      }
    } else {
      perr(line, "unknown instruction '" + op + "'");
    }
    define_value(in.result, in.ty, line);
    return in;
  }

  Term parse_term(const std::string& raw, int line) {
    Term t;
    std::string text = raw;
    if (starts_with(text, "ret")) {
      t.kind = "ret";
      return t;
    }
    if (starts_with(text, "switch")) {
      t.kind = "switch";
      Cursor c{text, 0, line};
      c.word();
      c.type();
      t.cond = c.operand();
      c.expect(",");
      c.expect("label");
      c.expect("%");
      t.t = c.word();  // default
      c.expect("[");
      while (!c.eat("]")) {
        const std::string lit = std::to_string(c.integer());
        c.expect(",");
        c.expect("label");
        c.expect("%");
        t.cases.push_back({lit, c.word()});
      }
      return t;
    }
    if (!starts_with(text, "br")) perr(line, "expected a terminator: " + raw);
    auto suffix = branch_suffixes(text, line);
    Cursor c{text, 0, line};
    c.word();  // br
    if (c.eat("label")) {
      t.kind = "br";
      c.expect("%");
      t.t = c.word();
      t.targs = suffix["args"];
    } else {
      t.kind = "condbr";
      c.type();  // i1
      t.cond = c.operand();
      c.expect(",");
      c.expect("label");
      c.expect("%");
      t.t = c.word();
      c.expect(",");
      c.expect("label");
      c.expect("%");
      t.f = c.word();
      t.targs = suffix["true_args"];
      t.fargs = suffix["false_args"];
    }
    return t;
  }

  static bool is_terminator(const std::string& s) {
    return starts_with(s, "br ") || starts_with(s, "switch ") || starts_with(s, "ret");
  }

  void parse(const std::string& text) {
    std::istringstream in(text);
    std::string raw;
    int line = 0;
    bool in_fn = false, closed = false;
    Block* cur = nullptr;
    std::map<std::string, Param*> by_name;
    while (std::getline(in, raw)) {
      ++line;
      const std::string s = trim(raw);
      if (s.empty()) continue;
      if (!in_fn) {
        if (starts_with(s, ";")) continue;  // comments before the function
        if (!starts_with(s, "define ")) perr(line, "expected 'define'");
        Cursor c{s, 0, line};
        c.word();
        c.type();  // void
        c.expect("@");
        fn.name = c.word();
        c.expect("(");
        const size_t close = s.rfind(')');
        if (close == std::string::npos || s.back() != '{') perr(line, "bad function header");
        for (const std::string& p : split_top(s.substr(c.i, close - c.i))) {
          Cursor pc{p, 0, line};
          Param prm;
          prm.ty = pc.type();
          pc.expect("%");
          prm.name = pc.word();
          fn.params.push_back(prm);
        }
        for (auto& p : fn.params) by_name[p.name] = &p;
        register_params();
        in_fn = true;
        continue;
      }
      if (s == "}") {
        closed = true;
        break;
      }
      if (starts_with(s, "; sile.param %")) {
        // "; sile.param %a [rank=2, shape_offset=0, elem=f32]"
        Cursor c{s, strlen("; sile.param %"), line};
        const std::string name = c.word();
        auto it = by_name.find(name);
        if (it == by_name.end()) perr(line, "sile.param for an unknown parameter %" + name);
        c.expect("[");
        const size_t close = s.rfind(']');
        for (const std::string& kv : split_top(s.substr(c.i, close - c.i))) {
          const size_t eq = kv.find('=');
          if (eq == std::string::npos) continue;
          const std::string k = trim(kv.substr(0, eq)), v = trim(kv.substr(eq + 1));
          if (k == "rank") it->second->rank = std::stoi(v);
          else if (k == "shape_offset") it->second->shape_offset = std::stoi(v);
          else if (k == "elem") {
            Cursor tc{v, 0, line};
            it->second->ty.elem = std::make_shared<Type>(tc.type());
          }
        }
        types[name] = it->second->ty;
        continue;
      }
      if (raw.size() && !isspace((unsigned char)raw[0]) && s.back() == ':') {
        fn.blocks.push_back(Block{});
        cur = &fn.blocks.back();
        cur->name = s.substr(0, s.size() - 1);
        continue;
      }
      if (!cur) perr(line, "instruction outside a block");
      if (starts_with(s, "; args(")) {
        // "; args(%k: i64, %acc: f32)"
        const std::string inner = s.substr(strlen("; args("), s.size() - strlen("; args(") - 1);
        for (const std::string& p : split_top(inner)) {
          Cursor pc{p, 0, line};
          pc.expect("%");
          const std::string name = pc.word();
          pc.expect(":");
          Type t = pc.type();
          cur->params.push_back({name, t});
          define_value(name, t, line);
        }
        continue;
      }
      if (starts_with(s, ";")) continue;  // other comments
      if (is_terminator(s)) {
        cur->term = parse_term(s, line);
        continue;
      }
      cur->insts.push_back(parse_inst(s, line));
    }
    if (!closed) perr(line, "missing closing '}'");
    if (fn.blocks.empty()) perr(line, "function has no blocks");
    for (const Block& b : fn.blocks)
      if (b.term.kind.empty()) perr(line, "block " + b.name + " has no terminator");
  }

  // register the parameters' types before the body is parsed
  void register_params() {
    for (const Param& p : fn.params) types[p.name] = p.ty;
  }
};

// ---------------------------------------------------------------------------
// HIP emitter
// ---------------------------------------------------------------------------
std::string c_scalar(const Type& t) {
  switch (t.k) {
    case TK::I1: return "bool";
    case TK::I32: return "int";
    case TK::I64: return "long long";
    case TK::F16: return "unsigned short";  // as the C backend (codegen.rs:674)
    case TK::F32: return "float";
    case TK::F64: return "double";
    case TK::Vec: return "llir_float4";
    default: return "void";
  }
}

// base element type and array dims of a (possibly nested) array type
void array_shape(const Type& t, Type& base, std::vector<int64_t>& dims) {
  const Type* cur = &t;
  while (cur->k == TK::Arr) {
    dims.push_back(cur->len);
    cur = cur->elem.get();
  }
  base = *cur;
}

// The pointee qualifier of a pointer in LLIR address space `addr`.  Global
// pointers (`ptr addrspace(1)`: the kernel's buffers and geps into them) keep
// their address space, so the compiler issues global loads and stores: through
// a generic pointer every access is a flat one, counted on the LDS counter as
// well, and each workgroup barrier then waits for all of the lane's stores to
// complete.  Other spaces stay generic (private and LDS tiles are declared as
// arrays, whose space the compiler knows).
std::string c_space(int addr) { return addr == 1 ? "__attribute__((address_space(1))) " : ""; }

// declaration of `name` with type t.  A pointer to an array is declared
// decayed, as a pointer to the array's first element (the backends' C form,
// crates/sile-backend/src/cpu/codegen.rs:625-664): `[R x [C x f32]]*` is
// `float (*)[C]`, `[C x f32]*` is `float*`.
std::string c_decl(const Type& t, const std::string& name) {
  if (t.k == TK::Ptr) {
    const std::string q = c_space(t.addr);
    if (!t.elem) return q + "float* " + name;  // untyped pointer: the CPU wrapper's float*
    Type base;
    std::vector<int64_t> dims;
    array_shape(*t.elem, base, dims);
    if (dims.size() <= 1) return q + c_scalar(base) + "* " + name;
    std::string d;
    for (size_t k = 1; k < dims.size(); ++k) d += "[" + std::to_string(dims[k]) + "]";
    return q + c_scalar(base) + " (*" + name + ")" + d;
  }
  return c_scalar(t) + " " + name;
}

// declaration of a kernel buffer parameter: restrict-qualified.  A DSL
// kernel's tensors are Rust references (`&T` inputs, `&mut T` outputs,
// crates/sile-core/src/kernel.rs:8-14), so no output aliases another
// parameter; the qualifier lets the compiler overlap the loads of one
// element with the stores of another.
std::string c_decl_buffer(const Type& t, const std::string& name) {
  if (t.k != TK::Ptr) return c_decl(t, name);
  const std::string q = c_space(t.addr);
  if (!t.elem) return q + "float* __restrict__ " + name;
  Type base;
  std::vector<int64_t> dims;
  array_shape(*t.elem, base, dims);
  if (dims.size() <= 1) return q + c_scalar(base) + "* __restrict__ " + name;
  std::string d;
  for (size_t k = 1; k < dims.size(); ++k) d += "[" + std::to_string(dims[k]) + "]";
  return q + c_scalar(base) + " (* __restrict__ " + name + ")" + d;
}

std::string ident(const std::string& name) {
  std::string out = "v_";
  for (char c : name) out += (isalnum((unsigned char)c) || c == '_') ? c : '_';
  return out;
}

// ---------------------------------------------------------------------------
// One workgroup per program (cooperative mode)
//
// The CPU backend runs a program on one thread (crates/sile-backend/src/cpu/codegen.rs:517-551)
// and the Metal template one thread per threadgroup
// (crates/sile-backend/src/metal/mod.rs:146-154).  A program whose tile loops
// are long (a softmax over 8192 columns, a 64 x 64 matmul tile) then runs each
// loop serially.  When the function has such a loop in a form whose
// iterations can be spread over lanes, the program runs on a workgroup of
// kCoopThreads lanes instead:
//   * a spread loop is a counted loop: header H(.., iv, ..) holding only
//     `icmp slt iv, bound` with constant start, bound and step and at least
//     kCoopMinTrip iterations, one body block B that branches back with
//     (.., iv + step, ..), no atomics, barriers, calls or memcpy in B;
//   * each other carried value is passed back unchanged (loop-invariant) or
//     is a fold the lanes can split: a sum c' = c + x (lane partials from
//     -0.0, a workgroup tree, then init + total: within fp32 rounding of the
//     sequential chain), or the max fold c' = x > c ? x : c (each lane keeps
//     its first maximum and its iteration, partials merge by value then
//     iteration, then total > init ? total : init: bit for bit the
//     sequential fold, NaN and +0 / -0 included); a fold's value is used in
//     B by its fold only;
//   * B's stores go to addresses that differ between iterations (a gep whose
//     last index is iv plus invariant terms, the other indices invariant; a
//     4-wide store at such an offset with step >= 4), and B loads an object
//     it stores only through the same pointer;
//   * a 2-D nest (row loop around a column loop whose body is a region of
//     blocks, e.g. the MMA's cell with its k loop) spreads its row x column
//     iterations as one flat loop, the region serial on each lane; with
//     every lane's slots full and the region's branches alike for all of a
//     lane's cells, a lane runs up to kCoopJam cells through one pass of the
//     region (the values that differ between them held per cell);
//   * lane l runs iterations l, l + W, ...; after the loop every lane holds
//     the folded values and the final counter; a barrier follows when another
//     lane's later access may conflict with the loop's;
//   * everything outside spread loops runs on every lane with the same values
//     (so its stores write identical values); an atomic there runs on lane 0
//     only (its result must be unused); tiles touched only by spread loops at
//     the iteration's element are split over the lanes' registers, others
//     live in LDS.
// Functions without such a loop keep one program per lane.
// ---------------------------------------------------------------------------
constexpr int kCoopThreads = 1024;
constexpr int64_t kCoopMinTrip = 256;
constexpr int64_t kCoopLdsBytes = 144 * 1024;

struct CoopFold {
  std::string param;   // carried header parameter
  int kind = 0;        // 0 unchanged, 1 sum, 2 max
  std::string next;    // the back-edge value
  std::string cond;    // max: the compare that selects the new value
};
// A load of a read-only buffer at [inv + iv] in a spread loop, kept per lane:
// the first loop (in block order) with the key (buffer, inv) stores what it
// loads in the lane's slot; later loops take the slot when the key's inv and
// the range of the loop that filled it match, and load otherwise.
struct CoopCacheUse {
  int cache = -1;
  bool fill = false;
};
struct CoopCache {
  std::string buf, inv;   // inv "" for an index of iv alone
  int64_t slots = 0;
  Type ty;                // the loaded value's type
  int64_t lo = 0, hi = 0; // the iterations the filling loop runs (constants)
};
struct CoopLoop {
  std::string header, body, exit;
  std::string iv;
  int64_t start = 0, bound = 0, step = 1;
  std::vector<CoopFold> folds;
  // step 1 and at most kCoopMaxSlots iterations a lane: lane l runs iteration
  // k W + l of slot k (k a compile-time index once unrolled)
  int64_t slots = 0;
  std::map<std::string, CoopCacheUse> cached;   // load result -> its cache
  // a workgroup barrier after the loop: unless it stores only into per-lane
  // slices and reads only those and memory the function never writes
  bool barrier = true;
  // a workgroup barrier before the loop: it writes LDS copies that code
  // outside the spread loops reads, which every lane must have done first
  bool pre_barrier = false;
  // A 2-D nest (rows > 0): `header` is the row header, `iv` the column and
  // `row_iv` the row; iteration f = row * cols + col of [0, rows * cols) runs
  // the region (the blocks between the column header and its back edges,
  // `entry` first) with that row and column.  `guards`: strides that must be
  // at least `cols` for the buffer stores of different iterations to differ
  // (checked at run time; otherwise lane 0 runs the nest in order).
  int64_t rows = 0, cols = 0;
  std::string row_iv, col_header, row_latch, entry;
  std::vector<std::string> region;
  std::vector<std::string> guards;
  // Jammed in groups of `jam` slots (every lane's slots full, every branch in
  // the region taken alike by all of a lane's cells): the region runs once a
  // group with each value that differs between a lane's cells (jam_nu) held
  // per slot, so the cells' loads and arithmetic interleave and what they
  // share (an inner loop's counter, its compare) is computed once.
  int jam = 0;
  std::set<std::string> jam_nu;
};
struct CoopPlan {
  bool on = false;
  std::map<std::string, CoopLoop> loops;   // by header block
  std::set<std::string> bodies;            // body blocks emitted inside their loop
  std::set<std::string> private_allocas;   // tiles split over the lanes (per-lane slices)
  // per-lane tiles whose elements at a constant last index c are read outside
  // the spread loops: an LDS copy of those elements (the tile minus its last
  // dimension) for each such c, written by the lane that stores the element
  std::map<std::string, std::set<int64_t>> shadows;
  // tiles [rows x cols] touched only at [row, col] by slot-form nests of that
  // shape: element f = row * cols + col is lane f % W's slot f / W
  std::set<std::string> nest_private;
  std::vector<CoopCache> caches;
  std::string why;                         // why the function stays one program per lane
};
constexpr int64_t kCoopMaxSlots = 16;
constexpr int kCoopJam = 4;   // slots a jammed nest interleaves

bool const_int(const Operand& o, int64_t& v) {
  if (o.is_value || o.ck != Operand::kInt) return false;
  try {
    v = std::stoll(o.name);
  } catch (...) {
    return false;
  }
  return true;
}

CoopPlan plan_coop(const Function& fn, const std::map<std::string, Type>& types) {
  CoopPlan plan;
  // where each value is defined: block name (function parameters: "")
  std::map<std::string, std::string> def_block;
  std::map<std::string, const Inst*> def_inst;
  for (const Block& b : fn.blocks) {
    for (auto& p : b.params) def_block[p.first] = b.name;
    for (const Inst& in : b.insts)
      if (!in.result.empty()) {
        def_block[in.result] = b.name;
        def_inst[in.result] = &in;
      }
  }
  auto block = [&](const std::string& n) -> const Block* {
    for (const Block& b : fn.blocks)
      if (b.name == n) return &b;
    return nullptr;
  };
  // the object (buffer parameter or alloca) a pointer value points into
  std::function<std::string(const std::string&)> root = [&](const std::string& v) -> std::string {
    auto it = def_inst.find(v);
    if (it == def_inst.end()) return v;  // a parameter
    if (it->second->op == "gep" && it->second->args[0].is_value) return root(it->second->args[0].name);
    return v;                            // an alloca (or an unknown pointer: itself)
  };
  int64_t alloca_bytes = 0;
  for (const Block& b : fn.blocks)
    for (const Inst& in : b.insts) {
      if (in.op == "alloca") {
        Type base;
        std::vector<int64_t> dims;
        array_shape(in.aux, base, dims);
        int64_t n = 4;
        for (int64_t d : dims) n *= d;
        alloca_bytes += n;
      }
    }

  for (const Block& h : fn.blocks) {
    if (h.params.empty() || h.insts.size() != 1 || h.term.kind != "condbr") continue;
    const Inst& cmp = h.insts[0];
    if (cmp.op != "cmp" || cmp.sub != "slt" || !cmp.args[0].is_value || !h.term.cond.is_value ||
        h.term.cond.name != cmp.result)
      continue;
    // the counter: the parameter the header compares (the reference's 2-D
    // loops carry the row before the column, tile_loops/grid.rs)
    size_t ivk = h.params.size();
    for (size_t k = 0; k < h.params.size(); ++k)
      if (h.params[k].first == cmp.args[0].name) ivk = k;
    if (ivk == h.params.size()) continue;
    CoopLoop L;
    L.header = h.name;
    L.iv = h.params[ivk].first;
    if (!const_int(cmp.args[1], L.bound)) continue;
    const Block* body = block(h.term.t);
    if (!body || !body->params.empty() || !h.term.targs.empty() || body->term.kind != "br" ||
        body->term.t != h.name || body->term.targs.size() != h.params.size())
      continue;
    L.body = body->name;
    L.exit = h.term.f;
    // iv' = iv + step
    const Operand& nx = body->term.targs[ivk];
    auto ni = nx.is_value ? def_inst.find(nx.name) : def_inst.end();
    if (ni == def_inst.end() || def_block[nx.name] != body->name || ni->second->op != "bin" ||
        ni->second->sub != "add")
      continue;
    const auto& na = ni->second->args;
    if (!((na[0].is_value && na[0].name == L.iv && const_int(na[1], L.step)) ||
          (na[1].is_value && na[1].name == L.iv && const_int(na[0], L.step))) ||
        L.step <= 0)
      continue;
    // the one entry edge from outside the loop gives a constant start
    int entries = 0;
    bool start_ok = true;
    for (const Block& b : fn.blocks) {
      if (b.name == body->name) continue;
      auto edge = [&](const std::string& t, const std::vector<Operand>& args) {
        if (t != h.name) return;
        ++entries;
        if (args.size() != h.params.size() || !const_int(args[ivk], L.start)) start_ok = false;
      };
      if (b.term.kind == "br") edge(b.term.t, b.term.targs);
      if (b.term.kind == "condbr") {
        edge(b.term.t, b.term.targs);
        edge(b.term.f, b.term.fargs);
      }
    }
    if (entries != 1 || !start_ok) continue;
    const int64_t trip = L.bound > L.start ? (L.bound - L.start + L.step - 1) / L.step : 0;
    if (trip < kCoopMinTrip) continue;

    // uses of each value inside the body (instructions and the back edge)
    std::map<std::string, int> uses;
    for (const Inst& in : body->insts)
      for (const Operand& a : in.args)
        if (a.is_value) ++uses[a.name];
    for (const Operand& a : body->term.targs)
      if (a.is_value) ++uses[a.name];
    bool ok = true;
    // loop-invariant: defined outside the loop, or computed in the body by a
    // pure operation of invariant operands (a row offset computed per iteration)
    std::map<std::string, bool> inv_memo;
    std::set<std::string> passthru;   // header parameters the back edge passes unchanged
    for (size_t k = 0; k < h.params.size(); ++k) {
      const Operand& back = body->term.targs[k];
      if (k != ivk && back.is_value && back.name == h.params[k].first) passthru.insert(back.name);
    }
    std::function<bool(const Operand&)> invariant = [&](const Operand& o) -> bool {
      if (!o.is_value) return true;
      if (passthru.count(o.name)) return true;
      auto it = def_block.find(o.name);
      const std::string db = it == def_block.end() ? "" : it->second;
      if (db == h.name) return false;
      if (db != body->name) return true;
      auto m = inv_memo.find(o.name);
      if (m != inv_memo.end()) return m->second;
      inv_memo[o.name] = false;
      const Inst& d = *def_inst[o.name];
      bool r = d.op == "bin" || d.op == "cmp" || d.op == "select" || d.op == "cast" || d.op == "gep";
      for (const Operand& a : d.args) r = r && invariant(a);
      inv_memo[o.name] = r;
      return r;
    };
    auto in_body = [&](const std::string& v) {
      auto it = def_block.find(v);
      return it != def_block.end() && it->second == body->name;
    };
    // carried values: unchanged (loop-invariant, any use) or folds
    for (size_t k = 0; k < h.params.size() && ok; ++k) {
      if (k == ivk) continue;
      CoopFold f;
      f.param = h.params[k].first;
      const Operand& back = body->term.targs[k];
      f.next = back.is_value ? back.name : "";
      if (back.is_value && back.name == f.param) {
        f.kind = 0;
      } else if (!back.is_value || !in_body(back.name) || uses[back.name] != 1) {
        ok = false;
      } else {
        const Inst& d = *def_inst[back.name];
        const Type* t = nullptr;
        auto ti = types.find(f.param);
        if (ti != types.end()) t = &ti->second;
        if (!t || t->k != TK::F32) {
          ok = false;
        } else if (d.op == "bin" && d.sub == "fadd" &&
                   ((d.args[0].is_value && d.args[0].name == f.param) !=
                    (d.args[1].is_value && d.args[1].name == f.param))) {
          f.kind = 1;
          if (uses[f.param] != 1) ok = false;
        } else if (d.op == "select" && d.args[0].is_value && d.args[2].is_value &&
                   d.args[2].name == f.param) {
          auto ci = def_inst.find(d.args[0].name);
          if (ci == def_inst.end() || !in_body(d.args[0].name) || ci->second->op != "cmp" ||
              ci->second->sub != "ogt" || !ci->second->args[1].is_value ||
              ci->second->args[1].name != f.param || !(ci->second->args[0].name == d.args[1].name &&
                                                        ci->second->args[0].is_value == d.args[1].is_value) ||
              uses[d.args[0].name] != 1 || uses[f.param] != 2) {
            ok = false;
          } else {
            f.kind = 2;
            f.cond = d.args[0].name;
          }
        } else {
          ok = false;
        }
      }
      L.folds.push_back(f);
    }
    if (!ok) continue;
    // body instructions and memory
    std::map<std::string, std::set<std::string>> stored;  // object -> store pointers / offsets
    // iv itself, or iv plus loop-invariant terms, added in any grouping (the
    // reference's `tile_base + (row * cols + col)`, tile_memory.rs:232-275):
    // a different address every iteration
    std::function<bool(const Operand&)> iter_index = [&](const Operand& o) -> bool {
      if (!o.is_value) return false;
      if (o.name == L.iv) return true;
      auto it = def_inst.find(o.name);
      if (it == def_inst.end() || !in_body(o.name)) return false;
      const Inst& a = *it->second;
      if (a.op != "bin" || a.sub != "add") return false;
      return (iter_index(a.args[0]) && invariant(a.args[1])) ||
             (iter_index(a.args[1]) && invariant(a.args[0]));
    };
    for (const Inst& in : body->insts) {
      if (in.op == "atomic" || in.op == "memcpy" || in.op == "call" || in.op == "alloca" ||
          (in.op == "intr" && in.sub == "barrier")) {
        ok = false;
        break;
      }
      if (in.op == "store" || (in.op == "intr" && in.sub == "vstore")) {
        const bool vec = in.op != "store";
        std::string obj, key;
        if (vec) {
          if (!in.args[0].is_value || !invariant(in.args[0]) || !iter_index(in.args[1]) ||
              L.step < in.dim) {
            ok = false;
            break;
          }
          obj = root(in.args[0].name);
          key = in.args[0].name + "+" + in.args[1].name;
        } else {
          const Operand& ptr = in.args[0];
          auto gi = ptr.is_value ? def_inst.find(ptr.name) : def_inst.end();
          if (gi == def_inst.end() || !in_body(ptr.name) || gi->second->op != "gep") {
            ok = false;
            break;
          }
          const Inst& g = *gi->second;
          bool gok = invariant(g.args[0]) && iter_index(g.args.back());
          for (size_t k = 1; k + 1 < g.args.size(); ++k) gok = gok && invariant(g.args[k]);
          if (!gok) {
            ok = false;
            break;
          }
          obj = root(g.args[0].name);
          key = ptr.name;
        }
        stored[obj].insert(key);
      }
    }
    if (!ok) continue;
    for (const Inst& in : body->insts) {
      if (in.op == "load" && in.args[0].is_value) {
        const std::string obj = root(in.args[0].name);
        if (stored.count(obj) && !stored[obj].count(in.args[0].name)) ok = false;
      } else if (in.op == "intr" && in.sub == "vload" && in.args[0].is_value) {
        const std::string obj = root(in.args[0].name);
        if (stored.count(obj) &&
            !stored[obj].count(in.args[0].name + "+" + (in.args[1].is_value ? in.args[1].name : "")))
          ok = false;
      }
    }
    if (!ok) continue;
    plan.loops[L.header] = L;
    plan.bodies.insert(L.body);
  }
  // Nests whose body is a region of blocks (the reference's tile loops and
  // its MMA, tile_loops/grid.rs:7-130, tile_compute/mma.rs:25-260, and its
  // column reductions, tile_compute/reduce.rs:160-277):
  //   RH(r): icmp slt r, M; true -> CH(0), false -> X
  //   CH(c): icmp slt c, N; true -> E, false -> RL
  //   RL: r' = r + 1; br RH(r')
  //   E ...: blocks entered only at E from CH and left only by br CH(c + 1)
  // or a column loop alone (M = 1: CH's false edge is the exit).  Iteration
  // f = r N + c of [0, M N) runs the region with (r, c) on lane f % W; a loop
  // inside the region stays serial on its lane (the MMA's k loop keeps its
  // order).  2-D nests first, then lone column loops.
  for (int pass = 0; pass < 2; ++pass)
  for (const Block& h : fn.blocks) {
    int64_t M = 1, N = 0, z = -1, one = 0;
    const Block* rh = pass == 0 ? &h : nullptr;
    const Block* ch = pass == 0 ? block(h.term.t) : &h;
    const Block* rl = nullptr;
    std::string rv;
    if (pass == 1) {
      bool taken = plan.loops.count(h.name) > 0;
      for (auto& kv : plan.loops)
        if (kv.second.rows > 0 && kv.second.col_header == h.name) taken = true;
      if (taken) continue;
    }
    if (rh) {
      if (rh->params.size() != 1 || rh->insts.size() != 1 || rh->term.kind != "condbr") continue;
      rv = rh->params[0].first;
      const Inst& rc = rh->insts[0];
      if (rc.op != "cmp" || rc.sub != "slt" || !rc.args[0].is_value || rc.args[0].name != rv ||
          !const_int(rc.args[1], M) || !rh->term.cond.is_value || rh->term.cond.name != rc.result)
        continue;
      if (!ch || ch == rh || rh->term.targs.size() != 1 || !const_int(rh->term.targs[0], z) || z != 0)
        continue;
    }
    if (!ch || ch->params.size() != 1 || ch->insts.size() != 1 || ch->term.kind != "condbr" ||
        !ch->term.targs.empty() || (rh && !ch->term.fargs.empty()))
      continue;
    const std::string cv = ch->params[0].first;
    const Inst& cc = ch->insts[0];
    if (cc.op != "cmp" || cc.sub != "slt" || !cc.args[0].is_value || cc.args[0].name != cv ||
        !const_int(cc.args[1], N) || !ch->term.cond.is_value || ch->term.cond.name != cc.result)
      continue;
    const Block* entry = block(ch->term.t);
    if (!entry || !entry->params.empty() || entry == ch || entry == rh) continue;
    if (rh) {
      rl = block(ch->term.f);
      if (!rl || rl == entry || rl == rh || rl->insts.size() != 1 || rl->term.kind != "br" ||
          rl->term.t != rh->name || rl->term.targs.size() != 1)
        continue;
      const Inst& a = rl->insts[0];
      if (a.op != "bin" || a.sub != "add" || !a.args[0].is_value || a.args[0].name != rv ||
          !const_int(a.args[1], one) || one != 1 || !rl->term.targs[0].is_value ||
          rl->term.targs[0].name != a.result)
        continue;
    }
    if (M <= 0 || N <= 0 || M * N < kCoopMinTrip) continue;
    const std::string rh_name = rh ? rh->name : "", rl_name = rl ? rl->name : "";
    // the region: what E reaches without passing CH
    std::set<std::string> region;
    bool ok = true;
    std::vector<std::string> work{entry->name};
    while (!work.empty() && ok) {
      const std::string n = work.back();
      work.pop_back();
      if (region.count(n)) continue;
      if (n == rh_name || n == rl_name || n == ch->name) {
        ok = false;
        break;
      }
      const Block* b = block(n);
      if (!b || b->term.kind == "ret" || b->term.kind == "switch") {
        ok = false;
        break;
      }
      region.insert(n);
      for (const std::string& t : {b->term.t, b->term.f})
        if (!t.empty() && t != ch->name) work.push_back(t);
    }
    if (!ok) continue;
    if (region.size() == 1 && N >= kCoopMinTrip) continue;   // the column loop spreads by itself
    if (!rh && region.size() == 1) continue;
    // entered only at E from CH; CH reached only from RH (with 0) and from the
    // region with c + 1; RH reached from one place outside (with 0) and RL
    int rh_entries = 0;
    for (const Block& b : fn.blocks) {
      auto edge = [&](const std::string& t, const std::vector<Operand>& args) {
        if (t.empty()) return;
        if (region.count(t) && !region.count(b.name) && !(b.name == ch->name && t == entry->name))
          ok = false;
        if (t == ch->name && (!rh || b.name != rh_name)) {
          if (!region.count(b.name)) {
            if (rh) {
              ok = false;
              return;
            }
            int64_t s0 = -1;   // a lone column loop: one entry from outside, with 0
            ++rh_entries;
            if (args.size() != 1 || !const_int(args[0], s0) || s0 != 0) ok = false;
            return;
          }
          if (args.size() != 1 || !args[0].is_value) {
            ok = false;
            return;
          }
          auto d = def_inst.find(args[0].name);
          int64_t inc = 0;
          if (d == def_inst.end() || d->second->op != "bin" || d->second->sub != "add" ||
              !d->second->args[0].is_value || d->second->args[0].name != cv ||
              !const_int(d->second->args[1], inc) || inc != 1)
            ok = false;
        }
        if (rh && t == rh_name && b.name != rl_name) {
          int64_t s0 = -1;
          ++rh_entries;
          if (args.size() != 1 || !const_int(args[0], s0) || s0 != 0) ok = false;
        }
      };
      if (b.term.kind == "br") edge(b.term.t, b.term.targs);
      if (b.term.kind == "condbr") {
        edge(b.term.t, b.term.targs);
        edge(b.term.f, b.term.fargs);
      }
    }
    if (!ok || rh_entries != 1) continue;
    auto in_region = [&](const std::string& v) {
      auto it = def_block.find(v);
      return it != def_block.end() && region.count(it->second);
    };
    // invariant over the nest: defined before it, or a pure operation of
    // invariant operands in the region
    std::map<std::string, bool> memo;
    std::function<bool(const Operand&)> invariant = [&](const Operand& o) -> bool {
      if (!o.is_value) return true;
      if ((!rv.empty() && o.name == rv) || o.name == cv) return false;
      auto it = def_block.find(o.name);
      const std::string db = it == def_block.end() ? "" : it->second;
      if ((rh && db == rh_name) || db == ch->name || (rl && db == rl_name)) return false;
      if (!region.count(db)) return true;
      auto m = memo.find(o.name);
      if (m != memo.end()) return m->second;
      memo[o.name] = false;
      auto di = def_inst.find(o.name);
      if (di == def_inst.end()) return false;        // a region block's parameter
      const Inst& d = *di->second;
      bool r = d.op == "bin" || d.op == "cmp" || d.op == "select" || d.op == "cast" || d.op == "gep";
      for (const Operand& a : d.args) r = r && invariant(a);
      memo[o.name] = r;
      return r;
    };
    // a buffer index `invariants + r * S + c` (any grouping): the stride S
    std::vector<std::string> guards;
    auto row_col_index = [&](const Operand& idx) -> bool {
      int cols_seen = 0, rows_seen = 0;
      bool good = true;
      std::function<void(const Operand&)> walk = [&](const Operand& o) {
        if (!good) return;
        if (invariant(o)) return;
        if (o.is_value && o.name == cv) {
          ++cols_seen;
          return;
        }
        auto di = o.is_value ? def_inst.find(o.name) : def_inst.end();
        if (di == def_inst.end() || !in_region(o.name)) {
          good = false;
          return;
        }
        const Inst& d = *di->second;
        if (d.op == "bin" && d.sub == "add") {
          walk(d.args[0]);
          walk(d.args[1]);
          return;
        }
        if (d.op == "bin" && d.sub == "mul") {
          const Operand* st = nullptr;
          if (!rv.empty() && d.args[0].is_value && d.args[0].name == rv) st = &d.args[1];
          else if (!rv.empty() && d.args[1].is_value && d.args[1].name == rv) st = &d.args[0];
          if (!st || !invariant(*st)) {
            good = false;
            return;
          }
          ++rows_seen;
          int64_t sv = 0;
          if (const_int(*st, sv)) {
            if (sv < N) good = false;
          } else if (st->is_value) {
            guards.push_back(st->name);
          } else {
            good = false;
          }
          return;
        }
        good = false;
      };
      walk(idx);
      return good && cols_seen == 1 && (rows_seen == 1 || (rows_seen == 0 && M == 1));
    };
    // a gep to the iteration's element: [r, c], or [0, c] of a lone column loop
    auto row_col_gep = [&](const Inst& g) {
      int64_t z0 = -1;
      const bool row_ok = rv.empty() ? (const_int(g.args[1], z0) && z0 == 0)
                                     : (g.args[1].is_value && g.args[1].name == rv);
      return g.args.size() == 3 && row_ok && g.args[2].is_value && g.args[2].name == cv;
    };
    std::vector<std::string> order;
    for (const Block& b : fn.blocks)
      if (region.count(b.name)) order.push_back(b.name);
    std::set<std::string> stored;      // objects the region stores
    std::set<std::string> store_ptrs;  // pointers it stores through
    bool any_store = false;
    for (const std::string& bn : order) {
      for (const Inst& in : block(bn)->insts) {
        if (in.op == "atomic" || in.op == "memcpy" || in.op == "call" || in.op == "alloca" ||
            (in.op == "intr" && (in.sub == "barrier" || in.sub == "vload" || in.sub == "vstore"))) {
          ok = false;
          break;
        }
        if (in.op != "store") continue;
        any_store = true;
        auto gi = in.args[0].is_value ? def_inst.find(in.args[0].name) : def_inst.end();
        if (gi == def_inst.end() || !in_region(in.args[0].name) || gi->second->op != "gep" ||
            !gi->second->args[0].is_value || !invariant(gi->second->args[0])) {
          ok = false;
          break;
        }
        const Inst& g = *gi->second;
        const std::string obj = root(g.args[0].name);
        const bool is_param = !def_inst.count(obj) && !def_block.count(obj);
        if (!(row_col_gep(g) || (is_param && g.args.size() == 2 && row_col_index(g.args[1])))) {
          ok = false;
          break;
        }
        stored.insert(obj);
        store_ptrs.insert(in.args[0].name);
      }
      if (!ok) break;
    }
    if (!ok) continue;
    // loads of what the region stores (or through a pointer of unknown
    // origin while it stores): only the iteration's own element
    for (const std::string& bn : order) {
      for (const Inst& in : block(bn)->insts) {
        if (in.op != "load" || !in.args[0].is_value) continue;
        const std::string obj = root(in.args[0].name);
        const bool known = !def_block.count(obj) || (def_inst.count(obj) && def_inst[obj]->op == "alloca");
        if (!stored.count(obj) && (known || !any_store)) continue;
        if (store_ptrs.count(in.args[0].name)) continue;
        auto gi = def_inst.find(in.args[0].name);
        if (gi == def_inst.end() || gi->second->op != "gep" || !row_col_gep(*gi->second)) ok = false;
      }
    }
    if (!ok) continue;
    CoopLoop L;
    L.header = rh ? rh_name : ch->name;
    L.exit = rh ? rh->term.f : ch->term.f;
    L.iv = cv;
    L.row_iv = rv;
    L.rows = M;
    L.cols = N;
    L.bound = M * N;
    L.col_header = ch->name;
    L.row_latch = rl_name;
    L.entry = entry->name;
    L.region = order;
    L.guards = guards;
    const int64_t slots = (M * N + kCoopThreads - 1) / kCoopThreads;
    if (slots <= kCoopMaxSlots) L.slots = slots;   // with guards: the spread branch
    // values that differ between a lane's cells: the row, the column unless
    // the column count divides the workgroup (then cell f + W keeps f's
    // column), and what depends on them (block parameters through their
    // edges' values)
    if (L.slots >= 2 && (M * N) % kCoopThreads == 0) {
      std::set<std::string> nu;
      if (kCoopThreads % N != 0) nu.insert(cv);
      if (!rv.empty()) nu.insert(rv);
      for (bool grew = true; grew;) {
        grew = false;
        for (const std::string& bn : order) {
          const Block* b = block(bn);
          for (const Inst& in : b->insts) {
            if (in.result.empty() || nu.count(in.result)) continue;
            for (const Operand& a : in.args)
              if (a.is_value && nu.count(a.name)) {
                nu.insert(in.result);
                grew = true;
                break;
              }
          }
          auto edge = [&](const std::string& t, const std::vector<Operand>& args) {
            const Block* tb = block(t);
            if (!tb || !region.count(t)) return;
            for (size_t k = 0; k < args.size() && k < tb->params.size(); ++k)
              if (args[k].is_value && nu.count(args[k].name) && !nu.count(tb->params[k].first)) {
                nu.insert(tb->params[k].first);
                grew = true;
              }
          };
          if (b->term.kind == "br") edge(b->term.t, b->term.targs);
          if (b->term.kind == "condbr") {
            edge(b->term.t, b->term.targs);
            edge(b->term.f, b->term.fargs);
          }
        }
      }
      bool uniform = true;
      for (const std::string& bn : order) {
        const Block* b = block(bn);
        if (b->term.kind == "condbr" && b->term.cond.is_value && nu.count(b->term.cond.name))
          uniform = false;
      }
      // groups of at most kCoopJam slots keep a group's values in registers
      for (int g = kCoopJam; g >= 2 && uniform && !L.jam; --g)
        if (L.slots % g == 0) L.jam = g;
      if (L.jam) L.jam_nu = nu;
    }
    plan.loops[L.header] = L;
  }
  // a nest inside another nest's region, or a loop inside one, stays serial
  {
    std::set<std::string> inner;
    for (auto& kv : plan.loops)
      if (kv.second.rows > 0)
        for (const std::string& b : kv.second.region) inner.insert(b);
    for (auto it = plan.loops.begin(); it != plan.loops.end();) {
      if (inner.count(it->first)) {
        plan.bodies.erase(it->second.body);
        it = plan.loops.erase(it);
      } else {
        ++it;
      }
    }
    for (auto& kv : plan.loops)
      if (kv.second.rows > 0) {
        if (!kv.second.row_iv.empty()) {   // a 2-D nest (a lone column loop is its own header)
          plan.bodies.insert(kv.second.col_header);
          plan.bodies.insert(kv.second.row_latch);
        }
        for (const std::string& b : kv.second.region) plan.bodies.insert(b);
      }
  }
  if (plan.loops.empty()) {
    plan.why = "no loop of at least " + std::to_string(kCoopMinTrip) + " iterations that lanes can split";
    return plan;
  }
  // Step-1 loops of at most kCoopMaxSlots iterations a lane take the slot
  // form: iteration e runs on lane e % W whatever the loop's start, in slot
  // e / W.
  for (auto& kv : plan.loops) {
    CoopLoop& L = kv.second;
    if (L.rows == 0 && L.step == 1 && L.bound > 0 &&
        (L.bound + kCoopThreads - 1) / kCoopThreads <= kCoopMaxSlots)
      L.slots = (L.bound + kCoopThreads - 1) / kCoopThreads;
  }
  // Loads of a buffer the function never writes, at [inv + iv] with inv
  // defined outside the loop, in slot-form loops: the first such loop in
  // block order fills a per-lane cache, later ones read it.
  {
    std::set<std::string> written;
    for (const Block& b : fn.blocks)
      for (const Inst& in : b.insts) {
        if ((in.op == "store" || in.op == "atomic" || (in.op == "intr" && in.sub == "vstore")) &&
            in.args[0].is_value)
          written.insert(root(in.args[0].name));
        if (in.op == "memcpy" && in.args[0].is_value) written.insert(root(in.args[0].name));
      }
    std::map<std::pair<std::string, std::string>, int> key_cache;
    for (const Block& hb : fn.blocks) {
      auto lp = plan.loops.find(hb.name);
      if (lp == plan.loops.end() || lp->second.slots == 0 || lp->second.rows > 0) continue;
      CoopLoop& L = lp->second;
      const Block* body = block(L.body);
      for (const Inst& in : body->insts) {
        if (in.op != "load" || !in.args[0].is_value || in.result.empty()) continue;
        auto gi = def_inst.find(in.args[0].name);
        if (gi == def_inst.end() || def_block[in.args[0].name] != body->name) continue;
        const Inst& g = *gi->second;
        if (g.op != "gep" || g.args.size() != 2 || !g.args[0].is_value || !g.args[1].is_value) continue;
        const std::string buf = g.args[0].name;
        if (def_inst.count(buf) || written.count(buf)) continue;   // a parameter, never written
        std::string inv;
        const std::string idx = g.args[1].name;
        if (idx != L.iv) {
          auto ai = def_inst.find(idx);
          if (ai == def_inst.end() || def_block[idx] != body->name || ai->second->op != "bin" ||
              ai->second->sub != "add")
            continue;
          const auto& aa = ai->second->args;
          const Operand* other = nullptr;
          if (aa[0].is_value && aa[0].name == L.iv) other = &aa[1];
          else if (aa[1].is_value && aa[1].name == L.iv) other = &aa[0];
          if (!other || !other->is_value) continue;
          auto od = def_block.find(other->name);
          if (od == def_block.end() || od->second == body->name || od->second == L.header) continue;
          inv = other->name;
        }
        const auto key = std::make_pair(buf, inv);
        auto kc = key_cache.find(key);
        if (kc == key_cache.end()) {
          const int c = (int)plan.caches.size();
          auto ti = types.find(in.result);
          if (ti == types.end()) continue;
          plan.caches.push_back(CoopCache{buf, inv, L.slots, ti->second, L.start, L.bound});
          key_cache[key] = c;
          L.cached[in.result] = CoopCacheUse{c, true};
        } else if (!L.cached.count(in.result)) {
          L.cached[in.result] = CoopCacheUse{kc->second, false};
        }
      }
    }
  }
  // A tile that is only touched inside step-1 spread loops (in the slot form,
  // or starting at 0) at [.., iv] (last index the loop counter) is touched at
  // element e only by lane e % W (iteration e runs on that lane in every such
  // loop): each lane keeps its slice [.., e / W] in registers instead of the
  // workgroup keeping the tile in LDS.
  {
    std::map<std::string, std::string> body_of_header;
    for (auto& kv : plan.loops) {
      if (kv.second.rows == 0) body_of_header[kv.second.body] = kv.first;
      for (const std::string& r : kv.second.region) body_of_header[r] = kv.first;
    }
    for (const Block& b : fn.blocks)
      for (const Inst& in : b.insts) {
        if (in.op != "alloca") continue;
        bool priv = true;
        bool in_nest = false, in_1d = false;   // touched by a nest / by a 1-D loop
        Type abase;
        std::vector<int64_t> adims;
        array_shape(in.aux, abase, adims);
        if (adims.empty()) priv = false;
        std::set<int64_t> cols;   // constant last indices read outside the spread loops
        // a value used only as the pointer of loads
        auto only_loaded = [&](const std::string& v) {
          for (const Block& u : fn.blocks) {
            for (const Inst& y : u.insts)
              for (size_t j = 0; j < y.args.size(); ++j)
                if (y.args[j].is_value && y.args[j].name == v && !(y.op == "load" && j == 0))
                  return false;
            for (const Operand& a : u.term.targs)
              if (a.is_value && a.name == v) return false;
            for (const Operand& a : u.term.fargs)
              if (a.is_value && a.name == v) return false;
            if (u.term.cond.is_value && u.term.cond.name == v) return false;
          }
          return true;
        };
        for (const Block& u : fn.blocks) {
          auto lp = body_of_header.find(u.name);
          const CoopLoop* L = lp == body_of_header.end() ? nullptr : &plan.loops[lp->second];
          for (const Inst& x : u.insts) {
            for (size_t k = 0; k < x.args.size(); ++k) {
              if (!x.args[k].is_value || x.args[k].name != in.result) continue;
              // in a slot-form lone column loop, at [.., col]: column col is
              // lane col % W's in every such loop and in 1-D spread loops
              if (L && L->rows > 0 && L->row_iv.empty()) {
                if (x.op == "gep" && k == 0 && L->slots > 0 && L->guards.empty() &&
                    x.args.back().is_value && x.args.back().name == L->iv &&
                    x.args.size() == adims.size() + 1) {
                  in_1d = true;
                  continue;
                }
                priv = false;
                continue;
              }
              // in a slot-form nest of the tile's shape, at [row, col]
              if (L && L->rows > 0) {
                int64_t z0 = -1;
                const bool row_ok = L->row_iv.empty()
                                        ? (x.args.size() == 3 && const_int(x.args[1], z0) && z0 == 0)
                                        : (x.args.size() == 3 && x.args[1].is_value &&
                                           x.args[1].name == L->row_iv);
                if (x.op == "gep" && k == 0 && L->slots > 0 && L->guards.empty() &&
                    adims.size() == 2 && adims[0] == L->rows && adims[1] == L->cols && row_ok &&
                    x.args[2].is_value && x.args[2].name == L->iv) {
                  in_nest = true;
                  continue;
                }
                priv = false;
                continue;
              }
              // as the base of a gep to an element (an index for each
              // dimension) in a spread loop with start 0, step 1, last index
              // the loop counter
              if (x.op == "gep" && k == 0 && L && L->step == 1 && (L->slots > 0 || L->start == 0) &&
                  x.args.back().is_value && x.args.back().name == L->iv &&
                  x.args.size() == adims.size() + 1) {
                in_1d = true;
                continue;
              }
              // outside the spread loops, a gep to an element at a constant
              // last index that only loads use (the reference's reduce reads
              // its first element, tile_compute/reduce.rs:325-335)
              int64_t c = -1;
              if (x.op == "gep" && k == 0 && !L && x.args.size() == adims.size() + 1 &&
                  const_int(x.args.back(), c) && c >= 0 && c < adims.back() &&
                  only_loaded(x.result)) {
                cols.insert(c);
                continue;
              }
              priv = false;
            }
          }
          for (const Operand& a : u.term.targs)
            if (a.is_value && a.name == in.result) priv = false;
          for (const Operand& a : u.term.fargs)
            if (a.is_value && a.name == in.result) priv = false;
        }
        if (priv && in_nest && (in_1d || !cols.empty())) priv = false;
        if (priv && in_nest) {
          plan.nest_private.insert(in.result);
          alloca_bytes -= 4 * adims[0] * adims[1];
        } else if (priv) {
          plan.private_allocas.insert(in.result);
          if (!cols.empty()) {
            plan.shadows[in.result] = cols;
            int64_t n = 4 * (int64_t)cols.size();
            for (size_t k = 0; k + 1 < adims.size(); ++k) n *= adims[k];
            alloca_bytes += n;   // the LDS copies
          }
          Type base;
          std::vector<int64_t> dims;
          array_shape(in.aux, base, dims);
          int64_t n = 4;
          for (int64_t d : dims) n *= d;
          alloca_bytes -= n;
        }
      }
  }
  if (alloca_bytes > kCoopLdsBytes) {
    plan.why = "allocas exceed the LDS budget";
    plan.loops.clear();
    plan.bodies.clear();
    return plan;
  }
  // A spread loop is followed by a workgroup barrier when another lane's later
  // access may conflict with one of its accesses: a store outside the per-lane
  // slices, or a read of memory the function writes anywhere (outside the
  // slices).  Neither: what follows touches only memory nobody writes and the
  // lane's own slice elements, ordered by the lane's program order.
  {
    std::set<std::string> written;
    for (const Block& b : fn.blocks)
      for (const Inst& in : b.insts) {
        if ((in.op == "store" || in.op == "atomic" || in.op == "memcpy" ||
             (in.op == "intr" && in.sub == "vstore")) && in.args[0].is_value)
          written.insert(root(in.args[0].name));
      }
    auto sliced = [&](const std::string& r) {
      return plan.private_allocas.count(r) || plan.nest_private.count(r);
    };
    // a buffer parameter or an alloca (else a pointer of unknown origin)
    auto known = [&](const std::string& r) {
      return !def_block.count(r) || (def_inst.count(r) && def_inst.at(r)->op == "alloca");
    };
    for (auto& kv : plan.loops) {
      CoopLoop& L = kv.second;
      bool need = false;
      std::vector<std::string> blocks = L.region;
      if (L.rows == 0) blocks.push_back(L.body);
      for (const std::string& bn : blocks)
        for (const Inst& in : block(bn)->insts) {
          const bool st = in.op == "store" || in.op == "atomic" || in.op == "memcpy" ||
                          (in.op == "intr" && in.sub == "vstore");
          const bool ld = in.op == "load" || (in.op == "intr" && in.sub == "vload");
          if (st) {
            if (!in.args[0].is_value || !sliced(root(in.args[0].name))) {
              need = true;
            } else if (plan.shadows.count(root(in.args[0].name))) {
              need = true;            // its LDS copies, read outside the loops
              L.pre_barrier = true;
            }
          }
          const Operand* src = ld ? &in.args[0] : in.op == "memcpy" ? &in.args[1] : nullptr;
          if (src) {
            if (!src->is_value) {
              need = true;
            } else {
              const std::string r = root(src->name);
              if (!known(r) || (!sliced(r) && written.count(r))) need = true;
            }
          }
        }
      L.barrier = need;
    }
  }
  // an atomic outside the spread loops runs once (lane 0): its result must be unused
  for (const Block& b : fn.blocks)
    for (const Inst& in : b.insts)
      if (in.op == "atomic" && !in.result.empty()) {
        for (const Block& u : fn.blocks) {
          for (const Inst& x : u.insts)
            for (const Operand& a : x.args)
              if (a.is_value && a.name == in.result) plan.why = "an atomic's result is used";
          for (const Operand& a : u.term.targs)
            if (a.is_value && a.name == in.result) plan.why = "an atomic's result is used";
          for (const Operand& a : u.term.fargs)
            if (a.is_value && a.name == in.result) plan.why = "an atomic's result is used";
        }
      }
  if (!plan.why.empty()) {
    plan.loops.clear();
    plan.bodies.clear();
    return plan;
  }
  plan.on = true;
  return plan;
}

// An array type with its last dimension cut to one lane's slice of kCoopThreads.
Type slice_type(const Type& t) {
  if (t.k != TK::Arr) return t;
  Type out = t;
  if (t.elem && t.elem->k == TK::Arr) {
    out.elem = std::make_shared<Type>(slice_type(*t.elem));
  } else {
    out.len = (t.len + kCoopThreads - 1) / kCoopThreads;
  }
  return out;
}

struct Emitter {
  const Function& fn;
  const std::map<std::string, Type>& types;
  const CoopPlan& coop;
  std::ostringstream o;
  const CoopLoop* cur = nullptr;   // the slot-form spread loop being emitted
  const CoopLoop* in_loop = nullptr;   // the spread loop being emitted (any form)
  std::map<std::string, std::string> relabel;   // block -> label inside a nest being emitted
  int nests = 0;
  // a jammed nest being emitted: values of its jam_nu set are written per
  // slot of the group (`v__s<k>`), the rest once
  const CoopLoop* jam = nullptr;
  int jam_k = -1;                  // the slot being written, -1 outside a replica
  std::string kslot = "coop_k";    // the C expressions of this slot and its iteration
  std::string itslot = "coop_it";

  bool per_slot(const std::string& v) const { return jam && jam->jam_nu.count(v); }
  std::string vname(const std::string& v) const {
    if (!per_slot(v)) return ident(v);
    if (jam_k < 0) throw ParseError{"internal: per-slot value %" + v + " read outside a slot"};
    return ident(v) + "__s" + std::to_string(jam_k);
  }
  void enter_slot(int k) {
    jam_k = k;
    kslot = "(coop_g * " + std::to_string(jam->jam) + " + " + std::to_string(k) + ")";
    itslot = "coop_it__s" + std::to_string(k);
  }
  void leave_slot() {
    jam_k = -1;
    kslot = "coop_k";
    itslot = "coop_it";
  }

  const Inst* def_of(const std::string& v) const {
    for (const Block& b : fn.blocks)
      for (const Inst& in : b.insts)
        if (in.result == v) return &in;
    return nullptr;
  }
  // `A_sh<c>[i0]...[i(n-2)]`: the LDS copy of a shadowed tile's elements at
  // last index c, indexed by a gep's other indices
  std::string shadow_ref(const Inst& g, int64_t c) {
    std::string r = ident(g.args[0].name) + "_sh" + std::to_string(c);
    if (g.args.size() == 2) return r + "[0]";
    for (size_t k = 1; k + 1 < g.args.size(); ++k) r += "[" + opnd(g.args[k]) + "]";
    return r;
  }

  std::string opnd(const Operand& x) {
    if (x.is_value) return vname(x.name);
    if (x.ck == Operand::kBool) return x.name;
    if (x.ck == Operand::kFloat) {
      if (x.name == "inf") return "__builtin_inff()";
      if (x.name == "-inf") return "(-__builtin_inff())";
      if (x.name == "NaN") return "__builtin_nanf(\"\")";
      return "(" + x.name + "f)";  // the decimal text as a float literal (emit.rs:104-110)
    }
    return "(" + x.name + "LL)";
  }

  static const char* bin_sym(const std::string& m) {
    if (m == "fadd" || m == "add") return "+";
    if (m == "fsub" || m == "sub") return "-";
    if (m == "fmul" || m == "mul") return "*";
    if (m == "fdiv" || m == "sdiv") return "/";
    if (m == "and") return "&";
    return "|";
  }
  static const char* cmp_sym(const std::string& p) {
    if (p == "eq") return "==";
    if (p == "ne") return "!=";
    if (p == "slt" || p == "olt") return "<";
    if (p == "sle" || p == "ole") return "<=";
    if (p == "sgt" || p == "ogt") return ">";
    return ">=";
  }

  void inst(const Inst& in) {
    if (jam && jam_k < 0) {
      // in a jammed nest: an instruction that reads or defines a per-slot
      // value runs once a slot
      bool rep = per_slot(in.result);
      for (const Operand& x : in.args) rep = rep || (x.is_value && per_slot(x.name));
      if (rep) {
        for (int k = 0; k < jam->jam; ++k) {
          enter_slot(k);
          inst(in);
        }
        leave_slot();
        return;
      }
    }
    const std::string r = in.result.empty() ? "" : vname(in.result);
    const auto& a = in.args;
    if (in.op == "alloca") return;  // storage declared at the top
    if (in.op == "gep") {
      // a per-lane slice of a tile: element e of the last dimension is the
      // lane's e / W
      if (coop.on && a[0].is_value && coop.nest_private.count(a[0].name)) {
        // [row, col] in a slot-form nest: this lane's slot
        o << "  " << r << " = &(" << opnd(a[0]) << "[" << kslot << "]);\n";
        return;
      }
      const bool slice = coop.on && a[0].is_value && coop.private_allocas.count(a[0].name);
      if (slice && !in_loop) {
        // outside the spread loops: the element's LDS copy
        auto sh = coop.shadows.find(a[0].name);
        int64_t c = -1;
        if (sh == coop.shadows.end() || !const_int(a.back(), c) || !sh->second.count(c))
          throw ParseError{"internal: per-lane tile %" + a[0].name + " addressed outside its loops"};
        o << "  " << r << " = &(" << shadow_ref(in, c) << ");\n";
        return;
      }
      // an element: its address; a sub-array: the sub-array, decayed
      const bool sub = in.ty.elem && in.ty.elem->k == TK::Arr;
      o << "  " << r << " = " << (sub ? "(" : "&(") << opnd(a[0]);
      for (size_t k = 1; k < a.size(); ++k) {
        if (slice && k + 1 == a.size() && cur && a[k].is_value && a[k].name == cur->iv)
          o << "[" << kslot << "]";   // the slot of this iteration
        else if (slice && k + 1 == a.size())
          o << "[(" << opnd(a[k]) << ") / " << kCoopThreads << "LL]";
        else
          o << "[" << opnd(a[k]) << "]";
      }
      o << ");\n";
    } else if (in.op == "load") {
      auto cu = cur ? cur->cached.find(in.result) : std::map<std::string, CoopCacheUse>::const_iterator();
      if (cur && cu != cur->cached.end()) {
        const std::string c = std::to_string(cu->second.cache);
        if (cu->second.fill) {
          o << "  " << r << " = *(" << opnd(a[0]) << ");\n";
          o << "  coop_cache" << c << "[coop_k] = " << r << ";\n";
        } else {
          const CoopCache& cc = coop.caches[cu->second.cache];
          o << "  if (coop_ok" << c << " && coop_it >= " << cc.lo << " && coop_it < " << cc.hi
            << ") " << r << " = coop_cache" << c << "[coop_k]; else " << r << " = *(" << opnd(a[0])
            << ");\n";
        }
        return;
      }
      o << "  " << r << " = *(" << opnd(a[0]) << ");\n";
    } else if (in.op == "store") {
      o << "  *(" << opnd(a[0]) << ") = " << opnd(a[1]) << ";\n";
      // the lane storing a shadowed element also writes its LDS copy
      const Inst* g = (coop.on && in_loop && a[0].is_value) ? def_of(a[0].name) : nullptr;
      if (g && g->op == "gep" && g->args[0].is_value) {
        auto sh = coop.shadows.find(g->args[0].name);
        if (sh != coop.shadows.end())
          for (int64_t c : sh->second)
            o << "  if (" << itslot << " == " << c << "LL) " << shadow_ref(*g, c) << " = "
              << opnd(a[1]) << ";\n";
      }
    } else if (in.op == "atomic" && coop.on) {
      // outside the spread loops every lane runs the program's code: add once
      o << "  if (threadIdx.x == 0) atomicAdd(" << opnd(a[0]) << ", " << opnd(a[1]) << ");\n";
    } else if (in.op == "atomic") {
      o << "  " << (r.empty() ? "" : r + " = ") << "atomicAdd(" << opnd(a[0]) << ", " << opnd(a[1])
        << ");\n";
    } else if (in.op == "memcpy") {
      o << "  __builtin_memcpy(" << opnd(a[0]) << ", " << opnd(a[1]) << ", " << opnd(a[2])
        << ");\n";
    } else if (in.op == "bin") {
      o << "  " << r << " = " << opnd(a[0]) << " " << bin_sym(in.sub) << " " << opnd(a[1])
        << ";\n";
    } else if (in.op == "cmp") {
      o << "  " << r << " = " << opnd(a[0]) << " " << cmp_sym(in.sub) << " " << opnd(a[1])
        << ";\n";
    } else if (in.op == "cast" && in.ty.k == TK::Ptr) {
      // a pointer bitcast may name another address space: convert explicitly
      o << "  " << r << " = (" << c_decl(in.ty, "") << ")(" << opnd(a[0]) << ");\n";
    } else if (in.op == "cast") {
      o << "  " << r << " = " << opnd(a[0]) << ";\n";
    } else if (in.op == "select") {
      o << "  " << r << " = (" << opnd(a[0]) << ") ? (" << opnd(a[1]) << ") : (" << opnd(a[2])
        << ");\n";
    } else if (in.op == "intr") {
      if (in.sub == "tid") o << "  " << r << " = 0;\n";
      else if (in.sub == "ctaid") o << "  " << r << " = sile_gid_" << in.dim << ";\n";
      else if (in.sub == "barrier") o << "  (void)0;\n";
      else if (in.sub == "exp") o << "  " << r << " = expf(" << opnd(a[0]) << ");\n";
      else if (in.sub == "vload")
        o << "  " << r << " = llir_vec_load_" << in.dim << "(" << opnd(a[0]) << ", " << opnd(a[1])
          << ");\n";
      else if (in.sub == "vstore")
        o << "  llir_vec_store_" << in.dim << "(" << opnd(a[0]) << ", " << opnd(a[1]) << ", "
          << opnd(a[2]) << ");\n";
      else if (in.sub == "vreduce")
        o << "  " << r << " = llir_vec_reduce_add(" << opnd(a[0]) << ");\n";
    }
  }

  // parallel assignment of branch arguments, then the jump
  // parallel assignment of branch arguments to the target's parameters
  void assign(const std::string& target, const std::vector<Operand>& args) {
    const Block* b = nullptr;
    for (const Block& x : fn.blocks)
      if (x.name == target) b = &x;
    if (!b) throw ParseError{"branch to unknown block %" + target};
    if (args.size() != b->params.size())
      throw ParseError{"branch to %" + target + " passes " + std::to_string(args.size()) +
                       " arguments for " + std::to_string(b->params.size()) + " parameters"};
    if (args.empty()) return;
    // in a jammed nest a per-slot parameter takes each slot's value
    const bool outer = jam && jam_k < 0;
    o << "  {\n";
    for (size_t k = 0; k < args.size(); ++k) {
      const int reps = outer && per_slot(b->params[k].first) ? jam->jam : 0;
      for (int s = 0; s < std::max(reps, 1); ++s) {
        if (reps) enter_slot(s);
        o << "    " << c_decl(b->params[k].second, "t" + std::to_string(k) + (reps ? "_" + std::to_string(s) : ""))
          << " = " << opnd(args[k]) << ";\n";
      }
      if (reps) leave_slot();
    }
    for (size_t k = 0; k < args.size(); ++k) {
      const int reps = outer && per_slot(b->params[k].first) ? jam->jam : 0;
      for (int s = 0; s < std::max(reps, 1); ++s) {
        if (reps) enter_slot(s);
        o << "    " << vname(b->params[k].first) << " = t" << k << (reps ? "_" + std::to_string(s) : "")
          << ";\n";
      }
      if (reps) leave_slot();
    }
    o << "  }\n";
  }

  void jump(const std::string& target, const std::vector<Operand>& args) {
    // a jammed nest's back edge: the next group sets the row and column itself
    if (!(jam && target == jam->col_header)) assign(target, args);
    auto rl = relabel.find(target);
    o << "  goto " << (rl != relabel.end() ? rl->second : "L_" + ident(target)) << ";\n";
  }

  void term(const Term& t) {
    if (t.kind == "ret") {
      o << "  return;\n";
    } else if (t.kind == "br") {
      jump(t.t, t.targs);
    } else if (t.kind == "condbr") {
      o << "  if (" << opnd(t.cond) << ") {\n";
      jump(t.t, t.targs);
      o << "  } else {\n";
      jump(t.f, t.fargs);
      o << "  }\n";
    }
  }

  bool is_shapes(const Param& p) const { return p.name == "__sile_shapes"; }

  // A loop whose header holds only its compare and whose body is one block,
  // entered only from the header and branching back to it: the body is
  // emitted inside a C loop at the header (the compiler may unroll it and
  // keep several iterations' loads in flight; each iteration still runs its
  // instructions in order).
  std::set<std::string> c_loop_bodies;
  const Block* c_loop_body(const Block& h) const {
    if (h.term.kind != "condbr" || h.insts.size() != 1 || h.insts[0].op != "cmp" ||
        !h.term.targs.empty() || !h.term.cond.is_value || h.term.cond.name != h.insts[0].result)
      return nullptr;
    const Block* b = nullptr;
    int preds = 0;
    for (const Block& x : fn.blocks) {
      if (x.name == h.term.t) b = &x;
      if (x.term.t == h.term.t) ++preds;
      if (x.term.kind == "condbr" && x.term.f == h.term.t) ++preds;
    }
    if (!b || b == &h || preds != 1 || !b->params.empty() || b->term.kind != "br" ||
        b->term.t != h.name || h.term.f == b->name)
      return nullptr;
    return b;
  }
  void block_code(const Block& b, const std::string& label) {
    o << label << ":;\n";
    if (const Block* body = c_loop_body(b)) {
      // inside a spread nest (a cell's k loop) the unrolled iterations are
      // what keeps a wave's loads in flight: 16 of them (the generated
      // canonical matmul ran 1.5x faster than with 4)
      o << "#pragma unroll " << (in_loop ? 16 : 4) << "\n  for (;;) {\n";
      inst(b.insts[0]);
      o << "  if (!(" << opnd(b.term.cond) << ")) break;\n";
      for (const Inst& in : body->insts) inst(in);
      assign(b.name, body->term.targs);
      o << "  }\n";
      jump(b.term.f, b.term.fargs);
      return;
    }
    for (const Inst& in : b.insts) inst(in);
    term(b.term);
  }

  // A 2-D nest at its row header: iteration f = row * cols + col runs the
  // region with that row and column on lane f % W, in slot f / W (slots
  // unrolled, or jammed a group at a time), or lane l runs f = l, l + W, ...
  // when the slots are too many.  With stride guards that spread runs when
  // every guarded stride is at least cols, and lane 0 runs all iterations in
  // order otherwise.  The region's back edges go to the next iteration.  Then
  // the counters take their final values, a barrier (when needed) and the row
  // header's exit branch.
  void coop_nest(const Block& rh, const CoopLoop& L) {
    const std::string id = std::to_string(nests++);
    const std::string n = std::to_string(L.cols) + "LL";
    if (L.pre_barrier) o << "  __syncthreads();\n";
    o << "  {\n";
    if (L.guards.empty()) {
      nest_copy(L, id, true);
    } else {
      o << "    const bool coop_par = true";
      for (const std::string& g : L.guards) o << " && " << ident(g) << " >= " << n;
      o << ";\n    if (coop_par) {\n";
      nest_copy(L, id + "p", true);
      o << "    } else if (threadIdx.x == 0) {\n";
      nest_copy(L, id + "s", false);
      o << "    }\n";
    }
    if (!L.row_iv.empty()) o << "    " << ident(L.row_iv) << " = " << L.rows << "LL;";
    o << "    " << ident(L.iv) << " = " << n << ";\n  }\n";
    if (L.barrier) o << "  __syncthreads();\n";
    jump(rh.term.f, rh.term.fargs);
  }

  // One copy of a nest's iterations: spread over the lanes (par) or all of
  // them in order.
  void nest_copy(const CoopLoop& L, const std::string& id, bool par) {
    const std::string mn = std::to_string(L.rows * L.cols) + "LL", n = std::to_string(L.cols) + "LL";
    // spread, a wave's 64 iterations start at a multiple of 64: with a column
    // count that 64 divides they share their row, which then goes to a scalar
    // register (and what the row alone addresses can come through the scalar
    // cache)
    auto row = [&](const std::string& it) {
      if (par && L.cols % 64 == 0 && L.rows < (int64_t(1) << 31))
        return "(long long)__builtin_amdgcn_readfirstlane((int)(" + it + " / " + n + "))";
      return it + " / " + n;
    };
    auto cell = [&](const std::string& it, const std::string& sfx) {
      if (L.row_iv.empty())
        o << "    " << ident(L.iv) << sfx << " = " << it << ";\n";
      else
        o << "    " << ident(L.row_iv) << sfx << " = " << row(it) << "; " << ident(L.iv) << sfx
          << " = " << it << " % " << n << ";\n";
    };
    if (par && L.jam) {
      const std::string g = std::to_string(L.jam);
      o << "#pragma unroll\n";
      o << "    for (int coop_g = 0; coop_g < " << L.slots / L.jam << "; ++coop_g) {\n";
      for (int k = 0; k < L.jam; ++k) {
        const std::string s = "__s" + std::to_string(k), it = "coop_it" + s;
        o << "    const long long " << it << " = (long long)(coop_g * " << g << " + " << k << ") * "
          << kCoopThreads << "LL + (long long)threadIdx.x;\n";
        if (L.jam_nu.count(L.iv)) {
          cell(it, s);
          continue;
        }
        // the column is the lane's in every slot
        if (k == 0) o << "    " << ident(L.iv) << " = " << it << " % " << n << ";\n";
        if (!L.row_iv.empty()) o << "    " << ident(L.row_iv) << s << " = " << row(it) << ";\n";
      }
    } else {
      if (par && L.slots > 0) {
        o << "#pragma unroll\n";
        o << "    for (int coop_k = 0; coop_k < " << L.slots << "; ++coop_k) {\n";
        o << "    const long long coop_it = (long long)coop_k * " << kCoopThreads
          << "LL + (long long)threadIdx.x;\n";
        o << "    if (coop_it >= " << mn << ") continue;\n";
      } else if (par) {
        o << "    for (long long coop_it = (long long)threadIdx.x; coop_it < " << mn
          << "; coop_it += " << kCoopThreads << "LL) {\n";
      } else {
        o << "    for (long long coop_it = 0; coop_it < " << mn << "; ++coop_it) {\n";
      }
      cell("coop_it", "");
    }
    for (const std::string& b : L.region) relabel[b] = "L_" + ident(b) + "_n" + id;
    relabel[L.col_header] = "coop_next" + id;
    o << "  goto " << relabel[L.entry] << ";\n";
    cur = par && L.slots > 0 ? &L : nullptr;
    jam = par && L.jam ? &L : nullptr;
    in_loop = &L;
    for (const std::string& bn : L.region) {
      if (c_loop_bodies.count(bn)) continue;   // inside its header's C loop
      const Block* b = nullptr;
      for (const Block& x : fn.blocks)
        if (x.name == bn) b = &x;
      block_code(*b, relabel[bn]);
    }
    cur = nullptr;
    jam = nullptr;
    in_loop = nullptr;
    for (const std::string& b : L.region) relabel.erase(b);
    relabel.erase(L.col_header);
    o << "    coop_next" << id << ":;\n    }\n";
  }

  // A spread loop at its header: lane l runs iterations l, l + W, ... of the
  // body with the carried values replaced by the lane's partial folds, the
  // partials are combined across the workgroup, the header's parameters get
  // their final values, a barrier orders the loop's stores, and the header's
  // exit branch follows.
  void coop_loop(const Block& h, const CoopLoop& L) {
    const Block* body = nullptr;
    for (const Block& b : fn.blocks)
      if (b.name == L.body) body = &b;
    const std::string iv = ident(L.iv), st = std::to_string(L.step), bd = std::to_string(L.bound);
    if (L.pre_barrier) o << "  __syncthreads();\n";
    o << "  {\n    const long long coop_start = " << iv << ";\n";
    for (size_t k = 0; k < L.folds.size(); ++k) {
      const CoopFold& f = L.folds[k];
      const std::string c = ident(f.param), ks = std::to_string(k);
      if (f.kind == 0) continue;  // unchanged by the loop
      o << "    const float coop_init" << ks << " = " << c << ";\n";
      if (f.kind == 1) o << "    float coop_p" << ks << " = -0.0f;\n";
      if (f.kind == 2)   // the partial's first iteration: 32-bit in the slot form
        o << "    float coop_p" << ks << " = -__builtin_inff(); "
          << (L.slots > 0 ? "int coop_i" + ks + " = INT_MAX;\n"
                          : "long long coop_i" + ks + " = LLONG_MAX;\n");
    }
    if (L.slots > 0) {
      // slot form: iteration k W + l on lane l, fully unrolled (compile-time
      // slots for the per-lane tiles and caches)
      std::set<int> fills, uses;
      for (auto& cu : L.cached) (cu.second.fill ? fills : uses).insert(cu.second.cache);
      for (int c : fills) {
        const CoopCache& cc = coop.caches[c];
        const std::string cs = std::to_string(c);
        o << "    coop_has" << cs << " = true; coop_tag" << cs << " = "
          << (cc.inv.empty() ? std::string("0") : "(long long)" + ident(cc.inv)) << ";\n";
      }
      for (int c : uses) {
        const CoopCache& cc = coop.caches[c];
        const std::string cs = std::to_string(c);
        o << "    const bool coop_ok" << cs << " = coop_has" << cs << " && coop_tag" << cs << " == "
          << (cc.inv.empty() ? std::string("0") : "(long long)" + ident(cc.inv)) << ";\n";
      }
      // the iteration, checked against the loop's constant start and bound
      // only where a slot can cross them
      o << "#pragma unroll\n";
      o << "    for (int coop_k = 0; coop_k < " << L.slots << "; ++coop_k) {\n";
      o << "    const long long coop_it = (long long)coop_k * " << kCoopThreads
        << "LL + (long long)threadIdx.x;\n";
      std::string skip;
      if (L.start > 0) skip = "coop_it < " + std::to_string(L.start) + "LL";
      if (L.slots * kCoopThreads > L.bound)
        skip += (skip.empty() ? "" : " || ") + std::string("coop_it >= ") + bd + "LL";
      if (!skip.empty()) o << "    if (" << skip << ") continue;\n";
    } else {
      // unrolled, so a lane has several iterations' loads in flight
      o << "#pragma unroll 8\n";
      o << "    for (long long coop_it = coop_start + (long long)threadIdx.x * " << st
        << "LL; coop_it < " << bd << "LL; coop_it += " << kCoopThreads << "LL * " << st << "LL) {\n";
    }
    o << "    " << iv << " = coop_it;\n";
    for (size_t k = 0; k < L.folds.size(); ++k)
      if (L.folds[k].kind != 0)
        o << "    " << ident(L.folds[k].param) << " = coop_p" << k << ";\n";
    cur = L.slots > 0 ? &L : nullptr;
    in_loop = &L;
    for (const Inst& in : body->insts) inst(in);
    cur = nullptr;
    in_loop = nullptr;
    for (size_t k = 0; k < L.folds.size(); ++k) {
      const CoopFold& f = L.folds[k];
      if (f.kind == 2)
        o << "    if (" << ident(f.cond) << ") coop_i" << k << " = "
          << (L.slots > 0 ? "(int)coop_it" : "coop_it") << ";\n";
      if (f.kind != 0) o << "    coop_p" << k << " = " << ident(f.next) << ";\n";
    }
    o << "    }\n";
    for (size_t k = 0; k < L.folds.size(); ++k) {
      const CoopFold& f = L.folds[k];
      const std::string c = ident(f.param), ks = std::to_string(k);
      if (f.kind == 0) {
        continue;
      } else if (f.kind == 1) {
        o << "    " << c << " = coop_init" << ks << " + coop_wg_sum(coop_p" << ks
          << ", coop_red_v, coop_rb);\n";
      } else {
        o << "    coop_wg_first_max(coop_p" << ks << ", coop_i" << ks << ", coop_red_v, "
          << (L.slots > 0 ? "coop_red_j" : "coop_red_i") << ", coop_rb);\n";
        o << "    " << c << " = coop_p" << ks << " > coop_init" << ks << " ? coop_p" << ks
          << " : coop_init" << ks << ";\n";
      }
    }
    o << "    " << iv << " = " << bd << "LL > coop_start ? coop_start + ((" << bd
      << "LL - coop_start + " << st << "LL - 1) / " << st << "LL) * " << st
      << "LL : coop_start;\n  }\n";
    if (L.barrier) o << "  __syncthreads();\n";
    jump(h.term.f, h.term.fargs);
  }

  void body() {
    o << "__device__ static void sile_llvm_ir_" << fn.name << "(";
    for (size_t k = 0; k < fn.params.size(); ++k) {
      const Param& p = fn.params[k];
      o << (k ? ", " : "") << (is_shapes(p) ? "long long* " + ident(p.name) : c_decl_buffer(p.ty, ident(p.name)));
    }
    o << ", long long sile_gid_0, long long sile_gid_1, long long sile_gid_2) {\n";
    o << "  (void)sile_gid_0; (void)sile_gid_1; (void)sile_gid_2;\n";
    // declarations: block parameters, instruction results, alloca storage,
    // and the per-slot copies of jammed nests' values
    std::map<std::string, int> copies;
    for (auto& kv : coop.loops)
      for (const std::string& v : kv.second.jam_nu) copies[v] = std::max(copies[v], kv.second.jam);
    auto slot_copies = [&](const Type& t, const std::string& v) {
      auto cp = copies.find(v);
      for (int k = 0; cp != copies.end() && k < cp->second; ++k)
        o << "  " << c_decl(t, ident(v) + "__s" + std::to_string(k)) << ";\n";
    };
    for (const Block& b : fn.blocks) {
      for (auto& p : b.params) {
        o << "  " << c_decl(p.second, ident(p.first)) << ";\n";
        slot_copies(p.second, p.first);
      }
      for (const Inst& in : b.insts) {
        if (in.result.empty()) continue;
        if (in.op == "alloca") {
          Type base;
          std::vector<int64_t> dims;
          array_shape(in.aux, base, dims);
          std::string d;
          for (int64_t n : dims) d += "[" + std::to_string(n) + "]";
          if (dims.empty()) d = "[1]";
          if (coop.on && coop.nest_private.count(in.result)) {
            // element f = row * cols + col of the tile is this lane's slot f / W
            int64_t n = 1;
            for (int64_t x : dims) n *= x;
            o << "  " << c_scalar(base) << " " << ident(in.result) << "_storage["
              << (n + kCoopThreads - 1) / kCoopThreads << "];\n";
            o << "  " << c_scalar(base) << "* " << ident(in.result) << " = " << ident(in.result)
              << "_storage;\n";
            continue;
          }
          // one program per workgroup: the program's tiles live in LDS, or, when
          // only spread loops touch them at [.., iv], as per-lane slices
          const bool priv = coop.on && coop.private_allocas.count(in.result);
          if (priv) {
            d.clear();
            for (size_t k = 0; k < dims.size(); ++k)
              d += "[" + std::to_string(k + 1 == dims.size()
                                             ? (dims[k] + kCoopThreads - 1) / kCoopThreads
                                             : dims[k]) + "]";
          }
          o << "  " << (coop.on && !priv ? "__shared__ " : "") << c_scalar(base) << " "
            << ident(in.result) << "_storage" << d << ";\n";
          auto sh = priv ? coop.shadows.find(in.result) : coop.shadows.end();
          if (sh != coop.shadows.end())
            for (int64_t c : sh->second) {
              std::string sd;
              for (size_t k = 0; k + 1 < dims.size(); ++k) sd += "[" + std::to_string(dims[k]) + "]";
              o << "  __shared__ " << c_scalar(base) << " " << ident(in.result) << "_sh" << c
                << (sd.empty() ? "[1]" : sd) << ";\n";
            }
          // the pointer is the storage decayed to its first element
          if (dims.empty())
            o << "  " << c_scalar(base) << "* " << ident(in.result) << " = " << ident(in.result)
              << "_storage;\n";
          else if (priv)
            o << "  " << c_decl(ptr_to(slice_type(in.aux), in.ty.addr), ident(in.result))
              << " = " << ident(in.result) << "_storage;\n";
          else
            o << "  " << c_decl(in.ty, ident(in.result)) << " = " << ident(in.result)
              << "_storage;\n";
        } else {
          o << "  " << c_decl(in.ty, ident(in.result)) << ";\n";
          slot_copies(in.ty, in.result);
        }
      }
    }
    if (coop.on)
      o << "  __shared__ float coop_red_v[2 * COOP_WAVES];\n"
           "  __shared__ long long coop_red_i[2 * COOP_WAVES];\n"
           "  __shared__ int coop_red_j[2 * COOP_WAVES];\n"
           "  int coop_rb = 0;\n";
    for (size_t c = 0; c < coop.caches.size(); ++c) {
      const std::string cs = std::to_string(c);
      o << "  " << c_scalar(coop.caches[c].ty) << " coop_cache" << cs << "[" << coop.caches[c].slots
        << "];\n  bool coop_has" << cs << " = false;\n  long long coop_tag" << cs << " = 0;\n";
    }
    std::set<std::string> spread_headers;   // spread loops' and nests' own headers
    for (auto& kv : coop.loops) {
      spread_headers.insert(kv.first);
      if (kv.second.rows > 0) spread_headers.insert(kv.second.col_header);
    }
    for (const Block& b : fn.blocks)
      if (!spread_headers.count(b.name))
        if (const Block* cb = c_loop_body(b)) c_loop_bodies.insert(cb->name);
    for (const Block& b : fn.blocks) {
      if (coop.bodies.count(b.name) || c_loop_bodies.count(b.name)) continue;  // emitted in their loop
      auto lp = coop.loops.find(b.name);
      if (lp != coop.loops.end()) {
        o << "L_" << ident(b.name) << ":;\n";
        if (lp->second.rows > 0)
          coop_nest(b, lp->second);
        else
          coop_loop(b, lp->second);
        continue;
      }
      block_code(b, "L_" + ident(b.name));
    }
    o << "}\n\n";
  }

  // the CPU backend's launch wrapper (crates/sile-backend/src/cpu/codegen.rs:409-555)
  void wrapper(int64_t plan_out, int64_t rows, int64_t cols) {
    const Param* out_param = nullptr;
    if (plan_out >= 0) {
      if (plan_out >= (int64_t)fn.params.size() || fn.params[plan_out].rank < 0)
        throw ParseError{"tile plan names parameter " + std::to_string(plan_out) +
                         ", which has no shape ABI"};
      out_param = &fn.params[plan_out];
    }
    const Param* last_buf = nullptr;
    const Param* first_buf = nullptr;
    for (const Param& p : fn.params) {
      if (is_shapes(p)) continue;
      if (!first_buf) first_buf = &p;
      last_buf = &p;
    }
    const int threads = coop.on ? kCoopThreads : 64;
    // one program per workgroup: ask for two workgroups per CU (8 waves per
    // SIMD, every wave slot: at most 64 VGPRs), so one program's loads overlap
    // the other's folds and barriers
    o << "extern \"C\" __global__ __launch_bounds__(" << threads << ") "
      << (coop.on ? "__attribute__((amdgpu_waves_per_eu(8))) " : "") << "void sile_kernel_" << fn.name
      << "(void** buffers, long long num_programs, const long long* shapes, long long num_shapes) {\n";
    if (coop.on)
      o << "  const long long sile_pid = (long long)blockIdx.x;  // one workgroup per program\n";
    else
      o << "  const long long sile_pid = (long long)blockIdx.x * 64 + threadIdx.x;\n";
    o << "  if (sile_pid >= num_programs) return;\n";
    o << "  (void)num_shapes;\n";
    // buffers in parameter order, each bound as its parameter's pointer type
    int bi = 0;
    for (const Param& p : fn.params) {
      if (is_shapes(p)) continue;
      o << "  " << c_decl(p.ty, ident(p.name)) << " = (" << c_decl(p.ty, "") << ")buffers["
        << bi++ << "];\n";
    }
    auto tile_count = [&](const Param& abi_param, int64_t r, int64_t c) {
      if (abi_param.rank == 1) {
        o << "  const long long sile_total_tiles = shapes[" << abi_param.shape_offset << "];\n";
        o << "  const long long sile_tiles_n = 1;\n";
      } else {
        o << "  const long long sile_tiles_n = shapes[" << abi_param.shape_offset + 1 << "] / " << c
          << ";\n";
        o << "  const long long sile_total_tiles = (shapes[" << abi_param.shape_offset << "] / " << r
          << ") * sile_tiles_n;\n";
      }
    };
    int output_rank = 1;
    if (out_param) {
      tile_count(*out_param, rows, cols);
      output_rank = out_param->rank;
    } else if (last_buf && last_buf->rank >= 0) {
      output_rank = last_buf->rank;
      if (last_buf->rank == 1) {
        const Param& fb = (first_buf && first_buf->rank >= 0) ? *first_buf : *last_buf;
        o << "  const long long sile_total_tiles = shapes[" << fb.shape_offset << "];\n";
        o << "  const long long sile_tiles_n = 1;\n";
      } else {
        tile_count(*last_buf, 32, 16);
      }
    } else {
      const Param* fp = fn.params.empty() ? nullptr : &fn.params[0];
      if (fp && !is_shapes(*fp) && fp->rank >= 0)
        o << "  const long long sile_total_tiles = shapes[" << fp->shape_offset << "];\n";
      else
        o << "  const long long sile_total_tiles = num_programs;\n";
      o << "  const long long sile_tiles_n = 1;\n";
      output_rank = last_buf && last_buf->rank >= 0 ? last_buf->rank : 1;
    }
    o << "  if (sile_pid < sile_total_tiles) {\n";
    if (output_rank <= 1)
      o << "    const long long g0 = sile_pid, g1 = 0;\n";
    else
      o << "    const long long g0 = sile_pid / sile_tiles_n, g1 = sile_pid % sile_tiles_n;\n";
    o << "    (void)sile_tiles_n;\n";
    o << "    sile_llvm_ir_" << fn.name << "(";
    for (size_t k = 0; k < fn.params.size(); ++k)
      o << (k ? ", " : "") << (is_shapes(fn.params[k]) ? "(long long*)shapes" : ident(fn.params[k].name));
    o << ", g0, g1, 0);\n  }\n}\n";
  }

  std::string emit(int64_t plan_out, int64_t rows, int64_t cols) {
    o << "// generated from sile LLIR function @" << fn.name << " for gfx950\n";
    o << "struct llir_float4 { float v[4]; };\n";
    o << "__device__ static inline llir_float4 llir_vec_load_4(const float* p, long long off) {\n"
         "  llir_float4 r; r.v[0] = p[off]; r.v[1] = p[off + 1]; r.v[2] = p[off + 2]; "
         "r.v[3] = p[off + 3]; return r;\n}\n";
    o << "__device__ static inline void llir_vec_store_4(float* p, long long off, llir_float4 v) {\n"
         "  p[off] = v.v[0]; p[off + 1] = v.v[1]; p[off + 2] = v.v[2]; p[off + 3] = v.v[3];\n}\n";
    o << "__device__ static inline float llir_vec_reduce_add(llir_float4 v) {\n"
         "  return v.v[0] + v.v[1] + v.v[2] + v.v[3];\n}\n\n";
    if (coop.on) {
      // Workgroup folds of the lanes' partials; every lane returns the result.
      // Within a wave: DPP steps lane ^ 1, lane ^ 2 (quad permutes), then the
      // half-row and row mirrors, after which every lane holds its 16-lane
      // row's fold; the four rows are combined from lanes 0, 16, 32, 48.  Across
      // the waves: lane 0 of each wave writes its fold to LDS, one barrier, and
      // every lane combines the waves' values in wave order.  The exchange
      // alternates between two halves of the LDS arrays (`rb`, the same
      // sequence on every lane): a fold writes the half the fold before last
      // read, which every wave finished reading before it passed the last
      // fold's barrier, so no barrier is needed before the write.
      o << "#ifndef LLONG_MAX\n#define LLONG_MAX 9223372036854775807LL\n#endif\n"
           "#ifndef INT_MAX\n#define INT_MAX 2147483647\n#endif\n"
        << "#define COOP_WAVES " << kCoopThreads / 64 << "\n"
        << "template <int C> __device__ static inline float coop_dpp_f(float v) {\n"
           "  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), C, 0xF, 0xF, false));\n}\n"
           "template <int C> __device__ static inline int coop_dpp_i(int v) {\n"
           "  return __builtin_amdgcn_update_dpp(0, v, C, 0xF, 0xF, false);\n}\n"
           "template <int C> __device__ static inline long long coop_dpp_i(long long v) {\n"
           "  const unsigned lo = (unsigned)__builtin_amdgcn_update_dpp(0, (int)(unsigned)v, C, 0xF, 0xF, false);\n"
           "  const unsigned hi = (unsigned)__builtin_amdgcn_update_dpp(0, (int)(unsigned)((unsigned long long)v >> 32), C, 0xF, 0xF, false);\n"
           "  return (long long)(((unsigned long long)hi << 32) | lo);\n}\n"
           "__device__ static inline float coop_lane_f(float v, int l) {\n"
           "  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), l));\n}\n"
           "__device__ static inline int coop_lane_i(int v, int l) {\n"
           "  return __builtin_amdgcn_readlane(v, l);\n}\n"
           "__device__ static inline long long coop_lane_i(long long v, int l) {\n"
           "  const unsigned lo = (unsigned)__builtin_amdgcn_readlane((int)(unsigned)v, l);\n"
           "  const unsigned hi = (unsigned)__builtin_amdgcn_readlane((int)(unsigned)((unsigned long long)v >> 32), l);\n"
           "  return (long long)(((unsigned long long)hi << 32) | lo);\n}\n"
           "__device__ static float coop_wg_sum(float v, float* red, int& rb) {\n"
           "  v += coop_dpp_f<0xB1>(v);\n"
           "  v += coop_dpp_f<0x4E>(v);\n"
           "  v += coop_dpp_f<0x141>(v);\n"
           "  v += coop_dpp_f<0x140>(v);\n"
           "  v = ((coop_lane_f(v, 0) + coop_lane_f(v, 16)) + coop_lane_f(v, 32)) + coop_lane_f(v, 48);\n"
           "  float* r = red + rb * COOP_WAVES;\n"
           "  rb ^= 1;\n"
           "  if ((threadIdx.x & 63) == 0) r[threadIdx.x >> 6] = v;\n"
           "  __syncthreads();\n"
           "  float s = r[0];\n"
           "#pragma unroll\n"
           "  for (int w = 1; w < COOP_WAVES; ++w) s += r[w];\n"
           "  return s;\n}\n"
           "template <class I> __device__ static void coop_merge(float& v, I& i, float ov, I oi) {\n"
           "  const bool take = ov > v || (ov == v && oi < i);\n"
           "  v = take ? ov : v; i = take ? oi : i;\n}\n"
           "template <class I> __device__ static void coop_wg_first_max(float& v, I& i, float* rv, I* ri, int& rb) {\n"
           "  coop_merge(v, i, coop_dpp_f<0xB1>(v), coop_dpp_i<0xB1>(i));\n"
           "  coop_merge(v, i, coop_dpp_f<0x4E>(v), coop_dpp_i<0x4E>(i));\n"
           "  coop_merge(v, i, coop_dpp_f<0x141>(v), coop_dpp_i<0x141>(i));\n"
           "  coop_merge(v, i, coop_dpp_f<0x140>(v), coop_dpp_i<0x140>(i));\n"
           "  float wv = coop_lane_f(v, 0);\n"
           "  I wi = coop_lane_i(i, 0);\n"
           "  for (int l = 16; l < 64; l += 16) coop_merge(wv, wi, coop_lane_f(v, l), coop_lane_i(i, l));\n"
           "  float* r = rv + rb * COOP_WAVES;\n"
           "  I* q = ri + rb * COOP_WAVES;\n"
           "  rb ^= 1;\n"
           "  if ((threadIdx.x & 63) == 0) { r[threadIdx.x >> 6] = wv; q[threadIdx.x >> 6] = wi; }\n"
           "  __syncthreads();\n"
           "  v = r[0]; i = q[0];\n"
           "#pragma unroll\n"
           "  for (int w = 1; w < COOP_WAVES; ++w) coop_merge(v, i, r[w], q[w]);\n}\n\n";
    }
    body();
    wrapper(plan_out, rows, cols);
    return o.str();
  }
};

// The backends' shared contract (crates/sile-backend/src/verify.rs:21-43): no
// switch terminators, no calls to tile helpers.  Like the Metal target
// (crates/sile-backend/src/metal/codegen.rs), other calls are rejected too: the
// generated HIP source defines no helpers to call.  Thread ids are allowed and
// are 0, as in the C target (one program per thread).
void verify(const Function& fn) {
  for (const Block& b : fn.blocks) {
    if (b.term.kind == "switch")
      throw ParseError{"HIP backend emit does not support switch terminators (block `" +
                       b.name + "`)"};
    for (const Inst& in : b.insts) {
      if (in.op != "call") continue;
      if (starts_with(in.sub, "tile_"))
        throw ParseError{"HIP backend emit does not allow tile helper calls in LLVM IR, got `" +
                         in.sub + "` (block `" + b.name + "`)"};
      throw ParseError{"HIP backend emit does not support LLVM IR call instructions, got `" +
                       in.sub + "` (block `" + b.name + "`)"};
    }
  }
}

// A block entered by one edge only takes its arguments from that edge: its
// parameters are replaced by the values the edge passes.  The reference's
// loops pass the header's values on to the body block and the exit block
// (crates/sile-tile-ir/src/passes/lowering/core/emit/tile_loops/*.rs,
// tile_compute/reduce.rs), so after this the body of a loop uses the header's
// values directly.  Safe for every use: the edge's source dominates the block
// (it is its only way in), and a use of a block parameter lies in blocks the
// block dominates, which control reaches from the source only through the
// block.  The entry block and a block whose only edge is its own back edge
// (unreachable) are left alone.
void forward_block_args(Function& fn) {
  for (bool changed = true; changed;) {
    changed = false;
    std::map<std::string, int> preds;
    for (const Block& b : fn.blocks) {
      if (b.term.kind == "br") ++preds[b.term.t];
      if (b.term.kind == "condbr") {
        ++preds[b.term.t];
        ++preds[b.term.f];
      }
      if (b.term.kind == "switch") return;  // rejected by verify()
    }
    for (size_t bi = 1; bi < fn.blocks.size() && !changed; ++bi) {
      Block& b = fn.blocks[bi];
      if (b.params.empty() || preds[b.name] != 1) continue;
      std::vector<Operand>* args = nullptr;
      for (Block& src : fn.blocks) {
        if (src.term.kind == "br" && src.term.t == b.name) args = &src.term.targs;
        if (src.term.kind == "condbr" && src.term.t == b.name) args = &src.term.targs;
        if (src.term.kind == "condbr" && src.term.f == b.name) args = &src.term.fargs;
        if (args && &src == &b) args = nullptr;
        if (args) break;
      }
      if (!args || args->size() != b.params.size()) continue;
      std::map<std::string, Operand> sub;
      for (size_t k = 0; k < b.params.size(); ++k) sub[b.params[k].first] = (*args)[k];
      auto fix = [&](Operand& o) {
        if (!o.is_value) return;
        auto it = sub.find(o.name);
        if (it != sub.end()) o = it->second;
      };
      args->clear();
      b.params.clear();
      for (Block& u : fn.blocks) {
        for (Inst& in : u.insts)
          for (Operand& a : in.args) fix(a);
        fix(u.term.cond);
        for (Operand& a : u.term.targs) fix(a);
        for (Operand& a : u.term.fargs) fix(a);
      }
      changed = true;
    }
  }
}

// A block parameter that every edge into the block passes the same value
// (or itself, around a loop) is that value: it is replaced by it and dropped
// from the edges.  The value dominates the block (it reaches the block on
// every edge), so it is available wherever the parameter was.  The
// reference's MMA loop carries the row and column through its k loop this way
// (tile_compute/mma.rs:58-75, 190-192).
bool drop_trivial_params(Function& fn) {
  bool any = false;
  for (size_t bi = 1; bi < fn.blocks.size(); ++bi) {
    Block& b = fn.blocks[bi];
    for (size_t k = 0; k < b.params.size();) {
      const std::string p = b.params[k].first;
      std::vector<std::vector<Operand>*> edges;
      for (Block& src : fn.blocks) {
        if (src.term.kind == "br" && src.term.t == b.name) edges.push_back(&src.term.targs);
        if (src.term.kind == "condbr" && src.term.t == b.name) edges.push_back(&src.term.targs);
        if (src.term.kind == "condbr" && src.term.f == b.name) edges.push_back(&src.term.fargs);
      }
      const Operand* same = nullptr;
      bool trivial = !edges.empty();
      for (auto* e : edges) {
        if (e->size() != b.params.size()) {
          trivial = false;
          break;
        }
        const Operand& a = (*e)[k];
        if (a.is_value && a.name == p) continue;
        if (!same) {
          same = &a;
        } else if (same->is_value != a.is_value || same->name != a.name || same->ck != a.ck) {
          trivial = false;
          break;
        }
      }
      if (!trivial || !same) {
        ++k;
        continue;
      }
      const Operand v = *same;
      for (auto* e : edges) e->erase(e->begin() + (long)k);
      b.params.erase(b.params.begin() + (long)k);
      for (Block& u : fn.blocks) {
        auto fix = [&](Operand& o) {
          if (o.is_value && o.name == p) o = v;
        };
        for (Inst& in : u.insts)
          for (Operand& a : in.args) fix(a);
        fix(u.term.cond);
        for (Operand& a : u.term.targs) fix(a);
        for (Operand& a : u.term.fargs) fix(a);
      }
      any = true;
    }
  }
  return any;
}

// The printed form gives a pointer block parameter no pointee (`ptr
// addrspace(5)`), but the reference's lowering passes tiles between blocks
// that way (a tile carried through a loop).  A gep on the parameter names
// the tile type; the parameter takes it, so it is declared as the tile
// pointer the backends' C form uses (`float (*)[C]`) and its geps index the
// tile's dimensions.
// A parameter also takes the pointee of a value an edge passes it (the
// alloca a loop starts from).
void type_pointer_params(Function& fn, std::map<std::string, Type>& types) {
  std::map<std::string, Type> pointee;
  for (const Block& b : fn.blocks)
    for (const Inst& in : b.insts)
      if (in.op == "gep" && in.args[0].is_value && in.aux.k == TK::Arr)
        pointee.emplace(in.args[0].name, in.aux);
  for (bool changed = true; changed;) {
    changed = false;
    for (Block& b : fn.blocks)
      for (size_t k = 0; k < b.params.size(); ++k) {
        auto& p = b.params[k];
        if (p.second.k != TK::Ptr || p.second.elem) continue;
        std::shared_ptr<Type> e;
        auto it = pointee.find(p.first);
        if (it != pointee.end()) e = std::make_shared<Type>(it->second);
        for (const Block& src : fn.blocks) {
          auto from = [&](const std::string& t, const std::vector<Operand>& args) {
            if (e || t != b.name || k >= args.size() || !args[k].is_value) return;
            auto ti = types.find(args[k].name);
            if (ti != types.end() && ti->second.k == TK::Ptr && ti->second.elem) e = ti->second.elem;
          };
          if (src.term.kind == "br") from(src.term.t, src.term.targs);
          if (src.term.kind == "condbr") {
            from(src.term.t, src.term.targs);
            from(src.term.f, src.term.fargs);
          }
        }
        if (!e) continue;
        p.second.elem = e;
        types[p.first] = p.second;
        changed = true;
      }
  }
}

// parse + emit; returns a status and fills `src` / the last error
int to_hip(const char* text, int64_t plan_out, int64_t rows, int64_t cols, std::string& src,
           std::string& name) {
  if (!text) return fail(SILE_ERR_SHAPE, "LLIR text is NULL");
  if (plan_out >= 0 && (rows <= 0 || cols <= 0))
    return fail(SILE_ERR_SHAPE, "tile plan needs positive rows and cols");
  try {
    Parser p;
    p.parse(std::string(text));
    verify(p.fn);
    do forward_block_args(p.fn);
    while (drop_trivial_params(p.fn));
    type_pointer_params(p.fn, p.types);
    const CoopPlan coop = plan_coop(p.fn, p.types);
    Emitter e{p.fn, p.types, coop, {}};
    src = e.emit(plan_out, rows, cols);
    name = "sile_kernel_" + p.fn.name;
  } catch (const ParseError& e) {
    return fail(SILE_ERR_COMPILE, "%s", e.msg.c_str());
  } catch (const std::exception& e) {
    return fail(SILE_ERR_COMPILE, "LLIR: %s", e.what());
  }
  return ok();
}

}  // namespace

extern "C" {

int sile_hip_llir_to_hip(const char* llir_text, int64_t plan_output_param, int64_t plan_rows,
                         int64_t plan_cols, char* out, size_t out_capacity, size_t* out_len) {
  std::string src, name;
  int rc = to_hip(llir_text, plan_output_param, plan_rows, plan_cols, src, name);
  if (rc != SILE_OK) return rc;
  if (out_len) *out_len = src.size();
  if (out && out_capacity) {
    const size_t n = std::min(out_capacity - 1, src.size());
    memcpy(out, src.data(), n);
    out[n] = 0;
    if (n < src.size()) return fail(SILE_ERR_SHAPE, "output buffer too small (%zu bytes needed)", src.size() + 1);
  }
  return ok();
}

int sile_hip_llir_compile(const char* llir_text, int64_t plan_output_param, int64_t plan_rows,
                          int64_t plan_cols, void** code_out, size_t* code_bytes,
                          char* kernel_name, size_t name_capacity) {
  std::string src, name;
  int rc = to_hip(llir_text, plan_output_param, plan_rows, plan_cols, src, name);
  if (rc != SILE_OK) return rc;
  if (!code_out || !code_bytes) return fail(SILE_ERR_SHAPE, "NULL output pointer");
  hiprtcProgram prog;
  if (hiprtcCreateProgram(&prog, src.c_str(), "sile_llir.hip", 0, nullptr, nullptr) !=
      HIPRTC_SUCCESS)
    return fail(SILE_ERR_COMPILE, "hiprtcCreateProgram failed");
  // -ffp-contract=off: the CPU backend's C is compiled without contraction
  // (crates/sile-backend/src/cpu/mod.rs:83, no -march, no FMA)
  const char* opts[] = {"--offload-arch=gfx950", "-O3",     "-ffp-contract=off", "-Xclang",
                        "-target-feature",       "-Xclang", "-packed-fp32-ops"};
  const hiprtcResult r = hiprtcCompileProgram(prog, 7, opts);
  if (r != HIPRTC_SUCCESS) {
    size_t ls = 0;
    hiprtcGetProgramLogSize(prog, &ls);
    std::string log(ls + 1, '\0');
    hiprtcGetProgramLog(prog, &log[0]);
    hiprtcDestroyProgram(&prog);
    return fail(SILE_ERR_COMPILE, "hiprtc: %s\n%s\n--- generated source ---\n%s",
                hiprtcGetErrorString(r), log.c_str(), src.c_str());
  }
  size_t cs = 0;
  hiprtcGetCodeSize(prog, &cs);
  void* code = malloc(cs);
  if (!code) {
    hiprtcDestroyProgram(&prog);
    return fail(SILE_ERR_RUNTIME, "out of host memory");
  }
  hiprtcGetCode(prog, static_cast<char*>(code));
  hiprtcDestroyProgram(&prog);
  *code_out = code;
  *code_bytes = cs;
  if (kernel_name && name_capacity) {
    const size_t n = std::min(name_capacity - 1, name.size());
    memcpy(kernel_name, name.data(), n);
    kernel_name[n] = 0;
  }
  return ok();
}

void sile_hip_llir_free_code(void* code) { free(code); }

}  // extern "C"
