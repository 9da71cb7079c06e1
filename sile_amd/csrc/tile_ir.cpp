// Pattern router from sile's Tile IR to the hand-written gfx950 kernels.
//
// Input: a kernel in the printed Tile IR form of the reference
// (crates/sile-tile-ir/src/print.rs:5-354 `format_tile_ir`, data model
// crates/sile-tile-ir/src/ir.rs:1-484), as it stands after the default Tile IR
// pass pipeline (crates/sile-tile-ir/src/passes/mod.rs:31-42), or before it:
// pointwise ops are matched through their `map` fusion and unfused alike.
//
// The router generalises the reference's canonical-matmul detector
// (crates/sile-tile-ir/src/passes/lowering/canonical_matmul.rs:446-666) to the
// other tile patterns on the hot path:
//   * canonical matmul      -> the exact-order f32 tile kernel
//                              (bit-identical to the CPU backend);
//   * the softmax chain     -> the row softmax kernel when a tile spans the
//     (crates/sile/examples/softmax.rs:3-16)      whole row, else the tile kernel;
//   * load + row reduce + store -> the row reduce kernel;
//   * load + reduce + extract + atomic add -> the parallel-reduce kernel
//     (crates/sile/examples/parallel_reduce.rs:3-9);
//   * the online-softmax attention loop the DSL can write (K given
//     transposed, no mask) -> the fp32 attention kernel;
//   * the matvec loop (crates/sile/examples/mlp.rs:26-44) -> the matvec
//     kernel (bit-identical to the CPU backend).
// A route is taken only where the routed kernel writes exactly the elements,
// in exactly the tile decomposition, that the CPU backend's launch wrapper
// writes for the same shapes and grid (crates/sile-backend/src/cpu/codegen.rs:409-555).
// Everything else gets SILE_ROUTE_NONE with the reason, and the caller lowers
// the kernel to LLIR and uses the generic code generation.
#include <algorithm>
#include <cctype>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <map>
#include <memory>
#include <sstream>
#include <string>
#include <vector>

#include "runtime_internal.h"

using sile_rt::fail;
using sile_rt::ok;

namespace {

// ---------------------------------------------------------------------------
// data model (crates/sile-tile-ir/src/ir.rs)
// ---------------------------------------------------------------------------
struct Ty {
  enum K { I64, F32, Shape, Tile, Buffer, Void } k = Void;
  int64_t rows = 0, cols = 0;  // Tile
  int rank = 0;                // Shape
};

struct Expr;
using ExprP = std::shared_ptr<Expr>;

// TileMapExpr (ir.rs:76-126)
struct Expr {
  enum K { Value, Load, Splat, Cmp, Add, Sub, Mul, Div, Neg, Exp, Select, Bcast } k = Value;
  uint32_t v = 0;                         // Value
  uint32_t buf = 0, row = 0, col = 0;     // Load
  int64_t rows = 0, cols = 0, stride = 0; // Load shape / stride dim; Bcast source shape
  double f = 0;                           // Splat
  std::string cmp;                        // Cmp
  std::vector<ExprP> a;                   // operands
};

// TileIrOp (ir.rs:128-262)
enum class Op {
  LoadTko, StoreTko, AtomicAdd, Splat, AddF, SubF, MulF, DivF, NegF, Exp, Mma, Reduce,
  Broadcast, Map, Extract, IBin, ICmp, ConstI64, ConstF64, ShapeDim
};

struct Inst {
  uint32_t result = 0;
  Op op = Op::ConstI64;
  std::vector<uint32_t> uses;            // value operands in printed order
  int64_t rows = 0, cols = 0;            // tko / broadcast / map shape; reduce input shape
  int64_t stride = 0;                    // tko stride dim
  int64_t m = 0, n = 0, k = 0;           // mma
  int64_t axis = 0;                      // reduce
  bool is_max = false;                   // reduce combiner
  int64_t ival = 0;                      // ConstI64, ShapeDim dim
  double fval = 0;                       // Splat, ConstF64
  std::string sub;                       // IBin / ICmp mnemonic
  ExprP expr;                            // Map
  Ty ty;
};

struct Term {
  enum K { Br, CondBr, Ret } k = Ret;
  uint32_t cond = 0, t = 0, f = 0;
  std::vector<uint32_t> targs, fargs;
};

struct Block {
  uint32_t id = 0;
  std::vector<uint32_t> params;
  std::vector<Inst> insts;
  Term term;
};

// TileIrParam / TileIrParamKind (ir.rs:139-151)
struct Param {
  uint32_t value = 0;
  std::string name;
  enum K { Buffer, Launch, Shape } kind = Buffer;
  int rank = 0;         // Buffer
  int64_t dim = 0;      // Launch
  uint32_t source = 0;  // Shape
};

struct Function {
  std::string name;
  std::vector<Param> params;
  std::vector<Block> blocks;
  uint32_t entry = 0;
  bool has_entry = false;
  std::map<uint32_t, Ty> types;

  const Block* block(uint32_t id) const {
    for (const Block& b : blocks)
      if (b.id == id) return &b;
    return nullptr;
  }
  const Param* param(uint32_t v) const {
    for (const Param& p : params)
      if (p.value == v) return &p;
    return nullptr;
  }
};

struct ParseError {
  std::string msg;
};

// ---------------------------------------------------------------------------
// parser of the printed form (print.rs:5-354)
// ---------------------------------------------------------------------------
class Cursor {
 public:
  Cursor(const std::string& s, int line) : s_(s), line_(line) {}

  [[noreturn]] void error(const std::string& what) const {
    throw ParseError{"Tile IR line " + std::to_string(line_) + ": " + what + " at '" +
                     s_.substr(std::min(p_, s_.size())) + "'"};
  }
  void ws() {
    while (p_ < s_.size() && isspace((unsigned char)s_[p_])) ++p_;
  }
  bool done() {
    ws();
    return p_ >= s_.size();
  }
  bool peek(const char* t) {
    ws();
    return s_.compare(p_, strlen(t), t) == 0;
  }
  bool eat(const char* t) {
    if (!peek(t)) return false;
    p_ += strlen(t);
    return true;
  }
  void expect(const char* t) {
    if (!eat(t)) error(std::string("expected '") + t + "'");
  }
  uint32_t value() {
    expect("%");
    return (uint32_t)unsigned_int();
  }
  uint32_t block_ref() {
    expect("^bb");
    return (uint32_t)unsigned_int();
  }
  uint64_t unsigned_int() {
    ws();
    size_t q = p_;
    while (q < s_.size() && isdigit((unsigned char)s_[q])) ++q;
    if (q == p_) error("expected an unsigned integer");
    const uint64_t v = strtoull(s_.c_str() + p_, nullptr, 10);
    p_ = q;
    return v;
  }
  int64_t integer() {
    ws();
    size_t q = p_;
    if (q < s_.size() && s_[q] == '-') ++q;
    const size_t digits = q;
    while (q < s_.size() && isdigit((unsigned char)s_[q])) ++q;
    if (q == digits) error("expected an integer");
    const int64_t v = strtoll(s_.c_str() + p_, nullptr, 10);
    p_ = q;
    return v;
  }
  // Rust's f64 Display: digits with an optional fraction, `inf`, `NaN`.
  double number() {
    ws();
    const char* b = s_.c_str() + p_;
    char* e = nullptr;
    const double v = strtod(b, &e);
    if (e == b) error("expected a number");
    p_ += (size_t)(e - b);
    return v;
  }
  std::string word() {
    ws();
    size_t q = p_;
    while (q < s_.size() && (isalnum((unsigned char)s_[q]) || s_[q] == '_' || s_[q] == '.')) ++q;
    if (q == p_) error("expected a word");
    std::string w = s_.substr(p_, q - p_);
    p_ = q;
    return w;
  }
  std::string quoted() {
    expect("\"");
    const size_t q = s_.find('"', p_);
    if (q == std::string::npos) error("unterminated string");
    std::string w = s_.substr(p_, q - p_);
    p_ = q + 1;
    return w;
  }
  // `[R, C]`
  void pair(int64_t& a, int64_t& b) {
    expect("[");
    a = integer();
    expect(",");
    b = integer();
    expect("]");
  }
  // `[%r, %c]`
  void coords(uint32_t& r, uint32_t& c) {
    expect("[");
    r = value();
    expect(",");
    c = value();
    expect("]");
  }

 private:
  const std::string& s_;
  size_t p_ = 0;
  int line_;
};

Ty parse_type(Cursor& c) {
  Ty t;
  if (c.eat("none")) return t;
  if (c.eat("shape_desc<")) {
    t.k = Ty::Shape;
    t.rank = (int)c.integer();
    c.expect(">");
    return t;
  }
  c.expect("tile<");
  if (c.eat("i64>")) {
    t.k = Ty::I64;
  } else if (c.eat("f32>")) {
    t.k = Ty::F32;
  } else if (c.eat("ptr<f32>>")) {
    t.k = Ty::Buffer;
  } else {
    // tile<RxCxf32>
    t.k = Ty::Tile;
    t.rows = c.integer();
    c.expect("x");
    t.cols = c.integer();
    c.expect("xf32>");
  }
  return t;
}

ExprP parse_expr(Cursor& c, int depth = 0) {
  if (depth > 256) c.error("map expression nested too deeply");
  auto e = std::make_shared<Expr>();
  if (c.peek("%")) {
    e->k = Expr::Value;
    e->v = c.value();
    return e;
  }
  const std::string w = c.word();
  c.expect("(");
  auto sub = [&]() { e->a.push_back(parse_expr(c, depth + 1)); };
  if (w == "load_ptr_tko") {
    e->k = Expr::Load;
    e->buf = c.value();
    c.expect(",");
    c.coords(e->row, e->col);
    c.expect(",");
    c.expect("shape=");
    c.pair(e->rows, e->cols);
    c.expect(",");
    c.expect("stride_dim=");
    e->stride = c.integer();
  } else if (w == "constant") {
    e->k = Expr::Splat;
    e->f = c.number();
  } else if (w == "cmpf") {
    e->k = Expr::Cmp;
    e->cmp = c.quoted();
    c.expect(",");
    sub();
    c.expect(",");
    sub();
  } else if (w == "addf" || w == "subf" || w == "mulf" || w == "divf") {
    e->k = w == "addf" ? Expr::Add : w == "subf" ? Expr::Sub : w == "mulf" ? Expr::Mul : Expr::Div;
    sub();
    c.expect(",");
    sub();
  } else if (w == "negf" || w == "exp") {
    e->k = w == "negf" ? Expr::Neg : Expr::Exp;
    sub();
  } else if (w == "select") {
    e->k = Expr::Select;
    sub();
    c.expect(",");
    sub();
    c.expect(",");
    sub();
  } else if (w == "broadcast") {
    e->k = Expr::Bcast;
    sub();
    c.expect(",");
    c.expect("src_shape=");
    c.pair(e->rows, e->cols);
  } else {
    c.error("unknown map expression '" + w + "'");
  }
  c.expect(")");
  return e;
}

void expr_uses(const Expr& e, std::vector<uint32_t>& out) {
  if (e.k == Expr::Value) out.push_back(e.v);
  if (e.k == Expr::Load) {
    out.push_back(e.buf);
    out.push_back(e.row);
    out.push_back(e.col);
  }
  for (const ExprP& s : e.a) expr_uses(*s, out);
}

// `%N = <op> : <type>` (print.rs:84-185)
Inst parse_inst(Cursor& c) {
  Inst in;
  in.result = c.value();
  c.expect("=");
  auto two = [&]() {
    in.uses.push_back(c.value());
    c.expect(",");
    in.uses.push_back(c.value());
  };
  const std::string w = c.word();
  if (w == "load_ptr_tko" || w == "store_ptr_tko") {
    const bool store = w == "store_ptr_tko";
    in.op = store ? Op::StoreTko : Op::LoadTko;
    in.uses.push_back(c.value());  // buffer
    c.expect(",");
    if (store) {
      in.uses.push_back(c.value());  // stored value
      c.expect(",");
    }
    uint32_t r, col;
    c.coords(r, col);
    in.uses.push_back(r);
    in.uses.push_back(col);
    c.expect("{");
    c.expect("shape");
    c.expect("=");
    c.pair(in.rows, in.cols);
    c.expect(",");
    c.expect("stride_dim");
    c.expect("=");
    in.stride = c.integer();
    c.expect("}");
  } else if (w == "sile.atomic_add") {
    in.op = Op::AtomicAdd;
    two();  // buffer, value
    c.expect(",");
    uint32_t r, col;
    c.coords(r, col);
    in.uses.push_back(r);
    in.uses.push_back(col);
    c.expect("{");
    c.expect("stride_dim");
    c.expect("=");
    in.stride = c.integer();
    c.expect("}");
  } else if (w == "constant") {
    c.expect("<");
    const std::string t = c.word();
    c.expect(":");
    if (t == "f32") {
      in.op = Op::Splat;
      in.fval = c.number();
    } else if (t == "i64") {
      in.op = Op::ConstI64;
      in.ival = c.integer();
    } else if (t == "f64") {
      in.op = Op::ConstF64;
      in.fval = c.number();
    } else {
      c.error("unknown constant type '" + t + "'");
    }
    c.expect(">");
  } else if (w == "addf" || w == "subf" || w == "mulf" || w == "divf") {
    in.op = w == "addf" ? Op::AddF : w == "subf" ? Op::SubF : w == "mulf" ? Op::MulF : Op::DivF;
    two();
  } else if (w == "negf" || w == "exp") {
    in.op = w == "negf" ? Op::NegF : Op::Exp;
    in.uses.push_back(c.value());
  } else if (w == "mmaf") {
    in.op = Op::Mma;
    two();
    c.expect(",");
    in.uses.push_back(c.value());
    c.expect("{");
    c.expect("m");
    c.expect("=");
    in.m = c.integer();
    c.expect(",");
    c.expect("n");
    c.expect("=");
    in.n = c.integer();
    c.expect(",");
    c.expect("k");
    c.expect("=");
    in.k = c.integer();
    c.expect("}");
  } else if (w == "reduce") {
    in.op = Op::Reduce;
    in.uses.push_back(c.value());
    c.expect("{");
    c.expect("axis");
    c.expect("=");
    in.axis = c.integer();
    c.expect(",");
    c.expect("combiner");
    c.expect("=");
    const std::string comb = c.quoted();
    if (comb != "sum" && comb != "max") c.error("unknown combiner '" + comb + "'");
    in.is_max = comb == "max";
    c.expect(",");
    c.expect("input_shape");
    c.expect("=");
    c.pair(in.rows, in.cols);
    c.expect("}");
  } else if (w == "broadcast") {
    in.op = Op::Broadcast;
    in.uses.push_back(c.value());
    c.expect("{");
    c.expect("shape");
    c.expect("=");
    c.pair(in.rows, in.cols);
    c.expect("}");
  } else if (w == "map") {
    in.op = Op::Map;
    in.expr = parse_expr(c);
    expr_uses(*in.expr, in.uses);
    c.expect("{");
    c.expect("shape");
    c.expect("=");
    c.pair(in.rows, in.cols);
    c.expect("}");
  } else if (w == "extract") {
    in.op = Op::Extract;
    in.uses.push_back(c.value());
    uint32_t r, col;
    c.coords(r, col);
    in.uses.push_back(r);
    in.uses.push_back(col);
  } else if (w == "addi" || w == "subi" || w == "muli" || w == "divi") {
    in.op = Op::IBin;
    in.sub = w;
    two();
  } else if (w == "cmpi") {
    in.op = Op::ICmp;
    in.sub = c.quoted();
    two();
  } else if (w == "sile.shape_dim") {
    in.op = Op::ShapeDim;
    in.uses.push_back(c.value());
    c.expect("{");
    c.expect("dim");
    c.expect("=");
    in.ival = c.integer();
    c.expect("}");
  } else {
    c.error("unknown op '" + w + "'");
  }
  c.expect(":");
  in.ty = parse_type(c);
  if (!c.done()) c.error("trailing text");
  return in;
}

std::vector<uint32_t> parse_args(Cursor& c) {
  std::vector<uint32_t> out;
  if (!c.eat("(")) return out;
  if (c.eat(")")) return out;
  do {
    out.push_back(c.value());
  } while (c.eat(","));
  c.expect(")");
  return out;
}

Term parse_term(Cursor& c) {
  Term t;
  if (c.eat("return")) {
    t.k = Term::Ret;
  } else if (c.eat("cf.cond_br")) {
    t.k = Term::CondBr;
    t.cond = c.value();
    c.expect(",");
    t.t = c.block_ref();
    t.targs = parse_args(c);
    c.expect(",");
    t.f = c.block_ref();
    t.fargs = parse_args(c);
  } else if (c.eat("cf.br")) {
    t.k = Term::Br;
    t.t = c.block_ref();
    t.targs = parse_args(c);
  } else {
    c.error("expected a terminator");
  }
  if (!c.done()) c.error("trailing text");
  return t;
}

// `%N {sym_name = "...", ...} : <type>[,]` (print.rs:6-20, 327-346)
Param parse_param(Cursor& c, Function& fn) {
  Param p;
  p.value = c.value();
  c.expect("{");
  c.expect("sym_name");
  c.expect("=");
  p.name = c.quoted();
  c.expect(",");
  if (c.eat("rank")) {
    c.expect("=");
    p.kind = Param::Buffer;
    p.rank = (int)c.integer();
  } else {
    c.expect("kind");
    c.expect("=");
    const std::string kind = c.quoted();
    c.expect(",");
    if (kind == "launch.index") {
      p.kind = Param::Launch;
      c.expect("dim");
      c.expect("=");
      p.dim = c.integer();
    } else if (kind == "shape.desc") {
      p.kind = Param::Shape;
      c.expect("source");
      c.expect("=");
      p.source = c.value();
    } else {
      c.error("unknown parameter kind '" + kind + "'");
    }
  }
  c.expect("}");
  c.expect(":");
  const Ty t = parse_type(c);
  c.eat(",");
  if (!c.done()) c.error("trailing text");
  const Ty::K want = p.kind == Param::Buffer ? Ty::Buffer
                     : p.kind == Param::Launch ? Ty::I64
                                               : Ty::Shape;
  if (t.k != want) c.error("parameter type does not match its kind");
  fn.types[p.value] = t;
  return p;
}

Function parse(const std::string& text) {
  Function fn;
  std::istringstream in(text);
  std::string raw;
  int line = 0;
  enum { kModule, kEntry, kParams, kBody, kClosed, kDone } state = kModule;
  Block* cur = nullptr;
  while (std::getline(in, raw)) {
    ++line;
    Cursor c(raw, line);
    if (c.done()) continue;
    switch (state) {
      case kModule:
        c.expect("module");
        c.expect("{");
        state = kEntry;
        break;
      case kEntry:
        c.expect("entry");
        c.expect("@");
        fn.name = c.word();
        c.expect("(");
        state = kParams;
        break;
      case kParams:
        if (c.eat(")")) {
          c.expect("{");
          state = kBody;
          break;
        }
        fn.params.push_back(parse_param(c, fn));
        break;
      case kBody:
        if (c.peek("^bb")) {
          if (cur) c.error("block header before the previous block's terminator");
          Block b;
          b.id = c.block_ref();
          if (c.eat("(")) {
            do {
              const uint32_t v = c.value();
              c.expect(":");
              fn.types[v] = parse_type(c);
              b.params.push_back(v);
            } while (c.eat(","));
            c.expect(")");
          }
          c.expect(":");
          if (c.eat("//")) {
            c.expect("entry");
            if (fn.has_entry) c.error("two entry blocks");
            fn.entry = b.id;
            fn.has_entry = true;
          }
          if (!c.done()) c.error("trailing text");
          if (fn.block(b.id)) c.error("block defined twice");
          fn.blocks.push_back(std::move(b));
          cur = &fn.blocks.back();
          break;
        }
        if (c.peek("}")) {
          c.expect("}");
          if (cur) c.error("block without a terminator");
          state = kClosed;
          break;
        }
        if (!cur) c.error("instruction outside a block");
        if (c.peek("%")) {
          Inst i = parse_inst(c);
          fn.types[i.result] = i.ty;
          cur->insts.push_back(std::move(i));
        } else {
          cur->term = parse_term(c);
          cur = nullptr;  // a terminator closes the block
        }
        break;
      case kClosed:
        c.expect("}");
        state = kDone;
        break;
      case kDone:
        c.error("text after the module");
    }
  }
  if (state != kDone) throw ParseError{"Tile IR: incomplete module"};
  if (!fn.has_entry) throw ParseError{"Tile IR: no entry block"};
  for (const Block& b : fn.blocks) {
    const std::vector<uint32_t>* lists[2] = {&b.term.targs, &b.term.fargs};
    const uint32_t targets[2] = {b.term.t, b.term.f};
    const int n = b.term.k == Term::Ret ? 0 : b.term.k == Term::Br ? 1 : 2;
    for (int i = 0; i < n; ++i) {
      const Block* t = fn.block(targets[i]);
      if (!t) throw ParseError{"Tile IR: branch to unknown block bb" + std::to_string(targets[i])};
      if (t->params.size() != lists[i]->size())
        throw ParseError{"Tile IR: branch to bb" + std::to_string(targets[i]) + " passes " +
                         std::to_string(lists[i]->size()) + " values for " +
                         std::to_string(t->params.size()) + " parameters"};
    }
  }
  return fn;
}

// ---------------------------------------------------------------------------
// pattern matching
// ---------------------------------------------------------------------------
struct NoRoute {
  std::string why;
};
[[noreturn]] void no_route(const std::string& why) { throw NoRoute{why}; }

const Inst* find_inst(const Block& b, uint32_t v) {
  for (const Inst& i : b.insts)
    if (i.result == v) return &i;
  return nullptr;
}

// Launch-index dimension of `v`, or -1.
int64_t launch_dim(const Function& fn, uint32_t v) {
  const Param* p = fn.param(v);
  return p && p->kind == Param::Launch ? p->dim : -1;
}

bool is_const(const Block& b, uint32_t v, int64_t want) {
  const Inst* i = find_inst(b, v);
  return i && i->op == Op::ConstI64 && i->ival == want;
}

// Index of buffer parameter `v` among the kernel's buffers (= its position in
// the `buffers` array and in the shape concatenation), or -1.
int buffer_index(const Function& fn, uint32_t v) {
  int idx = 0;
  for (const Param& p : fn.params) {
    if (p.kind != Param::Buffer) continue;
    if (p.value == v) return idx;
    ++idx;
  }
  return -1;
}

// Expands value `v` of block `b` into a map expression, following the
// pointwise ops the fusion pass folds into maps
// (crates/sile-tile-ir/src/passes/pointwise_fusion.rs:47-58), splats, and maps
// themselves; any other value stays a leaf.  Fused and unfused forms of the
// same computation give the same tree.
ExprP expand(const Block& b, uint32_t v, int depth = 0);

// Types of every value of the function being matched (block parameters
// included), for the source shape of a broadcast of a block parameter; set by
// detect() for the duration of one detection on this thread.
thread_local const std::map<uint32_t, Ty>* t_types = nullptr;

ExprP expand_expr(const Block& b, const ExprP& e, int depth) {
  if (depth > 64) no_route("pointwise chain too deep");
  if (e->k == Expr::Value) return expand(b, e->v, depth + 1);
  auto out = std::make_shared<Expr>(*e);
  for (ExprP& s : out->a) s = expand_expr(b, s, depth + 1);
  return out;
}

ExprP leaf(uint32_t v) {
  auto e = std::make_shared<Expr>();
  e->k = Expr::Value;
  e->v = v;
  return e;
}

ExprP expand(const Block& b, uint32_t v, int depth) {
  if (depth > 64) no_route("pointwise chain too deep");
  const Inst* i = find_inst(b, v);
  if (!i) return leaf(v);
  auto node = [&](Expr::K k, std::initializer_list<uint32_t> ops) {
    auto e = std::make_shared<Expr>();
    e->k = k;
    for (uint32_t o : ops) e->a.push_back(expand(b, o, depth + 1));
    return e;
  };
  switch (i->op) {
    case Op::Map:
      return expand_expr(b, i->expr, depth + 1);
    case Op::AddF: return node(Expr::Add, {i->uses[0], i->uses[1]});
    case Op::SubF: return node(Expr::Sub, {i->uses[0], i->uses[1]});
    case Op::MulF: return node(Expr::Mul, {i->uses[0], i->uses[1]});
    case Op::DivF: return node(Expr::Div, {i->uses[0], i->uses[1]});
    case Op::NegF: return node(Expr::Neg, {i->uses[0]});
    case Op::Exp: return node(Expr::Exp, {i->uses[0]});
    case Op::Splat: {
      // a splat reads as its constant, whether the fusion folded it into the
      // map (single use) or left it standing (several uses)
      auto e = std::make_shared<Expr>();
      e->k = Expr::Splat;
      e->f = i->fval;
      return e;
    }
    case Op::Broadcast: {
      auto e = node(Expr::Bcast, {i->uses[0]});
      // the source shape is the source value's tile type (pointwise_fusion.rs:150-163)
      const Inst* src = find_inst(b, i->uses[0]);
      Ty st;
      if (src) {
        st = src->ty;
      } else if (t_types) {
        auto it = t_types->find(i->uses[0]);
        if (it != t_types->end()) st = it->second;
      }
      if (st.k != Ty::Tile) no_route("broadcast of a value without a tile shape");
      e->rows = st.rows;
      e->cols = st.cols;
      return e;
    }
    default:
      return leaf(v);
  }
}

// `e` is Broadcast(Value(v)) of a [rows, 1] source; returns v.
bool bcast_col_of(const ExprP& e, int64_t rows, uint32_t& v) {
  if (e->k != Expr::Bcast || e->rows != rows || e->cols != 1) return false;
  if (e->a.size() != 1 || e->a[0]->k != Expr::Value) return false;
  v = e->a[0]->v;
  return true;
}

// Operand bound to one kernel buffer: its position in `buffers` and the
// offset / rank of its dims in `shapes`.
struct Operand {
  int index = -1;
  int rank = 0;
  int shape_offset = 0;
};

struct Match {
  int kind = SILE_ROUTE_NONE;
  int reduce_op = 0;
  Operand ops[4];  // inputs, then the output; a matmul's accumulator source fourth
  int nops = 0;
  int64_t tm = 0, tn = 0, tk = 0;
  bool out_rank1 = false;
  bool seed_from_tile = false;  // matmul: accumulator loaded from ops[3]
  double seed_value = 0.0;      // matmul: the accumulator's splat value otherwise
  float scale = 1.0f, m0 = 0.0f;  // attention: score scale, initial running max
};

Operand operand_of(const Function& fn, uint32_t v) {
  Operand o;
  int idx = 0, off = 0;
  for (const Param& p : fn.params) {
    if (p.kind != Param::Buffer) continue;
    if (p.value == v) {
      o.index = idx;
      o.rank = p.rank;
      o.shape_offset = off;
      return o;
    }
    ++idx;
    off += p.rank;
  }
  no_route("operand is not a buffer parameter");
}

// The canonical matmul, with the conditions of the reference's detector
// (canonical_matmul.rs:446-666) and the launch dimensions the exact-order tile
// kernel decodes: rows from launch index 0, columns from launch index 1.
Match match_matmul(const Function& fn) {
  const Block* entry = fn.block(fn.entry);
  if (entry->term.k != Term::Br || entry->term.targs.size() != 2)
    no_route("entry block does not jump into a loop with (k, acc)");
  const Inst* k_seed = find_inst(*entry, entry->term.targs[0]);
  const Inst* acc_seed = find_inst(*entry, entry->term.targs[1]);
  if (!k_seed || k_seed->op != Op::ConstI64 || k_seed->ival != 0)
    no_route("loop counter does not start at constant 0");
  // the accumulator's seed: a splat (0.0 for the reference's canonical matmul,
  // any value for the tile MMA lowering's LoopCarriedSplat,
  // crates/sile-tile-ir/src/passes/lowering/block.rs:294-377) or a tile loaded
  // before the loop (the MMA then starts every cell from it,
  // crates/sile-tile-ir/src/passes/lowering/tile_compute/mma.rs:213-229)
  int64_t tile_m = 0, tile_n = 0;
  const Inst* acc_load = nullptr;
  if (acc_seed && acc_seed->op == Op::Splat) {
    if (acc_seed->ty.k != Ty::Tile) no_route("accumulator is not a tile");
    tile_m = acc_seed->ty.rows;
    tile_n = acc_seed->ty.cols;
  } else if (acc_seed && acc_seed->op == Op::LoadTko && acc_seed->stride == 1) {
    acc_load = acc_seed;
    tile_m = acc_seed->rows;
    tile_n = acc_seed->cols;
  } else {
    no_route("accumulator is neither a splat nor a rank-2 tile load");
  }

  const Block* header = fn.block(entry->term.t);
  if (header->params.size() != 2) no_route("loop header does not carry (k, acc)");
  const uint32_t loop_k = header->params[0], loop_acc = header->params[1];
  const Term& ht = header->term;
  if (ht.k != Term::CondBr) no_route("loop header does not branch");
  if (ht.targs != std::vector<uint32_t>{loop_k, loop_acc} ||
      ht.fargs != std::vector<uint32_t>{loop_acc})
    no_route("loop header branch arguments are not (k, acc) / (acc)");
  const Inst* cmp = find_inst(*header, ht.cond);
  if (!cmp || cmp->op != Op::ICmp || cmp->sub != "lt" || cmp->uses[0] != loop_k)
    no_route("loop condition is not k < bound");
  // the bound shape(a)[1] / BK, computed in the loop header (the reference's
  // canonical form) or once before the loop (`let k_tiles = a.shape()[1] / BK`,
  // crates/sile/examples/mlp.rs:6-23)
  auto def = [&](uint32_t v) {
    const Inst* i = find_inst(*header, v);
    return i ? i : find_inst(*entry, v);
  };
  const Inst* ktiles = def(cmp->uses[1]);
  if (!ktiles || ktiles->op != Op::IBin || ktiles->sub != "divi")
    no_route("loop bound is not a division");
  const Inst* tile_k_inst = def(ktiles->uses[1]);
  if (!tile_k_inst || tile_k_inst->op != Op::ConstI64) no_route("loop bound divisor is not constant");
  const int64_t tile_k = tile_k_inst->ival;
  const Inst* sdim = def(ktiles->uses[0]);
  if (!sdim || sdim->op != Op::ShapeDim || sdim->ival != 1)
    no_route("loop bound is not shape(a)[1] / BK");
  const Param* sdesc = fn.param(sdim->uses[0]);
  if (!sdesc || sdesc->kind != Param::Shape) no_route("shape_dim of a non-descriptor");
  const uint32_t a_buf = sdesc->source;

  const Block* body = fn.block(ht.t);
  if (body->params.size() != 2) no_route("loop body does not take (k, acc)");
  const uint32_t body_k = body->params[0], body_acc = body->params[1];
  if (body->term.k != Term::Br || body->term.t != header->id || body->term.targs.size() != 2)
    no_route("loop body does not jump back with (k', acc')");
  const Inst* next_k = find_inst(*body, body->term.targs[0]);
  if (!next_k || next_k->op != Op::IBin || next_k->sub != "addi")
    no_route("loop step is not an addition");
  uint32_t one;
  if (next_k->uses[0] == body_k)
    one = next_k->uses[1];
  else if (next_k->uses[1] == body_k)
    one = next_k->uses[0];
  else
    no_route("loop step does not add to k");
  if (!is_const(*body, one, 1)) no_route("loop step is not 1");

  const Inst* mma = find_inst(*body, body->term.targs[1]);
  if (!mma || mma->op != Op::Mma) no_route("carried accumulator is not an mma result");
  if (mma->uses[2] != body_acc || mma->m != tile_m || mma->n != tile_n || mma->k != tile_k)
    no_route("mma tile sizes or accumulator do not match the loop");
  const Inst* la = find_inst(*body, mma->uses[0]);
  const Inst* lb = find_inst(*body, mma->uses[1]);
  if (!la || la->op != Op::LoadTko || la->stride != 1 || !lb || lb->op != Op::LoadTko ||
      lb->stride != 1)
    no_route("mma operands are not rank-2 tile loads");
  const uint32_t row_launch = la->uses[1], col_launch = lb->uses[2];
  if (la->uses[0] != a_buf || la->uses[2] != body_k || lb->uses[1] != body_k ||
      la->rows != tile_m || la->cols != tile_k || lb->rows != tile_k || lb->cols != tile_n)
    no_route("tile loads do not walk A[m, k] and B[k, n]");
  if (launch_dim(fn, row_launch) < 0 || launch_dim(fn, col_launch) < 0)
    no_route("tile row / column are not launch indices");

  const Block* exit = fn.block(ht.f);
  if (exit->params.size() != 1) no_route("loop exit does not take the accumulator");
  if (exit->insts.size() != 1) no_route("loop exit holds more than the store");
  const Inst& st = exit->insts[0];
  if (st.op != Op::StoreTko || st.stride != 1 || st.uses[1] != exit->params[0] ||
      st.uses[2] != row_launch || st.uses[3] != col_launch || st.rows != tile_m ||
      st.cols != tile_n || exit->term.k != Term::Ret)
    no_route("loop exit does not store the accumulator at the program's tile");
  // the tile kernel decodes pid as (launch 0, launch 1) = (row tile, column tile)
  if (launch_dim(fn, row_launch) != 0 || launch_dim(fn, col_launch) != 1)
    no_route("row / column tiles come from launch indices (" +
             std::to_string(launch_dim(fn, row_launch)) + ", " +
             std::to_string(launch_dim(fn, col_launch)) + "), not (0, 1)");

  if (acc_load && (acc_load->uses[1] != row_launch || acc_load->uses[2] != col_launch))
    no_route("accumulator tile is not loaded at the program's tile");

  Match m;
  m.kind = SILE_ROUTE_MATMUL;
  m.ops[0] = operand_of(fn, a_buf);
  m.ops[1] = operand_of(fn, lb->uses[0]);
  m.ops[2] = operand_of(fn, st.uses[0]);
  m.nops = 3;
  if (acc_load) {
    m.ops[3] = operand_of(fn, acc_load->uses[0]);
    m.nops = 4;
    m.seed_from_tile = true;
  } else {
    m.seed_value = acc_seed->fval;
  }
  for (int i = 0; i < m.nops; ++i)
    if (m.ops[i].rank != 2) no_route("matmul operand is not rank 2");
  m.tm = tile_m;
  m.tn = tile_n;
  m.tk = tile_k;
  return m;
}

// The single store (or atomic add) of a one-block kernel.
const Inst& single_side_effect(const Function& fn, const Block*& blk) {
  if (fn.blocks.size() != 1) no_route("more than one block");
  blk = &fn.blocks[0];
  if (blk->term.k != Term::Ret) no_route("block does not return");
  const Inst* found = nullptr;
  for (const Inst& i : blk->insts) {
    if (i.op != Op::StoreTko && i.op != Op::AtomicAdd) continue;
    if (found) no_route("more than one store");
    found = &i;
  }
  if (!found) no_route("no store");
  return *found;
}

// The softmax chain (crates/sile/examples/softmax.rs:3-16):
//   x = load X[pid0, pid1] [BM, BN]; m = reduce_max(x, 1);
//   e = exp(x - broadcast(m)); s = reduce_sum(e, 1); store Y[pid0, pid1] <- e / broadcast(s).
Match match_softmax(const Function& fn) {
  const Block* b;
  const Inst& st = single_side_effect(fn, b);
  if (st.op != Op::StoreTko) no_route("no tile store");
  const int64_t bm = st.rows, bn = st.cols;
  if (st.stride != 1) no_route("store is not rank 2");
  const ExprP y = expand(*b, st.uses[1]);
  uint32_t s_val;
  if (y->k != Expr::Div || !bcast_col_of(y->a[1], bm, s_val))
    no_route("stored value is not e / broadcast(sum)");
  const Inst* s = find_inst(*b, s_val);
  if (!s || s->op != Op::Reduce || s->is_max || s->axis != 1 || s->rows != bm || s->cols != bn)
    no_route("denominator is not a row sum over the tile");
  const ExprP num = y->a[0];
  const ExprP summed = expand(*b, s->uses[0]);
  // e = exp(x - broadcast(m)), the same tree for the sum and the numerator
  auto is_exp_shift = [&](const ExprP& e, uint32_t& x, uint32_t& m) {
    if (e->k != Expr::Exp || e->a[0]->k != Expr::Sub) return false;
    const ExprP& diff = e->a[0];
    if (diff->a[0]->k != Expr::Value || !bcast_col_of(diff->a[1], bm, m)) return false;
    x = diff->a[0]->v;
    return true;
  };
  uint32_t x1, m1, x2, m2;
  if (!is_exp_shift(num, x1, m1) || !is_exp_shift(summed, x2, m2) || x1 != x2 || m1 != m2)
    no_route("numerator / summand is not exp(x - broadcast(max))");
  const Inst* mx = find_inst(*b, m1);
  if (!mx || mx->op != Op::Reduce || !mx->is_max || mx->axis != 1 || mx->uses[0] != x1 ||
      mx->rows != bm || mx->cols != bn)
    no_route("shift is not the row max of x");
  const Inst* ld = find_inst(*b, x1);
  if (!ld || ld->op != Op::LoadTko || ld->stride != 1 || ld->rows != bm || ld->cols != bn)
    no_route("x is not a rank-2 [BM, BN] tile load");
  if (launch_dim(fn, ld->uses[1]) != 0 || launch_dim(fn, ld->uses[2]) != 1 ||
      st.uses[2] != ld->uses[1] || st.uses[3] != ld->uses[2])
    no_route("load / store are not at the program's tile (launch 0, launch 1)");
  Match m;
  m.kind = SILE_ROUTE_SOFTMAX_TILES;
  m.ops[0] = operand_of(fn, ld->uses[0]);
  m.ops[1] = operand_of(fn, st.uses[0]);
  m.nops = 2;
  if (m.ops[0].rank != 2 || m.ops[1].rank != 2) no_route("softmax operand is not rank 2");
  m.tm = bm;
  m.tn = bn;
  return m;
}

// load X[pid0, c] [BM, BN]; r = reduce(x, axis 1); store Y <- r, where c is 0
// or launch index 1 and Y is [M, 1] at (pid0, pid1 | 0) or rank 1 at (0, pid0).
Match match_row_reduce(const Function& fn) {
  const Block* b;
  const Inst& st = single_side_effect(fn, b);
  if (st.op != Op::StoreTko) no_route("no tile store");
  const Inst* r = find_inst(*b, st.uses[1]);
  if (!r || r->op != Op::Reduce || r->axis != 1) no_route("stored value is not a row reduce");
  const int64_t bm = r->rows, bn = r->cols;
  if (st.rows != bm || st.cols != 1) no_route("store shape is not [BM, 1]");
  const Inst* ld = find_inst(*b, r->uses[0]);
  if (!ld || ld->op != Op::LoadTko || ld->stride != 1 || ld->rows != bm || ld->cols != bn)
    no_route("reduced value is not a rank-2 [BM, BN] tile load");
  if (launch_dim(fn, ld->uses[1]) != 0) no_route("row tile is not launch index 0");
  if (!is_const(*b, ld->uses[2], 0) && launch_dim(fn, ld->uses[2]) != 1)
    no_route("column tile is neither 0 nor launch index 1");
  Match m;
  m.kind = SILE_ROUTE_REDUCE_ROWS;
  m.reduce_op = r->is_max ? SILE_REDUCE_MAX : SILE_REDUCE_SUM;
  m.ops[0] = operand_of(fn, ld->uses[0]);
  m.ops[1] = operand_of(fn, st.uses[0]);
  m.nops = 2;
  if (m.ops[0].rank != 2) no_route("reduce input is not rank 2");
  if (m.ops[1].rank == 2) {
    if (st.stride != 1 || st.uses[2] != ld->uses[1] ||
        !(is_const(*b, st.uses[3], 0) || launch_dim(fn, st.uses[3]) == 1))
      no_route("store is not at (launch 0, launch 1 | 0)");
  } else if (m.ops[1].rank == 1) {
    if (st.stride != 0 || !is_const(*b, st.uses[2], 0) || st.uses[3] != ld->uses[1])
      no_route("rank-1 store is not at (0, launch 0)");
    m.out_rank1 = true;
  } else {
    no_route("reduce output rank is not 1 or 2");
  }
  m.tm = bm;
  m.tn = bn;
  return m;
}

// load A[0, pid0] [1, TILE] (rank 1); s = reduce_sum; out[0] += s[0, 0]
// (crates/sile/examples/parallel_reduce.rs:3-9).
Match match_atomic_reduce(const Function& fn) {
  const Block* b;
  const Inst& at = single_side_effect(fn, b);
  if (at.op != Op::AtomicAdd) no_route("no atomic add");
  const Inst* ex = find_inst(*b, at.uses[1]);
  if (!ex || ex->op != Op::Extract || !is_const(*b, ex->uses[1], 0) ||
      !is_const(*b, ex->uses[2], 0))
    no_route("atomic value is not element [0, 0] of a tile");
  const Inst* r = find_inst(*b, ex->uses[0]);
  if (!r || r->op != Op::Reduce || r->is_max || r->axis != 1 || r->rows != 1)
    no_route("extracted tile is not the sum of a [1, TILE] tile");
  const Inst* ld = find_inst(*b, r->uses[0]);
  if (!ld || ld->op != Op::LoadTko || ld->stride != 0 || ld->rows != 1 || ld->cols != r->cols ||
      !is_const(*b, ld->uses[1], 0) || launch_dim(fn, ld->uses[2]) != 0)
    no_route("summed value is not the program's rank-1 tile");
  if (!is_const(*b, at.uses[2], 0) || !is_const(*b, at.uses[3], 0) || at.stride != 0)
    no_route("atomic add does not target element 0");
  Match m;
  m.kind = SILE_ROUTE_ATOMIC_REDUCE;
  m.ops[0] = operand_of(fn, ld->uses[0]);
  m.ops[1] = operand_of(fn, at.uses[0]);
  m.nops = 2;
  if (m.ops[0].rank != 1 || m.ops[1].rank != 1) no_route("reduce operands are not rank 1");
  m.tn = r->cols;
  return m;
}

// Structural equality of two expanded map expressions.
bool same(const ExprP& x, const ExprP& y) {
  if (x->k != y->k || x->a.size() != y->a.size()) return false;
  switch (x->k) {
    case Expr::Value: return x->v == y->v;
    case Expr::Load:
      return x->buf == y->buf && x->row == y->row && x->col == y->col && x->rows == y->rows &&
             x->cols == y->cols && x->stride == y->stride;
    case Expr::Splat: return x->f == y->f;
    case Expr::Cmp: if (x->cmp != y->cmp) return false; break;
    case Expr::Bcast: if (x->rows != y->rows || x->cols != y->cols) return false; break;
    default: break;
  }
  for (size_t i = 0; i < x->a.size(); ++i)
    if (!same(x->a[i], y->a[i])) return false;
  return true;
}

bool is_val(const ExprP& e, uint32_t v) { return e->k == Expr::Value && e->v == v; }

// e = op(l, r) with l and r matching the two predicates in either order
// (Add and Mul commute).
template <class L, class R>
bool commuted(const ExprP& e, Expr::K op, L lhs, R rhs) {
  if (e->k != op || e->a.size() != 2) return false;
  return (lhs(e->a[0]) && rhs(e->a[1])) || (lhs(e->a[1]) && rhs(e->a[0]));
}

// Value of an expression of splats and pointwise ops only, in fp32 with each
// operation rounded, as the CPU backend evaluates a map
// (crates/sile-tile-ir/src/passes/lowering/tile_expr.rs:646-813); false if it
// reads anything else.
bool const_eval(const ExprP& e, float& out) {
  float a = 0.0f, b = 0.0f;
  switch (e->k) {
    case Expr::Splat: out = (float)e->f; return true;
    case Expr::Neg:
      if (!const_eval(e->a[0], a)) return false;
      out = 0.0f - a;
      return true;
    case Expr::Exp:
      if (!const_eval(e->a[0], a)) return false;
      out = expf(a);
      return true;
    case Expr::Bcast: return const_eval(e->a[0], out);
    case Expr::Add: case Expr::Sub: case Expr::Mul: case Expr::Div:
      if (!const_eval(e->a[0], a) || !const_eval(e->a[1], b)) return false;
      out = e->k == Expr::Add ? a + b : e->k == Expr::Sub ? a - b : e->k == Expr::Mul ? a * b : a / b;
      return true;
    default: return false;
  }
}

// The value an entry-block loop argument starts from, when it is a constant
// tile of the given shape (a splat, or a map of splats).
bool const_tile(const Block& entry, uint32_t v, int64_t rows, int64_t cols, float& out) {
  const Inst* i = find_inst(entry, v);
  if (!i || i->ty.k != Ty::Tile || i->ty.rows != rows || i->ty.cols != cols) return false;
  return const_eval(expand(entry, v), out);
}

// The attention program of the DSL (online softmax, K given transposed as
// kt [D, S]; the DSL has no mask, so it is not causal):
//   qt = load Q[pid0, 0] [BM, D]; m, l, acc = m0, 0, 0 tiles;
//   for j in 0 .. shape(kt)[1] / BN {
//     s = mma(qt, load KT[0, j] [D, BN], splat 0) (* splat scale);
//     m_new = max_tile(m, reduce_max(s, 1));     (select(m >= r, m, r))
//     p = exp(s - broadcast(m_new)); alpha = exp(m - m_new);
//     l = l * alpha + reduce_sum(p, 1);
//     acc = mma(p, load V[j, 0] [BN, D], acc * broadcast(alpha)); m = m_new }
//   store O[pid0, pid1] <- acc / broadcast(l)
// with its loop-carried values in any order
// (find_loop_carried_vars, crates/sile-tile-ir/src/lower.rs:446-465).
Match match_attention(const Function& fn) {
  if (fn.blocks.size() != 4) no_route("not an entry / loop header / body / exit function");
  const Block* entry = fn.block(fn.entry);
  if (entry->term.k != Term::Br || entry->term.targs.size() != 4)
    no_route("entry block does not jump into a loop carrying three tiles");
  if (!is_const(*entry, entry->term.targs[0], 0)) no_route("loop counter does not start at 0");
  const Block* header = fn.block(entry->term.t);
  if (!header || header->params.size() != 4) no_route("loop header does not carry (j, three tiles)");
  const Term& ht = header->term;
  const std::vector<uint32_t> carried(header->params.begin() + 1, header->params.end());
  if (ht.k != Term::CondBr || ht.targs != header->params || ht.fargs != carried)
    no_route("loop header branch arguments are not (j, tiles) / (tiles)");
  const Block* body = fn.block(ht.t);
  const Block* exit = fn.block(ht.f);
  if (!body || !exit || body->params.size() != 4 || exit->params.size() != 3)
    no_route("loop body / exit do not take the carried tiles");
  if (body->term.k != Term::Br || body->term.t != header->id || body->term.targs.size() != 4)
    no_route("loop body does not jump back with (j', tiles')");
  const uint32_t bj = body->params[0];
  const Inst* next = find_inst(*body, body->term.targs[0]);
  if (!next || next->op != Op::IBin || next->sub != "addi" ||
      !((next->uses[0] == bj && is_const(*body, next->uses[1], 1)) ||
        (next->uses[1] == bj && is_const(*body, next->uses[0], 1))))
    no_route("loop step is not j + 1");

  // exit: store O[pid0, pid1] <- acc / broadcast(l)
  const Inst* st = nullptr;
  for (const Inst& i : exit->insts) {
    if (i.op == Op::StoreTko || i.op == Op::AtomicAdd) {
      if (st) no_route("loop exit holds more than one store");
      st = &i;
    }
  }
  if (!st || st->op != Op::StoreTko || st->stride != 1 || exit->term.k != Term::Ret)
    no_route("loop exit does not store a rank-2 tile");
  const int64_t bm = st->rows, d = st->cols;
  const ExprP out = expand(*exit, st->uses[1]);
  uint32_t e_l = 0;
  if (out->k != Expr::Div || out->a[0]->k != Expr::Value || !bcast_col_of(out->a[1], bm, e_l))
    no_route("stored value is not acc / broadcast(l)");
  const uint32_t e_acc = out->a[0]->v;
  int pa = -1, pl = -1;
  for (int i = 0; i < 3; ++i) {
    if (exit->params[i] == e_acc) pa = i;
    if (exit->params[i] == e_l) pl = i;
  }
  if (pa < 0 || pl < 0 || pa == pl) no_route("stored acc / l are not the loop's carried tiles");
  const int pm = 3 - pa - pl;
  const uint32_t b_acc = body->params[1 + pa], b_l = body->params[1 + pl],
                 b_m = body->params[1 + pm];
  const uint32_t n_acc = body->term.targs[1 + pa], n_l = body->term.targs[1 + pl],
                 n_m = body->term.targs[1 + pm];

  // m_new = select(m >= rowmax(s), m, rowmax(s))
  const ExprP mnew = expand(*body, n_m);
  if (mnew->k != Expr::Select || mnew->a[0]->k != Expr::Cmp || mnew->a[0]->cmp != "ge" ||
      !is_val(mnew->a[0]->a[0], b_m) || mnew->a[0]->a[1]->k != Expr::Value ||
      !is_val(mnew->a[1], b_m) || !same(mnew->a[2], mnew->a[0]->a[1]))
    no_route("carried max is not max_tile(m, reduce_max(s, 1))");
  const Inst* rmax = find_inst(*body, mnew->a[2]->v);
  if (!rmax || rmax->op != Op::Reduce || !rmax->is_max || rmax->axis != 1 || rmax->rows != bm)
    no_route("max_tile's second operand is not a row max");
  const int64_t bn = rmax->cols;
  // s = mma(qt, kt tile, 0) [* scale]
  const ExprP s_tree = expand(*body, rmax->uses[0]);
  ExprP mma_leaf = s_tree;
  float scale = 1.0f;
  if (s_tree->k == Expr::Mul) {
    const int si = s_tree->a[0]->k == Expr::Splat ? 0 : s_tree->a[1]->k == Expr::Splat ? 1 : -1;
    if (si < 0) no_route("scores are scaled by something other than a constant");
    scale = (float)s_tree->a[si]->f;
    mma_leaf = s_tree->a[1 - si];
  }
  if (mma_leaf->k != Expr::Value) no_route("scores are not an mma result");
  const Inst* smma = find_inst(*body, mma_leaf->v);
  if (!smma || smma->op != Op::Mma || smma->m != bm || smma->n != bn || smma->k != d)
    no_route("scores are not mma(Q tile, K^T tile) of [BM, D] x [D, BN]");
  const Inst* zero = find_inst(*body, smma->uses[2]);
  if (!zero) zero = find_inst(*entry, smma->uses[2]);
  if (!zero || zero->op != Op::Splat || zero->fval != 0.0)
    no_route("score mma does not start from a zero tile");
  const Inst* lq = find_inst(*entry, smma->uses[0]);
  if (!lq || lq->op != Op::LoadTko || lq->stride != 1 || lq->rows != bm || lq->cols != d ||
      launch_dim(fn, lq->uses[1]) != 0 || !is_const(*entry, lq->uses[2], 0))
    no_route("Q tile is not loaded at (launch 0, 0) before the loop");
  const Inst* lk = find_inst(*body, smma->uses[1]);
  if (!lk || lk->op != Op::LoadTko || lk->stride != 1 || lk->rows != d || lk->cols != bn ||
      !is_const(*body, lk->uses[1], 0) || lk->uses[2] != bj)
    no_route("K^T tile is not loaded at (0, j)");
  // loop bound: shape(kt)[1] / BN
  const Inst* cmp = find_inst(*header, ht.cond);
  if (!cmp || cmp->op != Op::ICmp || cmp->sub != "lt" || cmp->uses[0] != header->params[0])
    no_route("loop condition is not j < bound");
  auto def = [&](uint32_t v) {
    const Inst* i = find_inst(*header, v);
    return i ? i : find_inst(*entry, v);
  };
  const Inst* div = def(cmp->uses[1]);
  const Inst* sdim = div && div->op == Op::IBin && div->sub == "divi" ? def(div->uses[0]) : nullptr;
  const Inst* bnc = div && div->op == Op::IBin && div->sub == "divi" ? def(div->uses[1]) : nullptr;
  const Param* sdesc = sdim && sdim->op == Op::ShapeDim ? fn.param(sdim->uses[0]) : nullptr;
  if (!sdim || sdim->ival != 1 || !bnc || bnc->op != Op::ConstI64 || bnc->ival != bn || !sdesc ||
      sdesc->kind != Param::Shape || sdesc->source != lk->uses[0])
    no_route("loop bound is not shape(kt)[1] / BN");

  // p = exp(s - broadcast(m_new)); alpha = exp(m - m_new)
  auto bcast_of = [&](const ExprP& e, const ExprP& src) {
    return e->k == Expr::Bcast && e->rows == bm && e->cols == 1 && same(e->a[0], src);
  };
  auto is_p = [&](const ExprP& e) {
    return e->k == Expr::Exp && e->a[0]->k == Expr::Sub && same(e->a[0]->a[0], s_tree) &&
           bcast_of(e->a[0]->a[1], mnew);
  };
  auto is_alpha = [&](const ExprP& e) {
    return e->k == Expr::Exp && e->a[0]->k == Expr::Sub && is_val(e->a[0]->a[0], b_m) &&
           same(e->a[0]->a[1], mnew);
  };
  // acc' = mma(p, V tile, acc * broadcast(alpha))
  const Inst* pv = find_inst(*body, n_acc);
  if (!pv || pv->op != Op::Mma || pv->m != bm || pv->n != d || pv->k != bn)
    no_route("carried acc is not an mma of [BM, BN] x [BN, D]");
  if (!is_p(expand(*body, pv->uses[0]))) no_route("P is not exp(s - broadcast(m_new))");
  const Inst* lv = find_inst(*body, pv->uses[1]);
  if (!lv || lv->op != Op::LoadTko || lv->stride != 1 || lv->rows != bn || lv->cols != d ||
      lv->uses[1] != bj || !is_const(*body, lv->uses[2], 0))
    no_route("V tile is not loaded at (j, 0)");
  if (!commuted(expand(*body, pv->uses[2]), Expr::Mul,
                [&](const ExprP& e) { return is_val(e, b_acc); },
                [&](const ExprP& e) { return e->k == Expr::Bcast && e->rows == bm && e->cols == 1 &&
                                             is_alpha(e->a[0]); }))
    no_route("PV accumulator is not acc * broadcast(exp(m - m_new))");
  // l' = l * alpha + reduce_sum(p, 1)
  const ExprP lnew = expand(*body, n_l);
  uint32_t rsum_v = 0;
  const bool l_ok = commuted(
      lnew, Expr::Add,
      [&](const ExprP& e) {
        return commuted(e, Expr::Mul, [&](const ExprP& x) { return is_val(x, b_l); }, is_alpha);
      },
      [&](const ExprP& e) {
        if (e->k != Expr::Value) return false;
        rsum_v = e->v;
        return true;
      });
  const Inst* rsum = l_ok ? find_inst(*body, rsum_v) : nullptr;
  if (!rsum || rsum->op != Op::Reduce || rsum->is_max || rsum->axis != 1 || rsum->rows != bm ||
      rsum->cols != bn || !is_p(expand(*body, rsum->uses[0])))
    no_route("carried l is not l * alpha + reduce_sum(p, 1)");

  // initial tiles: m = m0 (any constant), l = 0, acc = 0
  float m0 = 0.0f, l0 = 1.0f, acc0 = 1.0f;
  if (!const_tile(*entry, entry->term.targs[1 + pm], bm, 1, m0))
    no_route("running max does not start from a constant tile");
  if (!const_tile(*entry, entry->term.targs[1 + pl], bm, 1, l0) || l0 != 0.0f ||
      !const_tile(*entry, entry->term.targs[1 + pa], bm, d, acc0) || acc0 != 0.0f)
    no_route("l and acc do not start from zero tiles");
  // the store at the program's tile
  if (st->uses[2] != lq->uses[1] || launch_dim(fn, st->uses[3]) != 1)
    no_route("output tile is not stored at (launch 0, launch 1)");
  if (d > 128) no_route("head dim above 128");

  Match m;
  m.kind = SILE_ROUTE_ATTENTION;
  m.ops[0] = operand_of(fn, lq->uses[0]);
  m.ops[1] = operand_of(fn, lk->uses[0]);
  m.ops[2] = operand_of(fn, lv->uses[0]);
  m.ops[3] = operand_of(fn, st->uses[0]);
  m.nops = 4;
  for (int i = 0; i < 4; ++i)
    if (m.ops[i].rank != 2) no_route("attention operand is not rank 2");
  m.tm = bm;
  m.tn = bn;
  m.tk = d;
  m.scale = scale;
  m.m0 = m0;
  return m;
}

// A tile load, whether the fusion pass folded it into a map (Expr::Load) or
// left it standing (a value defined by load_ptr_tko in block b).
struct TileLoad {
  uint32_t buf = 0, row = 0, col = 0;
  int64_t rows = 0, cols = 0, stride = 0;
};
bool tile_load_of(const Block& b, const ExprP& e, TileLoad& out) {
  if (e->k == Expr::Load) {
    out = TileLoad{e->buf, e->row, e->col, e->rows, e->cols, e->stride};
    return true;
  }
  if (e->k != Expr::Value) return false;
  const Inst* i = find_inst(b, e->v);
  if (!i || i->op != Op::LoadTko) return false;
  out = TileLoad{i->uses[0], i->uses[1], i->uses[2], i->rows, i->cols, i->stride};
  return true;
}

// The matvec kernel of crates/sile/examples/mlp.rs:26-44:
//   acc = constant(s, [BM]); k_tiles = x.shape()[1] / BK;
//   for k in 0..k_tiles {
//     acc = acc + reduce_sum(x.load_tile([BM, BK], [pid, k]) *
//                            y.load_tile([BK], [k]).broadcast([BM, BK]), 1) }
//   z.store(acc)
// with x rank 2, y and z rank 1: the [1, BM] accumulator is stored at
// [0, pid] (lower.rs:777-821).  Fused (the product and the broadcast load
// folded into one map, pointwise_fusion.rs:5-235) and unfused forms alike.
Match match_matvec(const Function& fn) {
  const Block* entry = fn.block(fn.entry);
  if (entry->term.k != Term::Br || entry->term.targs.size() != 2)
    no_route("entry block does not jump into a loop with (k, acc)");
  if (!is_const(*entry, entry->term.targs[0], 0)) no_route("loop counter does not start at constant 0");
  const Inst* acc_seed = find_inst(*entry, entry->term.targs[1]);
  if (!acc_seed || acc_seed->op != Op::Splat || acc_seed->ty.k != Ty::Tile || acc_seed->ty.rows != 1)
    no_route("accumulator is not a [1, BM] splat");
  const int64_t bm = acc_seed->ty.cols;

  const Block* header = fn.block(entry->term.t);
  if (header->params.size() != 2) no_route("loop header does not carry (k, acc)");
  const uint32_t loop_k = header->params[0], loop_acc = header->params[1];
  const Term& ht = header->term;
  if (ht.k != Term::CondBr || ht.targs != std::vector<uint32_t>{loop_k, loop_acc} ||
      ht.fargs != std::vector<uint32_t>{loop_acc})
    no_route("loop header does not branch with (k, acc) / (acc)");
  const Inst* cmp = find_inst(*header, ht.cond);
  if (!cmp || cmp->op != Op::ICmp || cmp->sub != "lt" || cmp->uses[0] != loop_k)
    no_route("loop condition is not k < bound");
  auto def = [&](uint32_t v) {
    const Inst* i = find_inst(*header, v);
    return i ? i : find_inst(*entry, v);
  };
  const Inst* ktiles = def(cmp->uses[1]);
  if (!ktiles || ktiles->op != Op::IBin || ktiles->sub != "divi") no_route("loop bound is not a division");
  const Inst* bk_inst = def(ktiles->uses[1]);
  if (!bk_inst || bk_inst->op != Op::ConstI64 || bk_inst->ival <= 0)
    no_route("loop bound divisor is not a positive constant");
  const int64_t bk = bk_inst->ival;
  const Inst* sdim = def(ktiles->uses[0]);
  if (!sdim || sdim->op != Op::ShapeDim || sdim->ival != 1) no_route("loop bound is not shape(x)[1] / BK");
  const Param* sdesc = fn.param(sdim->uses[0]);
  if (!sdesc || sdesc->kind != Param::Shape) no_route("shape_dim of a non-descriptor");
  const uint32_t x_buf = sdesc->source;

  const Block* body = fn.block(ht.t);
  if (body->params.size() != 2) no_route("loop body does not take (k, acc)");
  const uint32_t body_k = body->params[0], body_acc = body->params[1];
  if (body->term.k != Term::Br || body->term.t != header->id || body->term.targs.size() != 2)
    no_route("loop body does not jump back with (k', acc')");
  const Inst* next_k = find_inst(*body, body->term.targs[0]);
  if (!next_k || next_k->op != Op::IBin || next_k->sub != "addi") no_route("loop step is not an addition");
  const uint32_t one = next_k->uses[0] == body_k ? next_k->uses[1]
                       : next_k->uses[1] == body_k ? next_k->uses[0] : UINT32_MAX;
  if (one == UINT32_MAX || !is_const(*body, one, 1)) no_route("loop step is not k + 1");

  // acc' = acc + reduce_sum(..., 1), either operand order
  const ExprP next = expand(*body, body->term.targs[1]);
  if (next->k != Expr::Add || next->a.size() != 2) no_route("carried accumulator is not acc + partial");
  uint32_t red_v;
  if (is_val(next->a[0], body_acc) && next->a[1]->k == Expr::Value)
    red_v = next->a[1]->v;
  else if (is_val(next->a[1], body_acc) && next->a[0]->k == Expr::Value)
    red_v = next->a[0]->v;
  else
    no_route("carried accumulator is not acc + partial");
  const Inst* red = find_inst(*body, red_v);
  if (!red || red->op != Op::Reduce || red->is_max || red->axis != 1 || red->rows != bm ||
      red->cols != bk)
    no_route("partial is not a row sum of a [BM, BK] tile");
  // the reduced tile: x tile * broadcast(y tile), either order
  const ExprP prod = expand(*body, red->uses[0]);
  if (prod->k != Expr::Mul || prod->a.size() != 2) no_route("reduced tile is not a product");
  TileLoad lx, ly;
  ExprP other;
  if (tile_load_of(*body, prod->a[0], lx)) {
    other = prod->a[1];
  } else if (tile_load_of(*body, prod->a[1], lx)) {
    other = prod->a[0];
  } else {
    no_route("product has no tile load of x");
  }
  if (other->k != Expr::Bcast || other->rows != 1 || other->cols != bk || other->a.size() != 1 ||
      !tile_load_of(*body, other->a[0], ly))
    no_route("product's other factor is not a broadcast [1, BK] tile load");
  if (lx.buf != x_buf || lx.rows != bm || lx.cols != bk || lx.stride != 1 || lx.col != body_k)
    no_route("x tile is not x[pid, k] of [BM, BK]");
  const uint32_t pid = lx.row;
  if (launch_dim(fn, pid) != 0) no_route("x tile row is not launch index 0");
  if (ly.rows != 1 || ly.cols != bk || ly.stride != 0 || ly.col != body_k || !is_const(*body, ly.row, 0))
    no_route("y tile is not y[k] of [BK] (rank 1)");

  const Block* exit = fn.block(ht.f);
  if (exit->params.size() != 1 || exit->term.k != Term::Ret) no_route("loop exit does not take acc and return");
  const Inst* st = nullptr;
  for (const Inst& i : exit->insts) {
    if (i.op == Op::ConstI64) continue;
    if (st || i.op != Op::StoreTko) no_route("loop exit holds more than the store");
    st = &i;
  }
  if (!st || st->uses[1] != exit->params[0] || st->stride != 0 || st->rows != 1 || st->cols != bm ||
      !is_const(*exit, st->uses[2], 0) || st->uses[3] != pid)
    no_route("loop exit does not store acc at [0, pid] of a rank-1 output");

  Match m;
  m.kind = SILE_ROUTE_MATVEC;
  m.ops[0] = operand_of(fn, x_buf);
  m.ops[1] = operand_of(fn, ly.buf);
  m.ops[2] = operand_of(fn, st->uses[0]);
  m.nops = 3;
  if (m.ops[0].rank != 2 || m.ops[1].rank != 1 || m.ops[2].rank != 1)
    no_route("operand ranks are not x 2, y 1, z 1");
  m.tm = bm;
  m.tk = bk;
  m.seed_value = acc_seed->fval;
  return m;
}

// Tries each detector; collects the reasons of the ones that did not fire.
Match detect(const Function& fn, std::string& reasons) {
  struct TypesScope {
    explicit TypesScope(const std::map<uint32_t, Ty>* t) { t_types = t; }
    ~TypesScope() { t_types = nullptr; }
  } scope(&fn.types);
  using Fn = Match (*)(const Function&);
  const std::pair<const char*, Fn> detectors[] = {
      {"matmul", match_matmul},
      {"softmax", match_softmax},
      {"row reduce", match_row_reduce},
      {"atomic reduce", match_atomic_reduce},
      {"attention", match_attention},
      {"matvec", match_matvec},
  };
  for (const auto& d : detectors) {
    try {
      return d.second(fn);
    } catch (const NoRoute& e) {
      if (!reasons.empty()) reasons += "; ";
      reasons += std::string(d.first) + ": " + e.why;
    }
  }
  return Match{};
}

int64_t dim(const int64_t* shapes, const Operand& o, int d) { return shapes[o.shape_offset + d]; }

void set_reason(sile_hip_route* r, const std::string& s) {
  snprintf(r->reason, sizeof(r->reason), "%s", s.c_str());
}

// Chooses the kernel for the shapes of this launch.  Tile semantics of the
// CPU wrapper: tiles_n = shape(out)[1] / cols, total = (shape(out)[0] / rows)
// * tiles_n for a rank-2 output (shape(out)[0] for rank 1), and programs
// min(num_threadgroups, total) run (codegen.rs:409-431, 517-531).
void plan(const Match& m, const int64_t* shapes, int64_t programs, sile_hip_route* r) {
  r->kind = m.kind;
  r->reduce_op = m.reduce_op;
  r->seed_from_tile = m.seed_from_tile ? 1 : 0;
  r->seed_value = (float)m.seed_value;
  for (int i = 0; i < 4; ++i) {
    r->buffer[i] = i < m.nops ? m.ops[i].index : -1;
    r->shape_offset[i] = i < m.nops ? m.ops[i].shape_offset : -1;
    r->rank[i] = i < m.nops ? m.ops[i].rank : 0;
  }
  int n = 0;
  for (int i = 0; i < m.nops; ++i)
    for (int d = 0; d < m.ops[i].rank; ++d) r->operand_shapes[n++] = dim(shapes, m.ops[i], d);
  r->num_threadgroups = programs;
  r->tile_m = m.tm;
  r->tile_n = m.tn;
  r->tile_k = m.tk;
  r->rows = r->cols = 0;
  r->attn_scale = m.scale;
  r->attn_m0 = m.m0;
  if (m.kind == SILE_ROUTE_ATTENTION) {
    // o [n, d'] in tiles of [BM, D]: one column tile, programs take row bands
    const Operand &q = m.ops[0], &kt = m.ops[1], &v = m.ops[2], &o = m.ops[3];
    auto decline = [&](const char* why) {
      r->kind = SILE_ROUTE_NONE;
      set_reason(r, std::string("attention: ") + why);
    };
    if (dim(shapes, o, 1) / m.tk != 1) return decline("output has more than one column tile");
    const int64_t run = std::max<int64_t>(0, std::min(programs, dim(shapes, o, 0) / m.tm));
    const int64_t n_keys = (dim(shapes, kt, 1) / m.tn) * m.tn;
    if (dim(shapes, q, 0) < run * m.tm || dim(shapes, q, 1) < m.tk)
      return decline("Q does not cover the query tiles");
    if (dim(shapes, kt, 0) < m.tk || dim(shapes, v, 0) < n_keys || dim(shapes, v, 1) < m.tk)
      return decline("K^T / V do not cover the key tiles");
    r->rows = run * m.tm;
    r->cols = n_keys;
  } else if (m.kind == SILE_ROUTE_MATVEC) {
    // z rank 1: total = shape(z)[0] programs at most (codegen.rs:409-431);
    // program pid writes z[pid BM .. pid BM + BM) from rows of x
    const Operand &x = m.ops[0], &y = m.ops[1], &z = m.ops[2];
    auto decline = [&](const char* why) {
      r->kind = SILE_ROUTE_NONE;
      set_reason(r, std::string("matvec: ") + why);
    };
    const int64_t run = std::max<int64_t>(0, std::min(programs, dim(shapes, z, 0)));
    const int64_t rows = run * m.tm;
    const int64_t k = dim(shapes, x, 1);
    if (rows > dim(shapes, z, 0)) return decline("programs would write past the rank-1 output");
    if (rows > dim(shapes, x, 0)) return decline("x does not cover the programs' rows");
    if (dim(shapes, y, 0) < (k / m.tk) * m.tk) return decline("y does not cover the K tiles");
    r->rows = rows;
    r->cols = k;
  } else if (m.kind == SILE_ROUTE_SOFTMAX_TILES) {
    const Operand &x = m.ops[0], &y = m.ops[1];
    const int64_t tiles_n = m.tn > 0 ? dim(shapes, y, 1) / m.tn : 0;
    const int64_t total = m.tm > 0 ? (dim(shapes, y, 0) / m.tm) * tiles_n : 0;
    const int64_t run = std::max<int64_t>(0, std::min(programs, total));
    // one column tile per row band: each program's tile is whole rows of
    // [run * BM, BN], the row softmax's domain
    if (tiles_n == 1 && dim(shapes, x, 0) >= run * m.tm && dim(shapes, x, 1) >= m.tn) {
      r->kind = SILE_ROUTE_SOFTMAX_ROWS;
      r->rows = run * m.tm;
      r->cols = m.tn;
    }
  } else if (m.kind == SILE_ROUTE_REDUCE_ROWS) {
    const Operand &x = m.ops[0], &y = m.ops[1];
    int64_t run;
    if (m.out_rank1) {
      run = std::max<int64_t>(0, std::min(programs, dim(shapes, y, 0)));
      if (run * m.tm > dim(shapes, y, 0)) {
        r->kind = SILE_ROUTE_NONE;
        set_reason(r, "row reduce: programs would write past the rank-1 output");
        return;
      }
    } else {
      if (dim(shapes, y, 1) != 1) {
        r->kind = SILE_ROUTE_NONE;
        set_reason(r, "row reduce: output has more than one column tile");
        return;
      }
      run = std::max<int64_t>(0, std::min(programs, dim(shapes, y, 0) / m.tm));
    }
    if (dim(shapes, x, 1) < m.tn || dim(shapes, x, 0) < run * m.tm) {
      r->kind = SILE_ROUTE_NONE;
      set_reason(r, "row reduce: input does not cover the tiles");
      return;
    }
    r->rows = run * m.tm;
    r->cols = m.tn;
  }
  r->reason[0] = 0;
}

int check_shapes(const Function& fn, const int64_t* shapes, int64_t num_shapes) {
  int64_t want = 0;
  for (const Param& p : fn.params)
    if (p.kind == Param::Buffer) want += p.rank;
  if (num_shapes != want)
    return fail(SILE_ERR_SHAPE, "%lld shape values for buffers of total rank %lld",
                (long long)num_shapes, (long long)want);
  if (want > 0 && !shapes) return fail(SILE_ERR_SHAPE, "NULL shapes");
  for (int64_t i = 0; i < want; ++i)
    if (shapes[i] < 0) return fail(SILE_ERR_SHAPE, "negative extent in shapes[%lld]", (long long)i);
  return SILE_OK;
}

}  // namespace

extern "C" {

int sile_hip_tile_ir_route(const char* tile_ir_text, const int64_t* shapes, int64_t num_shapes,
                           int64_t num_threadgroups, sile_hip_route* out) {
  if (!tile_ir_text || !out) return fail(SILE_ERR_SHAPE, "NULL Tile IR text or route");
  if (num_threadgroups < 0) return fail(SILE_ERR_SHAPE, "negative num_threadgroups");
  memset(out, 0, sizeof(*out));
  try {
    const Function fn = parse(tile_ir_text);
    const int rc = check_shapes(fn, shapes, num_shapes);
    if (rc != SILE_OK) return rc;
    int nbuf = 0;
    for (const Param& p : fn.params) nbuf += p.kind == Param::Buffer;
    out->num_buffers = nbuf;
    out->num_shapes = num_shapes;
    std::string reasons;
    const Match m = detect(fn, reasons);
    if (m.kind == SILE_ROUTE_NONE) {
      out->kind = SILE_ROUTE_NONE;
      for (int i = 0; i < 4; ++i) out->buffer[i] = out->shape_offset[i] = -1;
      set_reason(out, reasons);
      return ok();
    }
    plan(m, shapes, num_threadgroups, out);
  } catch (const ParseError& e) {
    return fail(SILE_ERR_COMPILE, "%s", e.msg.c_str());
  } catch (const NoRoute& e) {
    return fail(SILE_ERR_COMPILE, "Tile IR: %s", e.why.c_str());
  } catch (const std::exception& e) {
    return fail(SILE_ERR_COMPILE, "Tile IR: %s", e.what());
  }
  return ok();
}

int sile_hip_tile_ir_launch(const sile_hip_route* route, void* const* buffers,
                            int64_t num_buffers, const int64_t* shapes, int64_t num_shapes,
                            int64_t num_threadgroups, sile_hip_stream stream) {
  if (!route) return fail(SILE_ERR_SHAPE, "NULL route");
  if (route->kind == SILE_ROUTE_NONE)
    return fail(SILE_ERR_UNSUPPORTED_BACKEND, "no hand-written kernel for this Tile IR (%s)",
                route->reason);
  if (num_buffers != route->num_buffers || num_shapes != route->num_shapes)
    return fail(SILE_ERR_SHAPE, "launch has %lld buffers / %lld shape values, route was made for "
                "%d / %lld", (long long)num_buffers, (long long)num_shapes, route->num_buffers,
                (long long)route->num_shapes);
  if (!buffers || (num_shapes > 0 && !shapes)) return fail(SILE_ERR_SHAPE, "NULL buffers / shapes");
  const int nops = route->kind == SILE_ROUTE_MATMUL ? (route->seed_from_tile ? 4 : 3)
                   : route->kind == SILE_ROUTE_ATTENTION ? 4
                   : route->kind == SILE_ROUTE_MATVEC ? 3 : 2;
  void* bufs[4] = {nullptr, nullptr, nullptr, nullptr};
  int64_t shp[8] = {0, 0, 0, 0, 0, 0, 0, 0};
  int64_t nshp = 0;
  for (int i = 0; i < nops; ++i) {
    const int b = route->buffer[i], off = route->shape_offset[i], rk = route->rank[i];
    if (b < 0 || b >= num_buffers || off < 0 || rk < 1 || rk > 2 || off + rk > num_shapes)
      return fail(SILE_ERR_SHAPE, "route operand %d out of range", i);
    bufs[i] = buffers[b];
    for (int d = 0; d < rk; ++d) shp[nshp++] = shapes[off + d];
  }
  // the kernel and its extents were chosen for one set of shapes and one grid
  for (int64_t i = 0; i < nshp; ++i)
    if (shp[i] != route->operand_shapes[i])
      return fail(SILE_ERR_SHAPE, "launch shapes differ from the shapes the route was made for");
  if (num_threadgroups != route->num_threadgroups)
    return fail(SILE_ERR_SHAPE, "launch grid (%lld programs) differs from the route's (%lld)",
                (long long)num_threadgroups, (long long)route->num_threadgroups);
  hipStream_t s = static_cast<hipStream_t>(stream);
  int rc = SILE_OK;
  switch (route->kind) {
    case SILE_ROUTE_MATMUL:
      // the canonical matmul, or the tile MMA from a splat or a loaded accumulator
      return sile_rt::kernel_matmul_seeded(bufs, num_threadgroups, 1, shp, route->tile_m, route->tile_n,
                                  route->tile_k,
                                  route->seed_from_tile ? static_cast<const float*>(bufs[3]) : nullptr,
                                  route->seed_from_tile ? shp + 6 : nullptr, route->seed_value, s);
    case SILE_ROUTE_SOFTMAX_TILES:
      return sile_hip_kernel_softmax(bufs, num_threadgroups, 1, shp, 4, route->tile_m,
                                     route->tile_n, stream);
    case SILE_ROUTE_ATOMIC_REDUCE:
      return sile_hip_kernel_parallel_reduce(bufs, num_threadgroups, 1, shp, 2, route->tile_n,
                                             nullptr, stream);
    case SILE_ROUTE_ATTENTION:
      // q [q0, q1], kt [k0, k1], v [v0, v1], o [o0, o1]: leading dimensions q1, k1, v1, o1
      rc = sile_hip_attention_f32_kt(route->rows, route->cols, route->tile_k,
                                     static_cast<const float*>(bufs[0]), shp[1],
                                     static_cast<const float*>(bufs[1]), shp[3],
                                     static_cast<const float*>(bufs[2]), shp[5],
                                     static_cast<float*>(bufs[3]), shp[7], route->attn_scale,
                                     route->attn_m0, stream);
      break;
    case SILE_ROUTE_MATVEC:
      // x [x0, x1] (row pitch x1 = K), y [y0], z [z0]
      rc = sile_hip_matvec_f32(route->rows, route->cols, route->tile_k,
                               static_cast<const float*>(bufs[0]), shp[1],
                               static_cast<const float*>(bufs[1]), route->seed_value,
                               static_cast<float*>(bufs[2]), stream);
      break;
    case SILE_ROUTE_SOFTMAX_ROWS:
      // x [x0, x1], y [y0, y1]: rows of BN elements at leading dimensions x1 / y1
      rc = sile_hip_softmax_rows(SILE_F32, SILE_F32, route->rows, route->cols, bufs[0], shp[1],
                                 bufs[1], shp[3], stream);
      break;
    case SILE_ROUTE_REDUCE_ROWS:
      // a reduce of a load is the reference's fused load + reduce: the sum in
      // its vec4 window order, which may read on into x past a row
      if (route->reduce_op == SILE_REDUCE_SUM)
        rc = sile_hip_reduce_rows_fused_sum(route->rows, route->cols,
                                            static_cast<const float*>(bufs[0]), shp[1],
                                            shp[0] * shp[1], static_cast<float*>(bufs[1]), stream);
      else
        rc = sile_hip_reduce_rows((sile_reduce_op)route->reduce_op, SILE_F32, route->rows,
                                  route->cols, bufs[0], shp[1], static_cast<float*>(bufs[1]),
                                  stream);
      break;
    default:
      return fail(SILE_ERR_SHAPE, "unknown route kind %d", route->kind);
  }
  if (rc != SILE_OK) return rc;
  // the tile entry points return after completion (apply() semantics); so do these
  SILE_HIP_CHECK(hipStreamSynchronize(s));
  return ok();
}

}  // extern "C"
