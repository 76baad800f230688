// Front end of libtforge_hip: parses the tforge program text, verifies it with
// the reference dialect's rules and messages, parses the GPU pipeline option
// string, and plans kernel launches by matching fused chains
// matmul [-> bias_add] [-> relu] [-> add] (and element-op chains).
//
// Reference behaviour restated here (paths in the TensorForge tree):
//  * op syntax and types: include/TensorForge/Dialect/TForge/TForgeOps.td:37-113,
//    program shape: python/tforge_cpu.py:29-53, examples/mbr.mlir:3-8;
//  * verifier order and messages: lib/Dialect/TForge/TForgeOps.cpp:27-124,
//    test/Dialect/TForge/invalid.mlir;
//  * option names/defaults/errors: include/TensorForge/Pipelines.h:45-72,
//    lib/Pipelines/Pipelines.cpp:214-263;
//  * staged shapes must be multiples of the tiles (and the located error):
//    lib/Transforms/Gpu.cpp:251-255, test/Pipelines/gpu-staged.mlir:39;
//  * epilogue fusion legality (single use, elementwise, in place):
//    lib/Transforms/TileAndFuse.cpp:78-131.
#include "frontend.h"

#include <cctype>
#include <map>
#include <sstream>

#include "tf_kernels.h"

namespace tff {

bool Type::static_shape() const {
  for (int64_t d : shape)
    if (d < 0) return false;
  return true;
}

// Product of dimensions, saturating at INT64_MAX (shapes are user text).
static int64_t product(const std::vector<int64_t> &dims, size_t count) {
  int64_t n = 1;
  for (size_t i = 0; i < count; ++i)
    if (__builtin_mul_overflow(n, dims[i], &n)) return INT64_MAX;
  return n;
}

int64_t Type::numel() const { return product(shape, shape.size()); }

int64_t Buffer::numel() const { return product(shape, shape.size()); }

std::string format_error(const std::string &source_name, Loc loc, const std::string &msg) {
  std::ostringstream os;
  os << (source_name.empty() ? "<input>" : source_name) << ":" << loc.line << ":" << loc.col
     << ": error: " << msg;
  return os.str();
}

static std::string shape_str(const std::vector<int64_t> &s) {
  if (s.empty()) return "scalar";
  std::string r;
  for (size_t i = 0; i < s.size(); ++i) r += (i ? "x" : "") + std::to_string(s[i]);
  return r;
}

// ---------------------------------------------------------------- parser ---

namespace {

struct Lexer {
  const std::string &s;
  size_t i = 0;
  int line = 1, col = 1;
  explicit Lexer(const std::string &src) : s(src) {}

  Loc loc() const { return Loc{line, col}; }
  bool eof() { skip(); return i >= s.size(); }
  void adv(size_t n = 1) {
    while (n-- && i < s.size()) {
      if (s[i] == '\n') {
        ++line;
        col = 1;
      } else {
        ++col;
      }
      ++i;
    }
  }
  void skip() {
    for (;;) {
      while (i < s.size() && std::isspace((unsigned char)s[i])) adv();
      if (i + 1 < s.size() && s[i] == '/' && s[i + 1] == '/') {
        while (i < s.size() && s[i] != '\n') adv();
        continue;
      }
      break;
    }
  }
  bool peek(const std::string &t) {
    skip();
    return s.compare(i, t.size(), t) == 0;
  }
  bool accept(const std::string &t) {
    if (!peek(t)) return false;
    adv(t.size());
    return true;
  }
  static bool idch(char c) { return std::isalnum((unsigned char)c) || c == '_' || c == '.' || c == '$' || c == '-'; }
  // identifier-like token (letters, digits, _ . $ -)
  std::string ident() {
    skip();
    size_t j = i;
    while (j < s.size() && idch(s[j])) ++j;
    std::string r = s.substr(i, j - i);
    adv(j - i);
    return r;
  }
};

struct Parser {
  Lexer lx;
  std::string src_name;
  std::string err;
  Parser(const std::string &text, const std::string &name) : lx(text), src_name(name) {}

  bool fail(Loc l, const std::string &m) {
    if (err.empty()) err = format_error(src_name, l, m);
    return false;
  }
  bool expect(const std::string &t) {
    Loc l = lx.loc();
    lx.skip();
    l = lx.loc();
    if (!lx.accept(t)) return fail(l, "expected '" + t + "'");
    return true;
  }

  bool value_name(std::string &out) {
    lx.skip();
    Loc l = lx.loc();
    if (!lx.accept("%")) return fail(l, "expected SSA value");
    std::string id = lx.ident();
    if (id.empty()) return fail(l, "expected SSA value name");
    out = "%" + id;
    return true;
  }

  // tensor<64x32xf32>, tensor<?x4xf32>, tensor<*xf32>, tensor<f32>, or a
  // builtin scalar type (f32, i32, ...).
  bool type(Type &t) {
    lx.skip();
    Loc l = lx.loc();
    if (lx.accept("tensor")) {
      t.is_tensor = true;
      if (!expect("<")) return false;
      t.shape.clear();
      if (lx.accept("*")) {
        t.ranked = false;
        if (!expect("x")) return false;
      } else {
        for (;;) {
          lx.skip();
          size_t i = lx.i;
          if (i < lx.s.size() && lx.s[i] == '?') {
            lx.adv();
            t.shape.push_back(-1);
            if (!expect("x")) return false;
            continue;
          }
          if (i < lx.s.size() && std::isdigit((unsigned char)lx.s[i])) {
            const Loc dl = lx.loc();
            size_t j = i;
            int64_t d = 0;
            bool too_big = false;
            for (; j < lx.s.size() && std::isdigit((unsigned char)lx.s[j]); ++j) {
              const int64_t digit = lx.s[j] - '0';
              if (d > (INT64_MAX - digit) / 10) too_big = true;
              else d = d * 10 + digit;
            }
            if (too_big) return fail(dl, "invalid dimension");  // past int64, as MLIR's type parser says
            t.shape.push_back(d);
            lx.adv(j - i);
            if (!expect("x")) return false;
            continue;
          }
          break;
        }
      }
      lx.skip();
      size_t j = lx.i;
      while (j < lx.s.size() && std::isalnum((unsigned char)lx.s[j])) ++j;
      t.elem = lx.s.substr(lx.i, j - lx.i);
      lx.adv(j - lx.i);
      if (t.elem.empty()) return fail(lx.loc(), "expected element type");
      if (!expect(">")) return false;
      std::string txt = "tensor<";
      if (!t.ranked) txt += "*x";
      for (int64_t d : t.shape) txt += (d < 0 ? std::string("?") : std::to_string(d)) + "x";
      t.text = txt + t.elem + ">";
      return true;
    }
    size_t j = lx.i;
    while (j < lx.s.size() && std::isalnum((unsigned char)lx.s[j])) ++j;
    std::string name = lx.s.substr(lx.i, j - lx.i);
    if (name.empty()) return fail(l, "expected type");
    lx.adv(j - lx.i);
    t.is_tensor = false;
    t.elem = name;
    t.text = name;
    return true;
  }

  bool op_stmt(Program &p) {
    Op op;
    if (!value_name(op.result)) return false;
    if (!expect("=")) return false;
    lx.skip();
    op.loc = lx.loc();
    bool generic = false;
    std::string full;
    if (lx.accept("\"")) {
      generic = true;
      full = lx.ident();
      if (!expect("\"")) return false;
    } else {
      full = lx.ident();
    }
    if (full.rfind("tforge.", 0) != 0) return fail(op.loc, "unsupported operation '" + full + "'");
    op.name = full.substr(7);
    if (op.name != "matmul" && op.name != "bias_add" && op.name != "relu" && op.name != "add")
      return fail(op.loc, "unknown operation '" + full + "'");
    const int arity = op.name == "relu" ? 1 : 2;
    if (generic) {
      if (!expect("(")) return false;
      for (int k = 0; k < arity; ++k) {
        std::string v;
        if (k && !expect(",")) return false;
        if (!value_name(v)) return false;
        op.operands.push_back(v);
      }
      if (!expect(")")) return false;
      if (!expect(":")) return false;
      if (!expect("(")) return false;
      for (int k = 0; k < arity; ++k) {
        Type t;
        if (k && !expect(",")) return false;
        if (!type(t)) return false;
        op.operand_types.push_back(t);
      }
      if (!expect(")")) return false;
    } else {
      for (int k = 0; k < arity; ++k) {
        std::string v;
        if (k && !expect(",")) return false;
        if (!value_name(v)) return false;
        op.operands.push_back(v);
      }
      if (lx.peek("{")) {  // empty attr-dict
        lx.accept("{");
        if (!expect("}")) return false;
      }
      if (!expect(":")) return false;
      for (int k = 0; k < arity; ++k) {
        Type t;
        if (k && !expect(",")) return false;
        if (!type(t)) return false;
        op.operand_types.push_back(t);
      }
    }
    if (!expect("->")) return false;
    if (!type(op.result_type)) return false;
    p.ops.push_back(op);
    return true;
  }

  bool func(Program &p) {
    lx.skip();
    p.func_loc = lx.loc();
    if (!lx.accept("func.func")) return fail(p.func_loc, "expected 'func.func'");
    lx.skip();
    Loc l = lx.loc();
    if (!lx.accept("@")) return fail(l, "expected function name");
    p.func_name = lx.ident();
    if (!expect("(")) return false;
    if (!lx.accept(")")) {
      for (;;) {
        std::string v;
        Type t;
        if (!value_name(v) || !expect(":") || !type(t)) return false;
        p.arg_names.push_back(v);
        p.arg_types.push_back(t);
        if (lx.accept(")")) break;
        if (!expect(",")) return false;
      }
    }
    if (lx.accept("->")) {
      if (lx.accept("(")) {
        for (;;) {
          Type t;
          if (!type(t)) return false;
          p.result_types.push_back(t);
          if (lx.accept(")")) break;
          if (!expect(",")) return false;
        }
      } else {
        Type t;
        if (!type(t)) return false;
        p.result_types.push_back(t);
      }
    }
    if (!expect("{")) return false;
    for (;;) {
      lx.skip();
      if (lx.peek("}")) break;
      if (lx.peek("return")) {
        p.ret_loc = lx.loc();
        lx.accept("return");
        p.has_return = true;
        lx.skip();
        if (lx.peek("%")) {
          if (!value_name(p.ret_value) || !expect(":") || !type(p.ret_type)) return false;
        }
        continue;
      }
      if (lx.peek("%")) {
        if (!op_stmt(p)) return false;
        continue;
      }
      return fail(lx.loc(), "expected operation or 'return'");
    }
    return expect("}");
  }
};

}  // namespace

bool parse_program(const std::string &text, const std::string &source_name, Program &out,
                   std::string &err) {
  Parser ps(text, source_name);
  out = Program();
  out.source_name = source_name;
  bool module = false;
  if (ps.lx.peek("module")) {
    ps.lx.accept("module");
    if (!ps.expect("{")) {
      err = ps.err;
      return false;
    }
    module = true;
  }
  if (!ps.func(out) || (module && !ps.expect("}"))) {
    err = ps.err;
    return false;
  }
  if (!ps.lx.eof()) {
    err = format_error(source_name, ps.lx.loc(), "expected a single func.func (trailing input)");
    return false;
  }
  return true;
}

// -------------------------------------------------------------- verifier ---

namespace {

// verifyTForgeTensor: ranked, then static, then f32 (TForgeOps.cpp:27-43).
bool check_tensor(const Program &p, const Op &op, const Type &t, const std::string &what,
                  std::string &err) {
  const std::string pre = "'tforge." + op.name + "' op ";
  if (!t.ranked) {
    err = format_error(p.source_name, op.loc, pre + what + " must be a ranked tensor, but got '" + t.text + "'");
    return false;
  }
  if (!t.static_shape()) {
    err = format_error(p.source_name, op.loc, pre + what + " must have a static shape, but got '" + t.text + "'");
    return false;
  }
  if (t.elem != "f32") {
    err = format_error(p.source_name, op.loc,
                       pre + what + " must have f32 elements, but has element type '" + t.elem + "'");
    return false;
  }
  return true;
}

bool verify_op(const Program &p, const Op &op, std::string &err) {
  const std::string pre = "'tforge." + op.name + "' op ";
  auto E = [&](const std::string &m) {
    err = format_error(p.source_name, op.loc, pre + m);
    return false;
  };
  // ODS operand constraint (AnyTensor) comes before the C++ verifier.
  for (size_t k = 0; k < op.operand_types.size(); ++k)
    if (!op.operand_types[k].is_tensor)
      return E("operand #" + std::to_string(k) + " must be tensor of any non-token type values, but got '" +
               op.operand_types[k].text + "'");
  if (!op.result_type.is_tensor)
    return E("result #0 must be tensor of any non-token type values, but got '" + op.result_type.text + "'");
  const Type &r = op.result_type;
  if (op.name == "add") {
    const Type &l = op.operand_types[0], &rh = op.operand_types[1];
    if (!check_tensor(p, op, l, "lhs", err) || !check_tensor(p, op, rh, "rhs", err) ||
        !check_tensor(p, op, r, "result", err))
      return false;
    if (l.shape != rh.shape)
      return E("operand shapes must match (no implicit broadcasting): lhs is " + shape_str(l.shape) +
               ", rhs is " + shape_str(rh.shape));
    if (r.shape != l.shape)
      return E("result shape " + shape_str(r.shape) + " does not match operand shape " + shape_str(l.shape));
    return true;
  }
  if (op.name == "relu") {
    const Type &in = op.operand_types[0];
    if (!check_tensor(p, op, in, "input", err) || !check_tensor(p, op, r, "result", err)) return false;
    if (r.shape != in.shape)
      return E("result shape " + shape_str(r.shape) + " does not match input shape " + shape_str(in.shape));
    return true;
  }
  if (op.name == "matmul") {
    const Type &l = op.operand_types[0], &rh = op.operand_types[1];
    if (!check_tensor(p, op, l, "lhs", err) || !check_tensor(p, op, rh, "rhs", err) ||
        !check_tensor(p, op, r, "result", err))
      return false;
    if (l.shape.size() != 2) return E("lhs must be rank 2 (M x K), but has rank " + std::to_string(l.shape.size()));
    if (rh.shape.size() != 2) return E("rhs must be rank 2 (K x N), but has rank " + std::to_string(rh.shape.size()));
    if (r.shape.size() != 2)
      return E("result must be rank 2 (M x N), but has rank " + std::to_string(r.shape.size()));
    const int64_t m = l.shape[0], kl = l.shape[1], kr = rh.shape[0], n = rh.shape[1];
    if (kl != kr)
      return E("contracting dimensions do not match: lhs is " + shape_str(l.shape) + " (K = " + std::to_string(kl) +
               "), rhs is " + shape_str(rh.shape) + " (K = " + std::to_string(kr) + ")");
    if (r.shape[0] != m || r.shape[1] != n)
      return E("result shape must be " + std::to_string(m) + "x" + std::to_string(n) + " (M x N), but got " +
               shape_str(r.shape));
    return true;
  }
  // bias_add
  const Type &in = op.operand_types[0], &bias = op.operand_types[1];
  if (!check_tensor(p, op, in, "input", err) || !check_tensor(p, op, bias, "bias", err) ||
      !check_tensor(p, op, r, "result", err))
    return false;
  if (in.shape.empty()) return E("input must have rank >= 1, but is a scalar");
  if (bias.shape.size() != 1) return E("bias must be rank 1, but has rank " + std::to_string(bias.shape.size()));
  const int64_t last = in.shape.back();
  if (bias.shape[0] != last)
    return E("bias length " + std::to_string(bias.shape[0]) + " does not match the last dimension of input " +
             shape_str(in.shape) + " (" + std::to_string(last) + ")");
  if (r.shape != in.shape)
    return E("result shape " + shape_str(r.shape) + " does not match input shape " + shape_str(in.shape));
  return true;
}

}  // namespace

bool verify_program(const Program &p, std::string &err) {
  std::map<std::string, Type> env;
  for (size_t i = 0; i < p.arg_names.size(); ++i) {
    if (env.count(p.arg_names[i])) {
      err = format_error(p.source_name, p.func_loc, "redefinition of SSA value '" + p.arg_names[i] + "'");
      return false;
    }
    env[p.arg_names[i]] = p.arg_types[i];
  }
  for (const Op &op : p.ops) {
    for (size_t k = 0; k < op.operands.size(); ++k) {
      auto it = env.find(op.operands[k]);
      if (it == env.end()) {
        err = format_error(p.source_name, op.loc, "use of undeclared SSA value name '" + op.operands[k] + "'");
        return false;
      }
      if (it->second.text != op.operand_types[k].text) {
        err = format_error(p.source_name, op.loc,
                           "use of value '" + op.operands[k] + "' expects different type than prior uses: '" +
                               op.operand_types[k].text + "' vs '" + it->second.text + "'");
        return false;
      }
    }
    if (!verify_op(p, op, err)) return false;
    if (env.count(op.result)) {
      err = format_error(p.source_name, op.loc, "redefinition of SSA value '" + op.result + "'");
      return false;
    }
    env[op.result] = op.result_type;
  }
  if (!p.has_return) {
    err = format_error(p.source_name, p.func_loc, "'func.func' op body must end with 'return'");
    return false;
  }
  if (p.ret_value.empty()) {
    if (!p.result_types.empty()) {
      err = format_error(p.source_name, p.ret_loc, "'func.return' op has 0 operands, but enclosing function returns " +
                                                       std::to_string(p.result_types.size()));
      return false;
    }
    return true;
  }
  auto it = env.find(p.ret_value);
  if (it == env.end()) {
    err = format_error(p.source_name, p.ret_loc, "use of undeclared SSA value name '" + p.ret_value + "'");
    return false;
  }
  if (p.result_types.size() != 1 || p.result_types[0].text != p.ret_type.text || it->second.text != p.ret_type.text) {
    err = format_error(p.source_name, p.ret_loc, "'func.return' op type of return operand 0 ('" + p.ret_type.text +
                                                     "') doesn't match function result type");
    return false;
  }
  return true;
}

// --------------------------------------------------------------- options ---

namespace {

bool parse_bool(const std::string &v, bool &out) {
  if (v == "1" || v == "true" || v == "TRUE" || v == "True") {
    out = true;
    return true;
  }
  if (v == "0" || v == "false" || v == "FALSE" || v == "False") {
    out = false;
    return true;
  }
  return false;
}

bool parse_int(const std::string &v, int64_t &out) {
  if (v.empty()) return false;
  size_t pos = 0;
  try {
    out = std::stoll(v, &pos, 0);
  } catch (...) {
    return false;
  }
  return pos == v.size();
}

bool parse_list(const std::string &v, std::vector<int64_t> &out) {
  out.clear();
  std::string item;
  std::stringstream ss(v);
  while (std::getline(ss, item, ',')) {
    int64_t x;
    if (!parse_int(item, x)) return false;
    out.push_back(x);
  }
  return !out.empty();
}

}  // namespace

bool parse_options(const std::string &text, Options &o, std::string &err) {
  o = Options();
  std::string s = text;
  // Accept the option string with or without surrounding braces.
  size_t a = s.find_first_not_of(" \t\n"), b = s.find_last_not_of(" \t\n");
  if (a != std::string::npos && s[a] == '{' && s[b] == '}') s = s.substr(a + 1, b - a - 1);
  std::stringstream ss(s);
  std::string tok;
  const std::string pipe = "tforge-gpu-pipeline: ";
  while (ss >> tok) {
    size_t eq = tok.find('=');
    std::string key = tok.substr(0, eq), val = eq == std::string::npos ? "" : tok.substr(eq + 1);
    bool bval = true;
    auto want_bool = [&](bool &dst) {
      if (eq != std::string::npos && !parse_bool(val, bval)) {
        err = pipe + "invalid value '" + val + "' for boolean option '" + key + "'";
        return false;
      }
      dst = bval;
      return true;
    };
    if (key == "fuse-elementwise") {
      if (!want_bool(o.fuse_elementwise)) return false;
    } else if (key == "promote") {
      if (!want_bool(o.promote)) return false;
    } else if (key == "vectorize") {
      if (!want_bool(o.vectorize)) return false;
    } else if (key == "print-after-each") {
      if (!want_bool(o.print_after_each)) return false;
    } else if (key == "print-script") {
      if (!want_bool(o.print_script)) return false;
    } else if (key == "xcd-swizzle") {
      if (!want_bool(o.xcd_swizzle)) return false;
    } else if (key == "mask-edges") {
      if (!want_bool(o.mask_edges)) return false;
    } else if (key == "wave-split-k") {
      if (!want_bool(o.wave_split_k)) return false;
    } else if (key == "block-tile" || key == "thread-tile") {
      std::vector<int64_t> &dst = key == "block-tile" ? o.block_tile : o.thread_tile;
      if (!parse_list(val, dst)) {
        err = pipe + "invalid value '" + val + "' for list option '" + key + "'";
        return false;
      }
    } else if (key == "split-k") {
      if (!parse_int(val, o.split_k) || o.split_k < 1 || o.split_k > 64) {
        err = pipe + "invalid value '" + val + "' for option 'split-k' (1 to 64)";
        return false;
      }
    } else if (key == "tile-k") {
      if (!parse_int(val, o.tile_k) || o.tile_k < 0) {
        err = pipe + "invalid value '" + val + "' for option 'tile-k'";
        return false;
      }
    } else {
      err = pipe + "no such option " + key;
      return false;
    }
  }
  std::vector<int64_t> bt = o.block_tile.empty() ? std::vector<int64_t>{16, 16} : o.block_tile;
  std::vector<int64_t> tt = o.thread_tile.empty() ? std::vector<int64_t>{1, 1} : o.thread_tile;
  if (bt.size() != 2 || tt.size() != 2 || tt[0] <= 0 || tt[1] <= 0 || bt[0] <= 0 || bt[1] <= 0 ||
      bt[0] % tt[0] || bt[1] % tt[1]) {
    err = "tforge-gpu-pipeline: block-tile and thread-tile need 2 values each, block a multiple of thread";
    return false;
  }
  o.bm = bt[0];
  o.bn = bt[1];
  o.tm = tt[0];
  o.tn = tt[1];
  o.align_vectors = o.vectorize && o.tile_k > 0 && o.tile_k % 4 == 0 && o.bn % 4 == 0 && o.tn % 4 == 0;
  return true;
}

// ------------------------------------------------------------------ plan ---

bool plan_program(const Program &p, const Options &o, Plan &plan, std::string &err) {
  plan = Plan();
  plan.nargs = (int)p.arg_names.size();
  std::map<std::string, int> buf_of;  // materialized values -> buffer id
  for (int i = 0; i < plan.nargs; ++i) {
    Buffer b;
    b.name = p.arg_names[i];
    b.role = BUF_INPUT;
    b.shape = p.arg_types[i].shape;
    plan.buffers.push_back(b);
    buf_of[p.arg_names[i]] = i;
  }
  if (p.ret_value.empty()) {
    err = format_error(p.source_name, p.ret_loc, "tforge-gpu-pipeline: the entry function must return a tensor");
    return false;
  }
  if (buf_of.count(p.ret_value)) {
    err = format_error(p.source_name, p.ret_loc, "tforge-gpu-pipeline: returning an argument needs no kernel");
    return false;
  }
  {
    Buffer out;
    out.name = p.ret_value;
    out.role = BUF_OUTPUT;
    out.shape = p.ret_type.shape;
    plan.buffers.push_back(out);
  }
  std::map<std::string, int> uses;
  for (const Op &op : p.ops)
    for (const std::string &v : op.operands) ++uses[v];
  ++uses[p.ret_value];

  bool has_matmul = false;
  for (const Op &op : p.ops) has_matmul |= op.name == "matmul";
  if (o.tile_k > 0 && !has_matmul) {
    err = format_error(p.source_name, p.func_loc, "tforge-gpu-tile: tile-k needs a matmul");
    return false;
  }

  int open = -1;              // index of the open stage
  std::string open_value;     // SSA value the open stage currently produces
  auto close = [&]() {
    if (open < 0) return;
    Stage &st = plan.stages[open];
    if (open_value == p.ret_value) {
      st.out = plan.nargs;
    } else {
      Buffer b;
      b.name = open_value;
      b.role = BUF_INTERMEDIATE;
      b.shape = st.kind == STAGE_GEMM ? std::vector<int64_t>{st.M, st.N}
                                      : plan.buffers[st.x].shape;
      st.out = (int)plan.buffers.size();
      plan.buffers.push_back(b);
    }
    buf_of[open_value] = st.out;
    open = -1;
    open_value.clear();
  };
  auto materialized = [&](const Op &op, const std::string &v, int &id) {
    auto it = buf_of.find(v);
    if (it == buf_of.end()) {
      err = format_error(p.source_name, op.loc,
                         "tforge-gpu-pipeline: operand " + v + " is produced inside the fused chain it feeds; "
                         "this program needs more than one pass over the same kernel");
      return false;
    }
    id = it->second;
    return true;
  };
  auto flat2d = [](const std::vector<int64_t> &s, int64_t &m, int64_t &n) {
    n = s.empty() ? 1 : s.back();
    m = s.empty() ? 1 : product(s, s.size() - 1);
  };

  for (const Op &op : p.ops) {
    if (op.name == "matmul") {
      close();
      Stage st;
      st.kind = STAGE_GEMM;
      if (!materialized(op, op.operands[0], st.a) || !materialized(op, op.operands[1], st.b)) return false;
      st.M = op.operand_types[0].shape[0];
      st.K = op.operand_types[0].shape[1];
      st.N = op.operand_types[1].shape[1];
      st.ops = "matmul";
      st.loc = op.loc;
      if (o.tile_k > 0 && !o.mask_edges && (st.M % o.bm || st.N % o.bn || st.K % o.tile_k)) {
        err = format_error(p.source_name, op.loc,
                           "tforge-gpu-tile: tile-k needs static tiles; pad the problem to multiples of the block "
                           "and K tiles");
        return false;
      }
      plan.stages.push_back(st);
      open = (int)plan.stages.size() - 1;
      open_value = op.result;
      continue;
    }
    // Element op: fuse into the open stage when it consumes that stage's
    // single-use result (the in-place epilogue rule), else start a stage.
    const bool self_add = op.name == "add" && op.operands[0] == op.operands[1];
    int main_idx = 0;
    if (op.name == "add" && open >= 0 && op.operands[1] == open_value && op.operands[0] != open_value) main_idx = 1;
    const std::string &main = op.operands[main_idx];
    const bool fusible = o.fuse_elementwise && open >= 0 && main == open_value &&
                         uses[open_value] == (self_add ? 2 : 1) &&
                         (int)plan.stages[open].epi.size() < tfk::kMaxEpi;
    if (!fusible) {
      close();
      Stage st;
      st.kind = STAGE_ELEMENTWISE;
      if (!materialized(op, main, st.x)) return false;
      flat2d(op.operand_types[main_idx].shape, st.M, st.N);
      st.loc = op.loc;
      plan.stages.push_back(st);
      open = (int)plan.stages.size() - 1;
    }
    Stage &st = plan.stages[open];
    EpiOp e{tfk::EPI_NONE, -1};
    if (op.name == "relu") {
      // relu(relu(x)) == relu(x) bit for bit (lib/Dialect/TForge/TForgeFolders.cpp,
      // ReluOp::fold: relu's results are NaN or >= +0.0, fixed points of maximum(., +0.0)).
      if (!st.epi.empty() && st.epi.back().kind == tfk::EPI_RELU) {
        open_value = op.result;
        continue;
      }
      e.kind = tfk::EPI_RELU;
    } else if (op.name == "bias_add") {
      e.kind = tfk::EPI_BIAS;
      if (!materialized(op, op.operands[1], e.buf)) return false;
    } else if (self_add) {
      e.kind = tfk::EPI_ADD_SELF;
    } else {
      e.kind = tfk::EPI_ADD;
      if (!materialized(op, op.operands[1 - main_idx], e.buf)) return false;
      int64_t m, n;
      flat2d(op.operand_types[1 - main_idx].shape, m, n);
      if (m != st.M || n != st.N) {
        err = format_error(p.source_name, op.loc, "tforge-gpu-pipeline: add operand shape does not match");
        return false;
      }
    }
    st.epi.push_back(e);
    st.ops += (st.ops.empty() ? "" : "+") + op.name;
    open_value = op.result;
  }
  if (open_value != p.ret_value) {
    err = format_error(p.source_name, p.ret_loc,
                       "tforge-gpu-pipeline: the returned value must be produced by the last operation");
    return false;
  }
  close();
  // The kernels take M, N and K as 32-bit integers (offsets are 64-bit, so a
  // matrix may still hold more than 2^31 elements).
  for (const Stage &st : plan.stages)
    if (st.M > INT32_MAX || st.N > INT32_MAX || st.K > INT32_MAX) {
      err = format_error(p.source_name, st.loc,
                         "tforge-gpu-pipeline: dimensions above 2^31 - 1 are not supported (M = " +
                             std::to_string(st.M) + ", N = " + std::to_string(st.N) + ", K = " +
                             std::to_string(st.K) + ")");
      return false;
    }
  return true;
}

}  // namespace tff
