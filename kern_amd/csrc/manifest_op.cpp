// Manifest-op runner of the C ABI (include/kern_amd.h, kern_op_*): runs one kern manifest op whose
// `impl` points at a gfx950 module, from the op's own JSON.
//
// The op object is the value of one `ops` entry of a kern manifest (crates/kern-manifest/src/types.rs):
//   {"params": ["in buffer<u8>", ..., "i32"],                       interface (types.rs:846-958)
//    "impl": {"launches": [{"module", "entry", "params"?, "block", "grid", "shared_mem"?, "when"?,
//                           "args"?}, ...]}}                          (types.rs:1002-1040)
// Grid and shared_mem are Expr trees over manifest vars (types.rs:1517-1576); args are LaunchArg
// (types.rs:1174-1191) with packs of Fields (types.rs:1193-1260). The checks at create follow the
// reference verifier (verify.rs:655-700): args match the launch params in count; a forwarded interface
// param matches its launch param in kind and dtype; no launch writes through an `in` param or reads an
// `out` param before a launch wrote it; a pack fills exactly its bytes<n>. The launch params are then
// checked against the code object's own kernel-argument sizes (compile.rs:385-415 does this with
// cuFuncGetParamInfo). What a gfx950 module has no use for (extern launches, scratch buffers, rank
// args, TMA descriptors, clusters, programmatic dependent launch) is rejected, not ignored.
#include <hip/hip_runtime.h>

#include <cerrno>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <map>
#include <memory>
#include <string>
#include <vector>

#include "../../include/kern_amd.h"
#include "json.h"

// error reporting of capi.cpp (same thread-local message)
int kern_amd_fail(int code, const char* fmt, ...);

namespace {

using kern_json::JVal;
using kern_json::parse_json;

// ------------------------------------------------------------------------------------ op model
struct ParamT {
  enum Kind { Buf, Scalar, Bytes } kind = Scalar;
  enum Dir { In, Out, InOut } dir = In;
  std::string dtype;  // buffer element type or scalar type (i32, i64, f32, u8)
  uint32_t size = 0;  // kernel-argument bytes
  uint32_t align = 1;
  std::string text;
};

bool parse_param(const std::string& s, ParamT& t, std::string& err) {
  t.text = s;
  if (s == "i32" || s == "f32") {
    t.kind = ParamT::Scalar, t.dtype = s, t.size = t.align = 4;
    return true;
  }
  if (s == "i64") {
    t.kind = ParamT::Scalar, t.dtype = s, t.size = t.align = 8;
    return true;
  }
  if (s == "u8") {
    t.kind = ParamT::Scalar, t.dtype = s, t.size = t.align = 1;
    return true;
  }
  if (s.rfind("bytes<", 0) == 0 && s.back() == '>') {
    long n = strtol(s.c_str() + 6, nullptr, 10);
    if (n <= 0 || n > 4096) {
      err = "bad bytes<n> `" + s + "`";
      return false;
    }
    t.kind = ParamT::Bytes, t.size = (uint32_t)n;
    t.align = (n == 1 || n == 2 || n == 4 || n == 8) ? (uint32_t)n : 8;
    return true;
  }
  size_t sp = s.find(' ');
  if (sp != std::string::npos) {
    std::string d = s.substr(0, sp), rest = s.substr(sp + 1);
    if (d == "in" || d == "out" || d == "inout") {
      t.dir = d == "in" ? ParamT::In : d == "out" ? ParamT::Out : ParamT::InOut;
      if (rest == "state") {
        err = "state param `" + s + "`: this runtime serves no state buffers";
        return false;
      }
      if (rest.rfind("buffer<", 0) == 0 && rest.back() == '>') {
        static const char* dts[] = {"bf16", "f16", "f32", "fp8e4m3", "fp8e8m0", "i8", "i32", "u32", "i64", "u64", "u8"};
        t.dtype = rest.substr(7, rest.size() - 8);
        bool ok = false;
        for (auto dt : dts) ok |= t.dtype == dt;
        if (!ok) {
          err = "unknown dtype in `" + s + "`";
          return false;
        }
        t.kind = ParamT::Buf, t.size = t.align = 8;
        return true;
      }
    }
  }
  err = "unknown param type `" + s + "`";
  return false;
}

struct Expr {
  enum Kind { Const, Var, CeilDiv, Mul, Add, Clamp } kind = Const;
  uint64_t c = 0, c2 = 0;
  std::string var;
  std::unique_ptr<Expr> a, b;
};

bool parse_expr(const JVal& v, Expr& e, std::string& err) {
  if (v.kind == JVal::Int && v.i >= 0) {
    e.kind = Expr::Const, e.c = v.u;
    return true;
  }
  if (v.kind == JVal::Str) {
    e.kind = Expr::Var, e.var = v.s;
    return true;
  }
  auto uconst = [&](const JVal& x, uint64_t& out) {
    if (x.kind != JVal::Int || (x.i < 0 && !x.is_u64)) return false;
    out = x.u;
    return true;
  };
  if (v.kind == JVal::Obj && v.o.size() == 1) {
    const std::string& k = v.o[0].first;
    const JVal& arr = v.o[0].second;
    if (arr.kind == JVal::Arr) {
      if ((k == "ceil_div" || k == "mul") && arr.a.size() == 2) {
        e.kind = k == "mul" ? Expr::Mul : Expr::CeilDiv;
        e.a.reset(new Expr);
        if (!parse_expr(arr.a[0], *e.a, err)) return false;
        if (!uconst(arr.a[1], e.c)) {
          err = k + ": second operand must be a constant";
          return false;
        }
        return true;
      }
      if (k == "add" && arr.a.size() == 2) {
        e.kind = Expr::Add;
        e.a.reset(new Expr);
        e.b.reset(new Expr);
        return parse_expr(arr.a[0], *e.a, err) && parse_expr(arr.a[1], *e.b, err);
      }
      if (k == "clamp" && arr.a.size() == 3) {
        e.kind = Expr::Clamp;
        e.a.reset(new Expr);
        if (!parse_expr(arr.a[0], *e.a, err)) return false;
        if (!uconst(arr.a[1], e.c) || !uconst(arr.a[2], e.c2)) {
          err = "clamp: start and len must be constants";
          return false;
        }
        return true;
      }
    }
  }
  err = "bad expression (a constant, a var name, ceil_div, mul, add or clamp)";
  return false;
}

typedef std::map<std::string, uint64_t> Vars;

// Expr::eval (types.rs:1560-1576): checked arithmetic, unknown vars are errors
bool eval_expr(const Expr& e, const Vars& vars, uint64_t& out, std::string& err) {
  uint64_t x = 0, y = 0;
  switch (e.kind) {
    case Expr::Const: out = e.c; return true;
    case Expr::Var: {
      auto it = vars.find(e.var);
      if (it == vars.end()) {
        err = "unknown var `" + e.var + "`";
        return false;
      }
      out = it->second;
      return true;
    }
    case Expr::CeilDiv:
      if (!eval_expr(*e.a, vars, x, err)) return false;
      if (e.c == 0) {
        err = "division by zero";
        return false;
      }
      if (x > UINT64_MAX - (e.c - 1)) {
        err = "arithmetic overflow";
        return false;
      }
      out = (x + e.c - 1) / e.c;
      return true;
    case Expr::Mul:
      if (!eval_expr(*e.a, vars, x, err)) return false;
      if (e.c && x > UINT64_MAX / e.c) {
        err = "arithmetic overflow";
        return false;
      }
      out = x * e.c;
      return true;
    case Expr::Add:
      if (!eval_expr(*e.a, vars, x, err) || !eval_expr(*e.b, vars, y, err)) return false;
      if (x > UINT64_MAX - y) {
        err = "arithmetic overflow";
        return false;
      }
      out = x + y;
      return true;
    case Expr::Clamp:
      if (!eval_expr(*e.a, vars, x, err)) return false;
      x = x > e.c ? x - e.c : 0;
      out = x < e.c2 ? x : e.c2;
      return true;
  }
  return false;
}

// a value source: an op param, a literal or (in packs) a var / expression
struct Src {
  enum Kind { Param, I32, I64, F32, U8, Var, ExprK } kind = I32;
  int param = 0;
  int64_t iv = 0;
  float fv = 0;
  std::string var;
  std::shared_ptr<Expr> expr;
};

bool parse_src(const JVal& v, bool in_pack, Src& s, std::string& err) {
  if (v.kind != JVal::Obj) {
    err = "an arg must be an object";
    return false;
  }
  auto one = [&](const char* key) { return v.get(key); };
  const JVal* x;
  if ((x = one("param"))) {
    if (x->kind != JVal::Int || x->i < 0) return err = "param index must be a non-negative integer", false;
    s.kind = Src::Param, s.param = (int)x->i;
  } else if ((x = one("i32"))) {
    if (x->kind != JVal::Int || x->i < INT32_MIN || x->i > INT32_MAX) return err = "i32 literal out of range", false;
    s.kind = Src::I32, s.iv = x->i;
  } else if ((x = one("i64"))) {
    if (x->kind != JVal::Int || x->is_u64) return err = "i64 literal out of range", false;
    s.kind = Src::I64, s.iv = x->i;
  } else if ((x = one("f32"))) {
    if (!x->is_num()) return err = "f32 literal must be a number", false;
    s.kind = Src::F32, s.fv = (float)x->f;
  } else if ((x = one("u8"))) {
    if (x->kind != JVal::Int || x->i < 0 || x->i > 255) return err = "u8 literal out of range", false;
    s.kind = Src::U8, s.iv = x->i;
  } else if (in_pack && (x = one("var"))) {
    if (x->kind != JVal::Str) return err = "var must be a name", false;
    s.kind = Src::Var, s.var = x->s;
  } else if (in_pack && (x = one("expr"))) {
    s.kind = Src::ExprK;
    s.expr = std::make_shared<Expr>();
    if (!parse_expr(*x, *s.expr, err)) return false;
  } else if (one("scratch")) {
    return err = "scratch buffers are not served by this runtime", false;
  } else if (one("rank")) {
    return err = "rank args are not served by this runtime (one GPU)", false;
  } else if (one("tensormap")) {
    return err = "TMA descriptors have no gfx950 counterpart", false;
  } else {
    return err = "unknown arg source", false;
  }
  // nothing else may sit beside the source (serde deny_unknown_fields)
  size_t extra = v.o.size() - 1 - (in_pack ? (v.get("at") ? 1 : 0) + (v.get("width") ? 1 : 0) : 0);
  if (extra) return err = "unexpected keys beside the arg source", false;
  return true;
}

struct Field {
  uint32_t at = 0, width = 0;  // width 0: the source's own
  Src src;
};

struct Arg {
  bool is_pack = false;
  Src src;
  uint32_t pack_size = 0;
  std::vector<Field> fields;
};

struct Launch {
  std::string module, entry;
  std::vector<ParamT> params;  // the launch ABI
  uint32_t block[3] = {1, 1, 1};
  Expr grid[3];
  bool has_shared = false;
  Expr shared;
  bool has_when = false;
  std::string when_var;
  bool has_min = false, has_max = false;
  uint64_t wmin = 0, wmax = 0;
  std::vector<Arg> args;
  kern_function fn = nullptr;
  std::vector<uint32_t> offsets;  // kernarg offsets from the code object (empty: natural alignment)
};

}  // namespace

struct kern_op_s {
  std::vector<ParamT> params;
  std::vector<Launch> launches;
};

namespace {

// The blocks kern_mx's entries are written for: their mapping of threads to work assumes these shapes (a
// block of 256 lanes, the 8 waves of a GEMM workgroup with their roles, a 1024-lane routing workgroup), so a
// launch with another block would compute something else without an error. Each needs block [x, 1, 1] with x
// exactly the given count, or, where `per_wave`, any whole number of waves up to it. Entries of other modules
// are not named here and are not checked.
struct BlockRule {
  const char* name;
  bool prefix;  // the rule covers a family of instances (name followed by their suffix)
  uint32_t x;
  bool per_wave;
};
const BlockRule kBlockRules[] = {
    {"kern_mx_quant_bf16", false, 256, false},      {"kern_mx_quant_f32", false, 256, false},
    {"kern_mx_w_shuffle", false, 256, false},       {"kern_mx_sf_shuffle", false, 256, false},
    {"kern_mx_gemv_bf16", false, 256, false},       {"kern_mx_gemv_bf16_rg", false, 256, false},
    {"kern_mx_gemv_bf16_r", true, 256, false},      {"kern_mx_gemv_bf16_p", true, 512, false},
    {"kern_mx_gemm_bf16_s", true, 512, false},      {"kern_mx_gemm_bf16", false, 512, false},
    {"kern_mx_gemm_e4m3", false, 512, false},       {"kern_mx_gemm_mxfp8", false, 512, false},
    {"kern_mx_bmm_fc1", false, 512, false},         {"kern_mx_bmm_fc2", false, 512, false},
    {"kern_mx_routing", false, 1024, false},        {"kern_mx_routing_count", false, 1024, false},
    {"kern_mx_routing_scan", false, 1024, false},   {"kern_mx_routing_rank", false, 1024, false},
    {"kern_mx_quant_routing", false, 1024, false},  {"kern_silu_mul_bf16", false, 256, false},
    {"kern_mx_moe_finalize", false, 256, false},    {"kern_mx_fill_random_u8", false, 256, false},
    {"kern_mx_moe_finalize_rms", false, 1024, true},
};

// "" when the block suits the entry (or the entry has no rule), else the reason
std::string block_rule_error(const std::string& entry, const uint32_t block[3]) {
  const BlockRule* hit = nullptr;
  for (const BlockRule& r : kBlockRules) {
    const size_t n = strlen(r.name);
    const bool match = r.prefix ? entry.size() > n && entry.compare(0, n, r.name) == 0 && entry != "kern_mx_gemv_bf16_rg"
                                : entry == r.name;
    if (match) hit = &r;
  }
  if (!hit) return "";
  const uint32_t x = block[0];
  const bool ok = block[1] == 1 && block[2] == 1 && (hit->per_wave ? x % 64 == 0 && x <= hit->x : x == hit->x);
  if (ok) return "";
  return "`" + entry + "` is written for block " +
         (hit->per_wave ? "[64·n, 1, 1] with 64·n <= " + std::to_string(hit->x) : "[" + std::to_string(hit->x) + ", 1, 1]") +
         ", not [" + std::to_string(block[0]) + ", " + std::to_string(block[1]) + ", " + std::to_string(block[2]) + "]";
}

bool parse_op(const char* json, kern_op_s& op, std::string& err) {
  JVal root;
  if (!parse_json(json, root, err)) return err = "op JSON: " + err, false;
  if (root.kind != JVal::Obj) return err = "op JSON: expected an object", false;
  const JVal* ps = root.get("params");
  if (!ps || ps->kind != JVal::Arr) return err = "op: missing `params` list", false;
  for (size_t i = 0; i < ps->a.size(); ++i) {
    ParamT t;
    if (ps->a[i].kind != JVal::Str || !parse_param(ps->a[i].s, t, err))
      return err = "op param #" + std::to_string(i) + ": " + (err.empty() ? "expected a string" : err), false;
    if (t.kind == ParamT::Bytes) return err = "op param #" + std::to_string(i) + ": bytes<n> is launch-private", false;
    op.params.push_back(t);
  }
  const JVal* impl = root.get("impl");
  const JVal* ls = impl ? impl->get("launches") : nullptr;
  if (!ls || ls->kind != JVal::Arr || ls->a.empty()) return err = "op: missing `impl.launches`", false;
  if (impl->get("scratch")) return err = "op impl: scratch buffers are not served by this runtime", false;
  std::vector<bool> written(op.params.size(), false);
  for (size_t li = 0; li < ls->a.size(); ++li) {
    const JVal& L = ls->a[li];
    const std::string ctx = "launch #" + std::to_string(li);
    Launch l;
    if (L.kind != JVal::Obj) return err = ctx + ": expected an object", false;
    static const char* known[] = {"module", "entry", "params", "block", "grid", "shared_mem", "cluster", "pdl",
                                  "when", "args", "algo"};
    for (auto& kv : L.o) {
      bool ok = false;
      for (auto k : known) ok |= kv.first == k;
      if (!ok) return err = ctx + ": unknown key `" + kv.first + "`", false;
    }
    const JVal* m = L.get("module");
    const JVal* e = L.get("entry");
    if (!e || e->kind != JVal::Str) return err = ctx + ": missing `entry`", false;
    if (!m) {
      return err = ctx + ": extern launch `" + e->s + "` has no gfx950 counterpart in this runtime", false;
    }
    if (m->kind != JVal::Str) return err = ctx + ": `module` must be a name", false;
    l.module = m->s, l.entry = e->s;
    if (L.get("cluster")) return err = ctx + ": thread-block clusters have no gfx950 counterpart", false;
    if (const JVal* pdl = L.get("pdl"); pdl && !(pdl->kind == JVal::Bool && !pdl->b))
      return err = ctx + ": programmatic dependent launch is not served by this runtime", false;
    if (L.get("algo")) return err = ctx + ": `algo` belongs to extern launches", false;
    if (const JVal* lp = L.get("params")) {
      if (lp->kind != JVal::Arr) return err = ctx + ": `params` must be a list", false;
      for (size_t i = 0; i < lp->a.size(); ++i) {
        ParamT t;
        if (lp->a[i].kind != JVal::Str || !parse_param(lp->a[i].s, t, err))
          return err = ctx + ": param #" + std::to_string(i) + ": " + (err.empty() ? "expected a string" : err), false;
        l.params.push_back(t);
      }
    } else {
      l.params = op.params;
    }
    const JVal* b = L.get("block");
    if (!b || b->kind != JVal::Arr || b->a.size() != 3) return err = ctx + ": `block` must be [x, y, z]", false;
    uint64_t threads = 1;
    for (int i = 0; i < 3; ++i) {
      if (b->a[i].kind != JVal::Int || b->a[i].i <= 0 || b->a[i].i > 1024)
        return err = ctx + ": block dims must be 1..1024", false;
      l.block[i] = (uint32_t)b->a[i].i;
      threads *= l.block[i];
    }
    if (threads > 1024) return err = ctx + ": block exceeds 1024 threads (gfx950)", false;
    if (const std::string why = block_rule_error(l.entry, l.block); !why.empty()) return err = ctx + ": " + why, false;
    const JVal* g = L.get("grid");
    if (!g || g->kind != JVal::Arr || g->a.size() != 3) return err = ctx + ": `grid` must be [x, y, z]", false;
    for (int i = 0; i < 3; ++i)
      if (!parse_expr(g->a[i], l.grid[i], err)) return err = ctx + ": grid." + "xyz"[i] + ": " + err, false;
    if (const JVal* sm = L.get("shared_mem")) {
      l.has_shared = true;
      if (!parse_expr(*sm, l.shared, err)) return err = ctx + ": shared_mem: " + err, false;
    }
    if (const JVal* w = L.get("when")) {
      const JVal* wv = w->kind == JVal::Obj ? w->get("var") : nullptr;
      if (!wv || wv->kind != JVal::Str) return err = ctx + ": `when` needs a var", false;
      l.has_when = true, l.when_var = wv->s;
      if (const JVal* mn = w->get("min")) {
        if (mn->kind != JVal::Int || mn->i < 0) return err = ctx + ": when.min must be >= 0", false;
        l.has_min = true, l.wmin = mn->u;
      }
      if (const JVal* mx = w->get("max")) {
        if (mx->kind != JVal::Int || mx->i < 0) return err = ctx + ": when.max must be >= 0", false;
        l.has_max = true, l.wmax = mx->u;
      }
    }
    // args: default forwards the op's params in order (types.rs:1160-1167)
    if (const JVal* as = L.get("args")) {
      if (as->kind != JVal::Arr) return err = ctx + ": `args` must be a list", false;
      for (size_t j = 0; j < as->a.size(); ++j) {
        const JVal& A = as->a[j];
        Arg arg;
        const JVal* pk = A.kind == JVal::Obj ? A.get("pack") : nullptr;
        if (pk) {
          arg.is_pack = true;
          const JVal* sz = pk->get("size");
          const JVal* fs = pk->get("fields");
          if (!sz || sz->kind != JVal::Int || sz->i <= 0 || !fs || fs->kind != JVal::Arr)
            return err = ctx + ": arg #" + std::to_string(j) + ": pack needs size and fields", false;
          arg.pack_size = (uint32_t)sz->i;
          for (size_t fi = 0; fi < fs->a.size(); ++fi) {
            const JVal& F = fs->a[fi];
            Field f;
            const JVal* at = F.kind == JVal::Obj ? F.get("at") : nullptr;
            if (!at || at->kind != JVal::Int || at->i < 0)
              return err = ctx + ": arg #" + std::to_string(j) + ": field #" + std::to_string(fi) + " needs `at`", false;
            f.at = (uint32_t)at->i;
            if (const JVal* wd = F.get("width")) {
              if (wd->kind != JVal::Int || !(wd->i == 1 || wd->i == 2 || wd->i == 4 || wd->i == 8))
                return err = ctx + ": arg #" + std::to_string(j) + ": field width must be 1, 2, 4 or 8", false;
              f.width = (uint32_t)wd->i;
            }
            if (!parse_src(F, true, f.src, err))
              return err = ctx + ": arg #" + std::to_string(j) + ": field #" + std::to_string(fi) + ": " + err, false;
            arg.fields.push_back(f);
          }
        } else if (!parse_src(A, false, arg.src, err)) {
          return err = ctx + ": arg #" + std::to_string(j) + ": " + err, false;
        }
        l.args.push_back(arg);
      }
    } else {
      for (size_t i = 0; i < op.params.size(); ++i) {
        Arg arg;
        arg.src.kind = Src::Param, arg.src.param = (int)i;
        l.args.push_back(arg);
      }
    }
    if (l.args.size() != l.params.size())
      return err = ctx + ": takes " + std::to_string(l.params.size()) + " params, got " + std::to_string(l.args.size()) +
                   " args", false;
    // type checks (verify.rs:655-700)
    for (size_t j = 0; j < l.args.size(); ++j) {
      const Arg& a = l.args[j];
      const ParamT& lp = l.params[j];
      const std::string actx = ctx + ": arg #" + std::to_string(j);
      if (a.is_pack) {
        if (lp.kind != ParamT::Bytes || lp.size != a.pack_size)
          return err = actx + ": a pack of " + std::to_string(a.pack_size) + " bytes bound to `" + lp.text + "`", false;
        for (auto& f : a.fields) {
          uint32_t w = f.width;
          if (!w) {
            switch (f.src.kind) {
              case Src::Param:
                if (f.src.param >= (int)op.params.size())
                  return err = actx + ": field param #" + std::to_string(f.src.param) + " out of range", false;
                w = op.params[f.src.param].size;
                break;
              case Src::I64: w = 8; break;
              case Src::U8: w = 1; break;
              default: w = 4; break;
            }
          }
          if (f.src.kind == Src::Param && f.src.param >= (int)op.params.size())
            return err = actx + ": field param #" + std::to_string(f.src.param) + " out of range", false;
          if ((uint64_t)f.at + w > a.pack_size)
            return err = actx + ": field at " + std::to_string(f.at) + " runs past the pack's " +
                         std::to_string(a.pack_size) + " bytes", false;
        }
        continue;
      }
      const Src& s = a.src;
      if (s.kind == Src::Param) {
        if (s.param >= (int)op.params.size())
          return err = actx + ": interface param #" + std::to_string(s.param) + " out of range (" +
                       std::to_string(op.params.size()) + " interface params)", false;
        const ParamT& ip = op.params[s.param];
        const bool compatible = ip.kind == lp.kind && ip.kind != ParamT::Bytes && ip.dtype == lp.dtype;
        if (!compatible)
          return err = actx + ": interface param `" + ip.text + "` does not match launch param `" + lp.text + "`", false;
        if (ip.kind == ParamT::Buf) {
          const bool lwrites = lp.dir != ParamT::In, lreads = lp.dir != ParamT::Out;
          if (lwrites && ip.dir == ParamT::In)
            return err = actx + ": launch writes through interface `in` param #" + std::to_string(s.param), false;
          if (lreads && ip.dir == ParamT::Out && !written[s.param])
            return err = actx + ": interface `out` param #" + std::to_string(s.param) + " read before any launch wrote it",
                   false;
          if (lwrites) written[s.param] = true;
        }
        continue;
      }
      const char* want = s.kind == Src::I32 ? "i32" : s.kind == Src::I64 ? "i64" : s.kind == Src::F32 ? "f32" : "u8";
      if (lp.kind != ParamT::Scalar || lp.dtype != want)
        return err = actx + ": literal " + want + " bound to `" + lp.text + "`", false;
    }
    op.launches.push_back(std::move(l));
  }
  return true;
}

bool eval_vars(const char* const* names, const uint64_t* values, int n, Vars& vars, std::string& err) {
  if (n && (!names || !values)) return err = "null var arrays", false;
  for (int i = 0; i < n; ++i) {
    if (!names[i]) return err = "null var name", false;
    vars[names[i]] = values[i];
  }
  return true;
}

// bytes of one source value (`width` bytes, little-endian)
bool src_bytes(const Src& s, const kern_op_s& op, const uint64_t* params, const Vars& vars, uint32_t width,
               unsigned char* dst, std::string& err) {
  uint64_t v = 0;
  switch (s.kind) {
    case Src::Param: v = params[s.param]; break;
    case Src::I32: v = (uint64_t)(int64_t)(int32_t)s.iv; break;
    case Src::I64: v = (uint64_t)s.iv; break;
    case Src::U8: v = (uint64_t)s.iv; break;
    case Src::F32: {
      uint32_t bits;
      memcpy(&bits, &s.fv, 4);
      v = bits;
      break;
    }
    case Src::Var: {
      auto it = vars.find(s.var);
      if (it == vars.end()) return err = "unknown var `" + s.var + "`", false;
      v = it->second;
      break;
    }
    case Src::ExprK:
      if (!eval_expr(*s.expr, vars, v, err)) return false;
      break;
  }
  (void)op;
  memcpy(dst, &v, width);  // little-endian: the low `width` bytes
  return true;
}

struct Plan {
  bool skip = false;
  uint32_t grid[3] = {0, 0, 0};
  uint32_t shared = 0;
  std::vector<unsigned char> args;
  std::vector<uint32_t> sizes;
  std::vector<size_t> offs;  // each argument's offset in `args`
};

// The LDS-ring GEMM entries of kern_mx address their activations (launch argument 2) by 32-bit byte offsets
// from the buffer's base, so the activations must stay below 4 GiB (the direct C-ABI entries refuse larger
// ones). For each entry: the launch arguments giving the activation rows (times `rows_mul`) and the row
// length k; FC1 gathers token rows through route_map, and no argument carries the token count.
struct RingEntry {
  const char* entry;
  int nargs, rows_arg, rows_mul, k_arg;
};
const RingEntry kRingEntries[] = {
    {"kern_mx_bmm_fc2", 14, 11, 128, 10},   // b [max_slots * 128, k]
    {"kern_mx_gemm_e4m3", 10, 6, 1, 8},     // b [M, k]
    {"kern_mx_gemm_bf16", 9, 5, 1, 7},      // b [M, k]
    {"kern_mx_gemm_bf16_s1", 10, 6, 1, 8},  // xq [M, K]
    {"kern_mx_gemm_bf16_s2", 10, 6, 1, 8},
    {"kern_mx_gemm_bf16_s4", 10, 6, 1, 8},
    {"kern_mx_gemm_bf16_s7", 10, 6, 1, 8},
    {"kern_mx_gemm_bf16_s8", 10, 6, 1, 8},
    {"kern_mx_bmm_fc1", 17, -1, 0, 14},     // b [tokens, k]: bound by the buffer (the program runtime checks it)
};

bool is_ring_entry(const std::string& e) {
  for (const RingEntry& r : kRingEntries)
    if (e == r.entry) return true;
  return false;
}

bool check_ring_extent(const Launch& l, const Plan& pl, std::string& err) {
  for (const RingEntry& r : kRingEntries) {
    if (l.entry != r.entry || r.rows_arg < 0 || (int)pl.offs.size() != r.nargs) continue;
    int32_t rows = 0, k = 0;
    memcpy(&rows, pl.args.data() + pl.offs[r.rows_arg], 4);
    memcpy(&k, pl.args.data() + pl.offs[r.k_arg], 4);
    if ((int64_t)rows * r.rows_mul * k >= ((int64_t)1 << 32))
      return err = "activations of " + std::to_string((int64_t)rows * r.rows_mul) + " rows x " + std::to_string(k) +
                   " bytes reach 4 GiB (the ring addresses them by 32-bit offsets)",
             false;
  }
  return true;
}

bool plan_launch(const kern_op_s& op, const Launch& l, const uint64_t* params, const Vars& vars, Plan& pl,
                 std::string& err) {
  if (l.has_when) {
    auto it = vars.find(l.when_var);
    if (it == vars.end()) return err = "when: unknown var `" + l.when_var + "`", false;
    const uint64_t v = it->second;
    if ((l.has_min && v < l.wmin) || (l.has_max && v > l.wmax)) {
      pl.skip = true;
      return true;
    }
  }
  for (int i = 0; i < 3; ++i) {
    uint64_t g = 0;
    if (!eval_expr(l.grid[i], vars, g, err)) return err = std::string("grid.") + "xyz"[i] + ": " + err, false;
    if (g > (i == 0 ? 0x7fffffffull : 65535ull))
      return err = std::string("grid.") + "xyz"[i] + " = " + std::to_string(g) + " exceeds the launch limit", false;
    pl.grid[i] = (uint32_t)g;
  }
  if (l.has_shared) {
    uint64_t s = 0;
    if (!eval_expr(l.shared, vars, s, err)) return err = "shared_mem: " + err, false;
    if (s > 163840) return err = "shared_mem = " + std::to_string(s) + " exceeds gfx950's 163840 bytes of LDS", false;
    pl.shared = (uint32_t)s;
  }
  // kernarg layout: the code object's offsets, else each argument at its natural alignment
  size_t n = 0;
  for (size_t j = 0; j < l.args.size(); ++j) {
    const ParamT& lp = l.params[j];
    const Arg& a = l.args[j];
    n = l.offsets.empty() ? (n + lp.align - 1) & ~(size_t)(lp.align - 1) : l.offsets[j];
    if (pl.args.size() < n + lp.size) pl.args.resize(n + lp.size, 0);
    if (a.is_pack) {
      for (auto& f : a.fields) {
        uint32_t w = f.width;
        if (!w) w = f.src.kind == Src::Param ? op.params[f.src.param].size
                    : f.src.kind == Src::I64 ? 8 : f.src.kind == Src::U8 ? 1 : 4;
        if (!src_bytes(f.src, op, params, vars, w, pl.args.data() + n + f.at, err))
          return err = "arg #" + std::to_string(j) + ": " + err, false;
      }
    } else if (!src_bytes(a.src, op, params, vars, lp.size, pl.args.data() + n, err)) {
      return err = "arg #" + std::to_string(j) + ": " + err, false;
    }
    pl.sizes.push_back(lp.size);
    pl.offs.push_back(n);
    n += lp.size;
  }
  pl.args.resize((pl.args.size() + 7) & ~(size_t)7, 0);
  return check_ring_extent(l, pl, err);
}

}  // namespace

// The param of the op (its JSON text) that a launch of an LDS-ring GEMM entry takes as its activations
// (launch argument 2, when it forwards a param), or -1: the program runtime holds the buffer bound there
// below 4 GiB.
int kern_op_ring_activation_param(const char* op_json) {
  kern_op_s op;
  std::string err;
  if (!op_json || !parse_op(op_json, op, err)) return -1;
  for (const Launch& l : op.launches)
    if (is_ring_entry(l.entry) && l.args.size() > 2 && !l.args[2].is_pack && l.args[2].src.kind == Src::Param)
      return l.args[2].src.param;
  return -1;
}

extern "C" int kern_op_create(const char* op_json, const char* module_name, kern_module mod, kern_op* out) {
  if (!op_json || !module_name || !mod || !out) return kern_amd_fail(KERN_ERR_API, "kern_op_create: null argument");
  std::unique_ptr<kern_op_s> op(new kern_op_s);
  std::string err;
  if (!parse_op(op_json, *op, err)) return kern_amd_fail(KERN_ERR_MANIFEST, "op: %s", err.c_str());
  for (size_t li = 0; li < op->launches.size(); ++li) {
    Launch& l = op->launches[li];
    if (l.module != module_name)
      return kern_amd_fail(KERN_ERR_MANIFEST, "op launch #%zu names module `%s`; the module bound here is `%s`", li,
                           l.module.c_str(), module_name);
    if (int rc = kern_module_function(mod, l.entry.c_str(), &l.fn))
      return kern_amd_fail(rc, "op launch #%zu: %s", li, kern_last_error());
    std::vector<uint32_t> sizes;
    for (auto& p : l.params) sizes.push_back(p.size);
    if (int rc = kern_function_check_params(l.fn, sizes.data(), (int)sizes.size()))
      return kern_amd_fail(rc, "op launch #%zu: %s", li, kern_last_error());
    int n = 0;
    l.offsets.assign(l.params.size(), 0);
    kern_function_param_offsets(l.fn, l.offsets.data(), (int)l.offsets.size(), &n);
    if (n != (int)l.params.size()) l.offsets.clear();
  }
  *out = op.release();
  return KERN_OK;
}

extern "C" int kern_op_verify(const char* op_json) {
  if (!op_json) return kern_amd_fail(KERN_ERR_API, "kern_op_verify: null op");
  kern_op_s op;
  std::string err;
  if (!parse_op(op_json, op, err)) return kern_amd_fail(KERN_ERR_MANIFEST, "op: %s", err.c_str());
  return KERN_OK;
}

extern "C" int kern_op_destroy(kern_op op) {
  if (!op) return KERN_OK;
  for (auto& l : op->launches) kern_function_release(l.fn);
  delete op;
  return KERN_OK;
}

extern "C" int kern_op_num_params(kern_op op) { return op ? (int)op->params.size() : -1; }

extern "C" int kern_op_num_launches(kern_op op) { return op ? (int)op->launches.size() : -1; }

extern "C" int kern_op_launch(kern_op op, const uint64_t* params, int nparams, const char* const* var_names,
                              const uint64_t* var_values, int nvars, void* stream) {
  if (!op) return kern_amd_fail(KERN_ERR_API, "kern_op_launch: null op");
  if (nparams != (int)op->params.size() || (nparams && !params))
    return kern_amd_fail(KERN_ERR_API, "kern_op_launch: the op takes %zu params, got %d", op->params.size(), nparams);
  for (int i = 0; i < nparams; ++i)
    if (op->params[i].kind == ParamT::Buf && params[i] == 0)
      return kern_amd_fail(KERN_ERR_API, "kern_op_launch: buffer param #%d (`%s`) is null", i,
                           op->params[i].text.c_str());
  Vars vars;
  std::string err;
  if (!eval_vars(var_names, var_values, nvars, vars, err)) return kern_amd_fail(KERN_ERR_API, "kern_op_launch: %s", err.c_str());
  for (size_t li = 0; li < op->launches.size(); ++li) {
    const Launch& l = op->launches[li];
    Plan pl;
    if (!plan_launch(*op, l, params, vars, pl, err))
      return kern_amd_fail(KERN_ERR_CALL, "op launch #%zu (%s): %s", li, l.entry.c_str(), err.c_str());
    if (pl.skip) continue;
    if (kern_launch(l.fn, pl.grid, l.block, pl.shared, stream, pl.args.data(), pl.args.size()) != KERN_OK)
      return kern_amd_fail(KERN_ERR_CALL, "op launch #%zu (%s): %s", li, l.entry.c_str(), kern_last_error());
  }
  return KERN_OK;
}

extern "C" int kern_op_plan(const char* op_json, int launch_index, const uint64_t* params, int nparams,
                            const char* const* var_names, const uint64_t* var_values, int nvars, uint32_t grid[3],
                            uint32_t block[3], uint32_t* shared_bytes, void* kernargs, size_t cap,
                            size_t* kernargs_size, int* skip) {
  if (!op_json || !grid || !block || !shared_bytes || !kernargs_size || !skip)
    return kern_amd_fail(KERN_ERR_API, "kern_op_plan: null argument");
  kern_op_s op;
  std::string err;
  if (!parse_op(op_json, op, err)) return kern_amd_fail(KERN_ERR_MANIFEST, "op: %s", err.c_str());
  if (launch_index < 0 || launch_index >= (int)op.launches.size())
    return kern_amd_fail(KERN_ERR_API, "kern_op_plan: launch #%d out of range (%zu launches)", launch_index,
                         op.launches.size());
  if (nparams != (int)op.params.size() || (nparams && !params))
    return kern_amd_fail(KERN_ERR_API, "kern_op_plan: the op takes %zu params, got %d", op.params.size(), nparams);
  Vars vars;
  if (!eval_vars(var_names, var_values, nvars, vars, err)) return kern_amd_fail(KERN_ERR_API, "kern_op_plan: %s", err.c_str());
  const Launch& l = op.launches[launch_index];
  Plan pl;
  if (!plan_launch(op, l, params, vars, pl, err))
    return kern_amd_fail(KERN_ERR_CALL, "op launch #%d (%s): %s", launch_index, l.entry.c_str(), err.c_str());
  *skip = pl.skip ? 1 : 0;
  for (int i = 0; i < 3; ++i) grid[i] = pl.grid[i], block[i] = l.block[i];
  *shared_bytes = pl.shared;
  *kernargs_size = pl.args.size();
  if (!pl.skip) {
    if (!kernargs || cap < pl.args.size())
      return kern_amd_fail(KERN_ERR_API, "kern_op_plan: the kernel-argument image needs %zu bytes", pl.args.size());
    memcpy(kernargs, pl.args.data(), pl.args.size());
  }
  return KERN_OK;
}
