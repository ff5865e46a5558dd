// Program runtime of the C ABI (include/kern_amd.h, kern_rt_*): loads a kern manifest whose ops point at
// gfx950 modules and runs its programs by name, the analog of crates/kern-runtime's Runtime
// (src/lib.rs:137-236) for this path.
//
// A runtime owns one device, one stream, the manifest's buffers (allocated at their vars' maxima and
// zeroed at load, as compile.rs:289-307 sizes them), its modules (loaded from `kernels_dir` by file name
// and pinned by sha256, cubin.rs:62-109) and its ops (kern_op_* objects, one module per op). Programs are
// straight-line call lists (types.rs:146-161, :1581-1595); a call binds each op param to a buffer (plus a
// byte offset), a var or a literal. A `graph` program is captured at each var assignment it is run with
// and replayed from then on (exec.rs:426-548); `derive` programs turn `source` buffers into the buffers
// the other programs read, once, after which the sources are freed (derive.rs:72-78).
//
// The manifest subset this runtime serves is the one this path needs: no states, topology, peers or
// host-placed weights, one lane per program, and `weight` / `source` buffers filled by name from the
// caller's bytes (kern_rt_load_weight). Two fields are carried without being acted on: a buffer's `bind`
// (the checkpoint tensors the reference's weights loader reads it from, load.rs:336-381; here the caller
// hands over those bytes) and a program's `batch` (the axes the serving batcher fills, which a caller of
// kern_rt_run states as var values). Everything else outside the subset is rejected with
// KERN_ERR_MANIFEST naming what was found, not ignored.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <fstream>
#include <strings.h>
#include <map>
#include <memory>
#include <mutex>
#include <string>
#include <vector>

#include "../../include/kern_amd.h"
#include "json.h"

int kern_amd_fail(int code, const char* fmt, ...);

namespace {

using kern_json::JVal;

enum BufKind { K_INPUT, K_OUTPUT, K_INOUT, K_WEIGHT, K_SOURCE, K_WORKSPACE, K_CARRY };

const char* kind_name(int k) {
  static const char* n[] = {"input", "output", "inout", "weight", "source", "workspace", "carry"};
  return n[k];
}

struct Dim {
  bool is_var = false;
  uint64_t c = 0;
  int var = -1;
};

struct RtBuffer {
  std::string name, dtype;
  std::vector<Dim> shape;
  int kind = K_WORKSPACE;
  size_t bytes = 0;
  void* dev = nullptr;
  void* staging = nullptr;  // pinned host bytes of an input / inout buffer
  bool freed = false;       // a source buffer after derive
};

// one interface param of an op, as a call binds it
struct OpParam {
  bool buf = false;
  int dir = 0;  // 0 in, 1 out, 2 inout
  std::string dtype;  // buffer element type or scalar type
  std::string text;
};

struct RtArg {
  enum Kind { Buf, Var, Lit } kind = Lit;
  int buf = -1;
  uint64_t offset = 0;
  int var = -1;
  uint64_t bits = 0;
};

struct RtCall {
  std::string label;
  int op = -1;
  std::vector<RtArg> args;
};

struct RtProgram {
  std::string name;
  bool graph = false, derive = false, once = false;
  std::vector<RtCall> calls;
};

struct RtOp {
  std::string name;
  kern_op op = nullptr;
  std::vector<OpParam> params;
  int ring_param = -1;  // the param an LDS-ring GEMM launch takes as activations (bound below 4 GiB)
};

size_t dtype_size(const std::string& d) {
  if (d == "bf16" || d == "f16") return 2;
  if (d == "f32" || d == "i32" || d == "u32") return 4;
  if (d == "i64" || d == "u64") return 8;
  if (d == "fp8e4m3" || d == "fp8e8m0" || d == "i8" || d == "u8") return 1;
  return 0;
}

bool parse_op_param(const std::string& s, OpParam& p) {
  p.text = s;
  if (s == "i32" || s == "i64" || s == "f32" || s == "u8") {
    p.buf = false, p.dtype = s;
    return true;
  }
  size_t sp = s.find(' ');
  if (sp == std::string::npos) return false;
  const std::string d = s.substr(0, sp), rest = s.substr(sp + 1);
  if (d != "in" && d != "out" && d != "inout") return false;
  if (rest.rfind("buffer<", 0) != 0 || rest.back() != '>') return false;
  p.buf = true, p.dir = d == "in" ? 0 : d == "out" ? 1 : 2;
  p.dtype = rest.substr(7, rest.size() - 8);
  return dtype_size(p.dtype) > 0;
}

std::mutex g_capture;  // graph capture is serialized process-wide (exec.rs:435-440)

}  // namespace

int kern_op_ring_activation_param(const char* op_json);  // manifest_op.cpp

struct kern_runtime_s {
  int gpu = 0;
  hipStream_t stream = nullptr;
  std::mutex mu;
  std::vector<std::string> var_names;
  std::vector<uint64_t> var_max;
  std::map<std::string, int> var_index;
  std::vector<RtBuffer> buffers;
  std::map<std::string, int> buf_index;
  std::map<std::string, kern_module> modules;
  std::vector<RtOp> ops;
  std::map<std::string, int> op_index;
  std::vector<RtProgram> programs;
  std::map<std::string, int> prog_index;
  std::map<std::pair<int, std::vector<uint64_t>>, hipGraphExec_t> graphs;
  bool has_derive = false, derived = false;

  ~kern_runtime_s() {
    (void)hipSetDevice(gpu);
    if (stream) (void)hipStreamSynchronize(stream);
    for (auto& g : graphs) (void)hipGraphExecDestroy(g.second);
    for (auto& b : buffers) {
      if (b.dev) (void)hipFree(b.dev);
      if (b.staging) (void)hipHostFree(b.staging);
    }
    for (auto& o : ops) kern_op_destroy(o.op);
    for (auto& m : modules) kern_module_unload(m.second);
    if (stream) (void)hipStreamDestroy(stream);
  }
};

namespace {

#define RT_HIP(call, what)                                                                                   \
  do {                                                                                                     \
    hipError_t e_ = (call);                                                                                \
    if (e_ != hipSuccess) return kern_amd_fail(KERN_ERR_HIP, "%s: %s", what, hipGetErrorString(e_));     \
  } while (0)

int manifest_fail(const char* fmt, ...) {
  char buf[1024];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof buf, fmt, ap);
  va_end(ap);
  return kern_amd_fail(KERN_ERR_MANIFEST, "manifest: %s", buf);
}

// ------------------------------------------------------------------------------------ load
// host_only: read every module file and check its sha256 on the host, verify every op, create nothing on
// the device (kern_rt_check)
int parse_manifest(kern_runtime_s& rt, const char* text, const JVal& root, const char* kernels_dir, bool host_only) {
  if (root.kind != JVal::Obj) return manifest_fail("expected an object");
  if (const JVal* v = root.get("schema_version"))
    if (v->kind != JVal::Int || v->i != 7) return manifest_fail("schema_version must be 7");
  for (const char* unsupported : {"topology", "states"}) {
    const JVal* v = root.get(unsupported);
    if (v && !((v->kind == JVal::Obj && v->o.empty()) || v->kind == JVal::Null))
      return manifest_fail("`%s` is not served by this runtime (the MXFP4 matmul path has none)", unsupported);
  }
  // vars
  if (const JVal* vs = root.get("vars")) {
    if (vs->kind != JVal::Obj) return manifest_fail("`vars` must be an object");
    for (auto& kv : vs->o) {
      const JVal* mx = kv.second.get("max");
      if (!mx || mx->kind != JVal::Int || mx->i <= 0) return manifest_fail("var `%s`: `max` must be a positive integer", kv.first.c_str());
      rt.var_index[kv.first] = (int)rt.var_names.size();
      rt.var_names.push_back(kv.first);
      rt.var_max.push_back(mx->u);
    }
  }
  // buffers
  const JVal* bs = root.get("buffers");
  if (!bs || bs->kind != JVal::Obj) return manifest_fail("missing `buffers` object");
  for (auto& kv : bs->o) {
    const JVal& b = kv.second;
    RtBuffer rb;
    rb.name = kv.first;
    const JVal* dt = b.get("dtype");
    if (!dt || dt->kind != JVal::Str || !dtype_size(dt->s)) return manifest_fail("buffer `%s`: unknown dtype", kv.first.c_str());
    rb.dtype = dt->s;
    const JVal* k = b.get("kind");
    static const char* kinds[] = {"input", "output", "inout", "weight", "source", "workspace", "carry"};
    int kind = -1;
    if (k && k->kind == JVal::Str)
      for (int i = 0; i < 7; ++i)
        if (k->s == kinds[i]) kind = i;
    if (kind < 0)
      return manifest_fail("buffer `%s`: kind `%s` is not served (input, output, inout, weight, source, workspace, carry)",
                           kv.first.c_str(), k && k->kind == JVal::Str ? k->s.c_str() : "?");
    rb.kind = kind;
    if (const JVal* pl = b.get("placement"))
      if (!(pl->kind == JVal::Str && pl->s == "device")) return manifest_fail("buffer `%s`: only device placement", kv.first.c_str());
    if (const JVal* ex = b.get("export"))
      if (ex->kind == JVal::Bool && ex->b) return manifest_fail("buffer `%s`: exported buffers are not served", kv.first.c_str());
    const JVal* sh = b.get("shape");
    if (!sh || sh->kind != JVal::Arr) return manifest_fail("buffer `%s`: missing `shape`", kv.first.c_str());
    size_t n = dtype_size(rb.dtype);
    for (auto& d : sh->a) {
      Dim dm;
      if (d.kind == JVal::Int && d.i >= 0) {
        dm.c = d.u;
        n *= d.u;
      } else if (d.kind == JVal::Str && rt.var_index.count(d.s)) {
        dm.is_var = true, dm.var = rt.var_index[d.s];
        n *= rt.var_max[dm.var];
      } else {
        return manifest_fail("buffer `%s`: a dim is neither a count nor a declared var", kv.first.c_str());
      }
      rb.shape.push_back(dm);
    }
    rb.bytes = n;
    rt.buf_index[rb.name] = (int)rt.buffers.size();
    rt.buffers.push_back(rb);
  }
  // modules: a file under kernels_dir, pinned by its sha256
  const JVal* ms = root.get("modules");
  if (!ms || ms->kind != JVal::Obj) return manifest_fail("missing `modules` object");
  for (auto& kv : ms->o) {
    const JVal* src = kv.second.get("source");
    const JVal* sha = kv.second.get("sha256");
    if (!src || src->kind != JVal::Str || !sha || sha->kind != JVal::Str)
      return manifest_fail("module `%s`: needs `source` and `sha256`", kv.first.c_str());
    const std::string path = std::string(kernels_dir) + "/" + src->s;
    std::ifstream f(path, std::ios::binary);
    if (!f)
      return kern_amd_fail(KERN_ERR_KERNEL_ARTIFACT, "module `%s`: cannot read `%s`", kv.first.c_str(), path.c_str());
    std::vector<char> image((std::istreambuf_iterator<char>(f)), std::istreambuf_iterator<char>());
    if (host_only) {
      char hex[65];
      kern_sha256_hex(image.data(), image.size(), hex);
      if (strcasecmp(hex, sha->s.c_str()) != 0)
        return kern_amd_fail(KERN_ERR_KERNEL_ARTIFACT, "module `%s` (%s): sha256 %s, the manifest pins %s", kv.first.c_str(),
                             path.c_str(), hex, sha->s.c_str());
      rt.modules[kv.first] = nullptr;
      continue;
    }
    kern_module mod = nullptr;
    if (int rc = kern_module_load(image.data(), image.size(), sha->s.c_str(), &mod))
      return kern_amd_fail(rc, "module `%s` (%s): %s", kv.first.c_str(), path.c_str(), kern_last_error());
    rt.modules[kv.first] = mod;
  }
  // ops: one module per op, created from the op's own JSON text
  const JVal* os = root.get("ops");
  if (!os || os->kind != JVal::Obj) return manifest_fail("missing `ops` object");
  for (auto& kv : os->o) {
    RtOp ro;
    ro.name = kv.first;
    const JVal* ps = kv.second.get("params");
    if (!ps || ps->kind != JVal::Arr) return manifest_fail("op `%s`: missing `params`", kv.first.c_str());
    for (auto& p : ps->a) {
      OpParam op;
      if (p.kind != JVal::Str || !parse_op_param(p.s, op))
        return manifest_fail("op `%s`: param `%s` is not served", kv.first.c_str(), p.kind == JVal::Str ? p.s.c_str() : "?");
      ro.params.push_back(op);
    }
    const JVal* im = kv.second.get("impl");
    const JVal* ls = im ? im->get("launches") : nullptr;
    if (!ls || ls->kind != JVal::Arr || ls->a.empty()) return manifest_fail("op `%s`: no launches", kv.first.c_str());
    const JVal* m0 = ls->a[0].get("module");
    if (!m0 || m0->kind != JVal::Str) return manifest_fail("op `%s`: launch #0 names no module", kv.first.c_str());
    for (size_t li = 1; li < ls->a.size(); ++li) {
      const JVal* m = ls->a[li].get("module");
      if (!m || m->kind != JVal::Str || m->s != m0->s)
        return manifest_fail("op `%s`: every launch must name module `%s`", kv.first.c_str(), m0->s.c_str());
    }
    auto mod = rt.modules.find(m0->s);
    if (mod == rt.modules.end()) return manifest_fail("op `%s`: module `%s` is not declared", kv.first.c_str(), m0->s.c_str());
    const std::string op_text(text + kv.second.off, kv.second.len);
    if (int rc = host_only ? kern_op_verify(op_text.c_str()) : kern_op_create(op_text.c_str(), m0->s.c_str(), mod->second, &ro.op))
      return kern_amd_fail(rc, "op `%s`: %s", kv.first.c_str(), kern_last_error());
    ro.ring_param = kern_op_ring_activation_param(op_text.c_str());
    rt.op_index[ro.name] = (int)rt.ops.size();
    rt.ops.push_back(std::move(ro));
  }
  // programs
  const JVal* prs = root.get("programs");
  if (!prs || prs->kind != JVal::Obj) return manifest_fail("missing `programs` object");
  for (auto& kv : prs->o) {
    RtProgram pg;
    pg.name = kv.first;
    const JVal& p = kv.second;
    if (const JVal* g = p.get("graph")) pg.graph = g->kind == JVal::Bool && g->b;
    if (const JVal* d = p.get("derive")) pg.derive = d->kind == JVal::Bool && d->b;
    if (const JVal* o = p.get("once")) pg.once = o->kind == JVal::Bool && o->b;
    if (pg.derive && pg.graph) return manifest_fail("program `%s`: a derive program is not a graph", kv.first.c_str());
    const JVal* cs = p.get("calls");
    if (!cs || cs->kind != JVal::Arr) return manifest_fail("program `%s`: missing `calls`", kv.first.c_str());
    for (size_t ci = 0; ci < cs->a.size(); ++ci) {
      const JVal& c = cs->a[ci];
      RtCall call;
      if (const JVal* l = c.get("label")) call.label = l->kind == JVal::Str ? l->s : "";
      if (const JVal* ln = c.get("lane"))
        if (!(ln->kind == JVal::Int && ln->i == 0))
          return manifest_fail("program `%s` call #%zu: one lane per program here", kv.first.c_str(), ci);
      if (const JVal* af = c.get("after"))
        for (auto& x : af->a)
          if (!(x.kind == JVal::Int && x.i == 0))
            return manifest_fail("program `%s` call #%zu: one lane per program here", kv.first.c_str(), ci);
      const JVal* on = c.get("op");
      if (!on || on->kind != JVal::Str || !rt.op_index.count(on->s))
        return manifest_fail("program `%s` call #%zu: unknown op", kv.first.c_str(), ci);
      call.op = rt.op_index[on->s];
      const RtOp& op = rt.ops[call.op];
      const JVal* as = c.get("args");
      if (!as || as->kind != JVal::Arr || as->a.size() != op.params.size())
        return manifest_fail("program `%s` call #%zu (%s): op `%s` takes %zu args", kv.first.c_str(), ci,
                             call.label.c_str(), op.name.c_str(), op.params.size());
      for (size_t ai = 0; ai < as->a.size(); ++ai) {
        const JVal& a = as->a[ai];
        const OpParam& prm = op.params[ai];
        RtArg ra;
        if (a.kind != JVal::Obj || a.o.empty())
          return manifest_fail("program `%s` call #%zu arg #%zu: expected an object", kv.first.c_str(), ci, ai);
        const std::string& key = a.o[0].first;
        const JVal& val = a.o[0].second;
        if (prm.buf) {
          const JVal* bn = a.get("buf");
          if (!bn || bn->kind != JVal::Str || !rt.buf_index.count(bn->s))
            return manifest_fail("program `%s` call #%zu arg #%zu: param `%s` needs a declared buffer", kv.first.c_str(),
                                 ci, ai, prm.text.c_str());
          ra.kind = RtArg::Buf, ra.buf = rt.buf_index[bn->s];
          if (const JVal* off = a.get("offset")) ra.offset = off->u;
          const RtBuffer& b = rt.buffers[ra.buf];
          if (b.dtype != prm.dtype)
            return manifest_fail("program `%s` call #%zu arg #%zu: buffer `%s` is %s, param `%s`", kv.first.c_str(), ci,
                                 ai, b.name.c_str(), b.dtype.c_str(), prm.text.c_str());
          if (ra.offset >= b.bytes)
            return manifest_fail("program `%s` call #%zu arg #%zu: offset past buffer `%s`", kv.first.c_str(), ci, ai,
                                 b.name.c_str());
          // the LDS-ring GEMMs address their activations by 32-bit byte offsets from the bound address
          if ((int)ai == op.ring_param && b.bytes - ra.offset >= ((uint64_t)1 << 32))
            return manifest_fail("program `%s` call #%zu arg #%zu: `%s` binds %zu bytes of buffer `%s` as activations "
                                 "of a ring GEMM, which must stay below 4 GiB", kv.first.c_str(), ci, ai,
                                 prm.text.c_str(), (size_t)(b.bytes - ra.offset), b.name.c_str());
          // who may write and read what (types.rs:674-694, :150-155)
          const bool writes = prm.dir != 0;
          if (pg.derive && (b.kind == K_INPUT || b.kind == K_OUTPUT || b.kind == K_INOUT))
            return manifest_fail("derive program `%s` call #%zu: reads no input or output (`%s`)", kv.first.c_str(), ci,
                                 b.name.c_str());
          if (!pg.derive && b.kind == K_SOURCE)
            return manifest_fail("program `%s` call #%zu: source buffer `%s` is only for derive programs",
                                 kv.first.c_str(), ci, b.name.c_str());
          if (!pg.derive && writes && (b.kind == K_WEIGHT || b.kind == K_INPUT))
            return manifest_fail("program `%s` call #%zu: param `%s` writes %s buffer `%s`", kv.first.c_str(), ci,
                                 prm.text.c_str(), kind_name(b.kind), b.name.c_str());
          if (pg.derive && writes && b.kind == K_SOURCE)
            return manifest_fail("derive program `%s` call #%zu: writes its source `%s`", kv.first.c_str(), ci,
                                 b.name.c_str());
        } else if (key == "var") {
          if (val.kind != JVal::Str || !rt.var_index.count(val.s))
            return manifest_fail("program `%s` call #%zu arg #%zu: unknown var", kv.first.c_str(), ci, ai);
          if (prm.dtype != "i32" && prm.dtype != "i64")
            return manifest_fail("program `%s` call #%zu arg #%zu: a var binds an i32 or i64 param, not `%s`",
                                 kv.first.c_str(), ci, ai, prm.text.c_str());
          ra.kind = RtArg::Var, ra.var = rt.var_index[val.s];
        } else {
          if (key != prm.dtype || !val.is_num())
            return manifest_fail("program `%s` call #%zu arg #%zu: param `%s` needs {\"%s\": value}", kv.first.c_str(),
                                 ci, ai, prm.text.c_str(), prm.dtype.c_str());
          ra.kind = RtArg::Lit;
          if (key == "f32") {
            float f = (float)val.f;
            uint32_t u;
            memcpy(&u, &f, 4);
            ra.bits = u;
          } else if (key == "i32") {
            ra.bits = (uint32_t)(int32_t)val.i;
          } else if (key == "u8") {
            ra.bits = (uint8_t)val.i;
          } else {
            ra.bits = (uint64_t)val.i;
          }
        }
        call.args.push_back(ra);
      }
      pg.calls.push_back(std::move(call));
    }
    rt.has_derive |= pg.derive;
    rt.prog_index[pg.name] = (int)rt.programs.size();
    rt.programs.push_back(std::move(pg));
  }
  return KERN_OK;
}

// the caller's var values, checked against the manifest: one entry per manifest var (UINT64_MAX = unset)
int dense_vars(const kern_runtime_s& rt, const char* const* names, const uint64_t* values, int n,
               std::vector<uint64_t>& dense) {
  dense.assign(rt.var_names.size(), UINT64_MAX);
  if (n < 0 || (n && (!names || !values))) return kern_amd_fail(KERN_ERR_API, "vars: %d names without values", n);
  for (int i = 0; i < n; ++i) {
    auto it = rt.var_index.find(names[i] ? names[i] : "");
    if (it == rt.var_index.end()) return kern_amd_fail(KERN_ERR_API, "vars: `%s` is not a manifest var", names[i]);
    if (values[i] > rt.var_max[it->second])
      return kern_amd_fail(KERN_ERR_API, "vars: %s = %llu exceeds its max %llu", names[i], (unsigned long long)values[i],
                           (unsigned long long)rt.var_max[it->second]);
    dense[it->second] = values[i];
  }
  return KERN_OK;
}

// issue a program's calls onto the runtime's stream, launch by launch
// Issue calls [lo, hi) of a program on the runtime's stream; with `after`, event after[ci - lo] is recorded
// behind call ci (time_range's per-call brackets).
int issue_calls(kern_runtime_s& rt, const RtProgram& pg, const std::vector<uint64_t>& dense, size_t lo = 0,
                size_t hi = SIZE_MAX, hipEvent_t* after = nullptr) {
  std::vector<const char*> vn;
  std::vector<uint64_t> vv;
  for (size_t i = 0; i < dense.size(); ++i)
    if (dense[i] != UINT64_MAX) vn.push_back(rt.var_names[i].c_str()), vv.push_back(dense[i]);
  std::vector<uint64_t> params;
  hi = std::min(hi, pg.calls.size());
  for (size_t ci = lo; ci < hi; ++ci) {
    const RtCall& c = pg.calls[ci];
    const RtOp& op = rt.ops[c.op];
    params.assign(c.args.size(), 0);
    for (size_t ai = 0; ai < c.args.size(); ++ai) {
      const RtArg& a = c.args[ai];
      if (a.kind == RtArg::Buf) {
        const RtBuffer& b = rt.buffers[a.buf];
        if (b.freed)
          return kern_amd_fail(KERN_ERR_CALL, "program `%s` call #%zu (%s): buffer `%s` was freed after derive",
                               pg.name.c_str(), ci, c.label.c_str(), b.name.c_str());
        params[ai] = (uint64_t)(uintptr_t)b.dev + a.offset;
      } else if (a.kind == RtArg::Var) {
        if (dense[a.var] == UINT64_MAX)
          return kern_amd_fail(KERN_ERR_CALL, "program `%s` call #%zu (%s): var `%s` is not bound", pg.name.c_str(), ci,
                               c.label.c_str(), rt.var_names[a.var].c_str());
        const bool i32 = op.params[ai].dtype == "i32";
        if (i32 && dense[a.var] > 0x7fffffffull)
          return kern_amd_fail(KERN_ERR_CALL, "program `%s` call #%zu (%s): var `%s` does not fit an i32",
                               pg.name.c_str(), ci, c.label.c_str(), rt.var_names[a.var].c_str());
        params[ai] = i32 ? (uint64_t)(uint32_t)dense[a.var] : dense[a.var];
      } else {
        params[ai] = a.bits;
      }
    }
    if (kern_op_launch(op.op, params.data(), (int)params.size(), vn.data(), vv.data(), (int)vn.size(), rt.stream))
      return kern_amd_fail(KERN_ERR_CALL, "program `%s` call #%zu (%s, op `%s`): %s", pg.name.c_str(), ci,
                           c.label.c_str(), op.name.c_str(), kern_last_error());
    if (after) RT_HIP(hipEventRecord(after[ci - lo], rt.stream), "hipEventRecord");
  }
  return KERN_OK;
}

// hipEvents released on every path out of a timing call
struct Events {
  std::vector<hipEvent_t> ev;
  ~Events() {
    for (hipEvent_t e : ev) (void)hipEventDestroy(e);
  }
  int create(size_t n) {
    for (size_t i = 0; i < n; ++i) {
      hipEvent_t e = nullptr;
      RT_HIP(hipEventCreate(&e), "hipEventCreate");
      ev.push_back(e);
    }
    return KERN_OK;
  }
};

int find_program(kern_runtime_s& rt, const char* name, const RtProgram** out) {
  auto it = rt.prog_index.find(name ? name : "");
  if (it == rt.prog_index.end()) return kern_amd_fail(KERN_ERR_API, "no program `%s`", name ? name : "(null)");
  const RtProgram& pg = rt.programs[it->second];
  if (pg.derive) return kern_amd_fail(KERN_ERR_API, "program `%s` is a derive program: kern_rt_derive runs it", name);
  if (rt.has_derive && !rt.derived)
    return kern_amd_fail(KERN_ERR_API, "the manifest's derive programs have not run: call kern_rt_derive after loading weights");
  *out = &pg;
  return KERN_OK;
}

int capture_program(kern_runtime_s& rt, const RtProgram& pg, const std::vector<uint64_t>& dense) {
  std::lock_guard<std::mutex> serial(g_capture);
  RT_HIP(hipStreamBeginCapture(rt.stream, hipStreamCaptureModeThreadLocal), "hipStreamBeginCapture");
  const int rc = issue_calls(rt, pg, dense);
  hipGraph_t graph = nullptr;
  const hipError_t end = hipStreamEndCapture(rt.stream, &graph);
  if (rc) {
    if (graph) (void)hipGraphDestroy(graph);
    return rc;
  }
  if (end != hipSuccess) return kern_amd_fail(KERN_ERR_HIP, "hipStreamEndCapture: %s", hipGetErrorString(end));
  hipGraphExec_t exec = nullptr;
  const hipError_t inst = hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0);
  (void)hipGraphDestroy(graph);
  if (inst != hipSuccess) return kern_amd_fail(KERN_ERR_HIP, "hipGraphInstantiate: %s", hipGetErrorString(inst));
  const int pi = rt.prog_index[pg.name];
  auto key = std::make_pair(pi, dense);
  auto old = rt.graphs.find(key);
  if (old != rt.graphs.end()) (void)hipGraphExecDestroy(old->second);
  rt.graphs[key] = exec;
  return KERN_OK;
}

int graph_of(kern_runtime_s& rt, const RtProgram& pg, const std::vector<uint64_t>& dense, hipGraphExec_t* out) {
  auto it = rt.graphs.find(std::make_pair(rt.prog_index[pg.name], dense));
  if (it != rt.graphs.end()) {
    *out = it->second;
    return KERN_OK;
  }
  std::string others;
  for (auto& g : rt.graphs) {
    if (g.first.first != rt.prog_index[pg.name]) continue;
    others += " {";
    for (size_t i = 0; i < g.first.second.size(); ++i)
      if (g.first.second[i] != UINT64_MAX)
        others += rt.var_names[i] + "=" + std::to_string(g.first.second[i]) + " ";
    others += "}";
  }
  if (others.empty()) return kern_amd_fail(KERN_ERR_API, "program `%s` has not been captured", pg.name.c_str());
  return kern_amd_fail(KERN_ERR_API, "program `%s` was captured at%s, not at these vars", pg.name.c_str(), others.c_str());
}

int buffer_of(kern_runtime_s& rt, const char* name, RtBuffer** out) {
  auto it = rt.buf_index.find(name ? name : "");
  if (it == rt.buf_index.end()) return kern_amd_fail(KERN_ERR_API, "no buffer `%s`", name ? name : "(null)");
  RtBuffer& b = rt.buffers[it->second];
  if (b.freed) return kern_amd_fail(KERN_ERR_API, "buffer `%s` was freed after derive", b.name.c_str());
  *out = &b;
  return KERN_OK;
}

}  // namespace

// ------------------------------------------------------------------------------------ C ABI
#define RT_ENTER(rt)                                                                         \
  if (!(rt)) return kern_amd_fail(KERN_ERR_API, "null runtime");                           \
  std::lock_guard<std::mutex> lock_((rt)->mu);                                             \
  RT_HIP(hipSetDevice((rt)->gpu), "hipSetDevice")

extern "C" int kern_rt_load(const char* manifest_json, const char* kernels_dir, int gpu, kern_runtime* out) {
  if (!manifest_json || !kernels_dir || !out) return kern_amd_fail(KERN_ERR_API, "kern_rt_load: null argument");
  *out = nullptr;
  int ndev = 0;
  RT_HIP(hipGetDeviceCount(&ndev), "hipGetDeviceCount");
  if (gpu < 0 || gpu >= ndev) return kern_amd_fail(KERN_ERR_API, "kern_rt_load: gpu %d of %d", gpu, ndev);
  RT_HIP(hipSetDevice(gpu), "hipSetDevice");
  std::unique_ptr<kern_runtime_s> rt(new kern_runtime_s);
  rt->gpu = gpu;
  JVal root;
  std::string err;
  if (!kern_json::parse_json(manifest_json, root, err)) return manifest_fail("%s", err.c_str());
  if (int rc = parse_manifest(*rt, manifest_json, root, kernels_dir, false)) return rc;
  RT_HIP(hipStreamCreateWithFlags(&rt->stream, hipStreamNonBlocking), "hipStreamCreate");
  for (auto& b : rt->buffers) {
    if (!b.bytes) continue;
    RT_HIP(hipMalloc(&b.dev, b.bytes), "hipMalloc");
    RT_HIP(hipMemsetAsync(b.dev, 0, b.bytes, rt->stream), "hipMemsetAsync");
    if (b.kind == K_INPUT || b.kind == K_INOUT) RT_HIP(hipHostMalloc(&b.staging, b.bytes, hipHostMallocDefault), "hipHostMalloc");
  }
  RT_HIP(hipStreamSynchronize(rt->stream), "hipStreamSynchronize");
  *out = rt.release();
  return KERN_OK;
}

extern "C" int kern_rt_check(const char* manifest_json, const char* kernels_dir) {
  if (!manifest_json || !kernels_dir) return kern_amd_fail(KERN_ERR_API, "kern_rt_check: null argument");
  kern_runtime_s rt;
  JVal root;
  std::string err;
  if (!kern_json::parse_json(manifest_json, root, err)) return manifest_fail("%s", err.c_str());
  return parse_manifest(rt, manifest_json, root, kernels_dir, true);
}

extern "C" int kern_rt_destroy(kern_runtime rt) {
  if (!rt) return KERN_OK;
  delete rt;
  return KERN_OK;
}

extern "C" int kern_rt_write_input(kern_runtime rt, const char* name, const void* data, size_t len) {
  RT_ENTER(rt);
  RtBuffer* b = nullptr;
  if (int rc = buffer_of(*rt, name, &b)) return rc;
  if (b->kind != K_INPUT && b->kind != K_INOUT)
    return kern_amd_fail(KERN_ERR_API, "write_input: `%s` is a %s buffer, not input or inout", name, kind_name(b->kind));
  if (len > b->bytes || (len && !data))
    return kern_amd_fail(KERN_ERR_API, "write_input: %zu bytes for `%s` of %zu", len, name, b->bytes);
  // through the buffer's pinned staging: a true async copy on the runtime's stream (lib.rs:293-318)
  memcpy(b->staging, data, len);
  RT_HIP(hipMemcpyAsync(b->dev, b->staging, len, hipMemcpyHostToDevice, rt->stream), "hipMemcpyAsync");
  RT_HIP(hipStreamSynchronize(rt->stream), "hipStreamSynchronize");
  return KERN_OK;
}

extern "C" int kern_rt_read_output(kern_runtime rt, const char* name, void* data, size_t len) {
  RT_ENTER(rt);
  RtBuffer* b = nullptr;
  if (int rc = buffer_of(*rt, name, &b)) return rc;
  if (b->kind != K_OUTPUT && b->kind != K_INOUT)
    return kern_amd_fail(KERN_ERR_API, "read_output: `%s` is a %s buffer, not output or inout", name, kind_name(b->kind));
  if (len > b->bytes || (len && !data))
    return kern_amd_fail(KERN_ERR_API, "read_output: %zu bytes from `%s` of %zu", len, name, b->bytes);
  RT_HIP(hipStreamSynchronize(rt->stream), "hipStreamSynchronize");
  RT_HIP(hipMemcpy(data, b->dev, len, hipMemcpyDeviceToHost), "hipMemcpy");
  return KERN_OK;
}

extern "C" int kern_rt_write_buffer(kern_runtime rt, const char* name, size_t offset, const void* data, size_t len) {
  RT_ENTER(rt);
  RtBuffer* b = nullptr;
  if (int rc = buffer_of(*rt, name, &b)) return rc;
  if (offset > b->bytes || len > b->bytes - offset || (len && !data))
    return kern_amd_fail(KERN_ERR_API, "write_buffer: [%zu, +%zu) outside `%s` of %zu bytes", offset, len, name, b->bytes);
  RT_HIP(hipStreamSynchronize(rt->stream), "hipStreamSynchronize");
  RT_HIP(hipMemcpy((char*)b->dev + offset, data, len, hipMemcpyHostToDevice), "hipMemcpy");
  return KERN_OK;
}

extern "C" int kern_rt_read_buffer(kern_runtime rt, const char* name, size_t offset, void* data, size_t len) {
  RT_ENTER(rt);
  RtBuffer* b = nullptr;
  if (int rc = buffer_of(*rt, name, &b)) return rc;
  if (offset > b->bytes || len > b->bytes - offset || (len && !data))
    return kern_amd_fail(KERN_ERR_API, "read_buffer: [%zu, +%zu) outside `%s` of %zu bytes", offset, len, name, b->bytes);
  RT_HIP(hipStreamSynchronize(rt->stream), "hipStreamSynchronize");
  RT_HIP(hipMemcpy(data, (const char*)b->dev + offset, len, hipMemcpyDeviceToHost), "hipMemcpy");
  return KERN_OK;
}

extern "C" int kern_rt_load_weight(kern_runtime rt, const char* name, const void* data, size_t len) {
  RT_ENTER(rt);
  RtBuffer* b = nullptr;
  if (int rc = buffer_of(*rt, name, &b)) return rc;
  if (b->kind != K_WEIGHT && b->kind != K_SOURCE)
    return kern_amd_fail(KERN_ERR_API, "load_weight: `%s` is a %s buffer, not weight or source", name, kind_name(b->kind));
  if (len != b->bytes || !data)
    return kern_amd_fail(KERN_ERR_API, "load_weight: %zu bytes for `%s` of %zu", len, name, b->bytes);
  RT_HIP(hipStreamSynchronize(rt->stream), "hipStreamSynchronize");
  RT_HIP(hipMemcpy(b->dev, data, len, hipMemcpyHostToDevice), "hipMemcpy");
  return KERN_OK;
}

extern "C" int kern_rt_derive(kern_runtime rt) {
  RT_ENTER(rt);
  if (rt->derived) return kern_amd_fail(KERN_ERR_API, "derive: already run (its sources are freed)");
  const std::vector<uint64_t> none(rt->var_names.size(), UINT64_MAX);
  for (auto& pg : rt->programs)
    if (pg.derive)
      if (int rc = issue_calls(*rt, pg, none)) return rc;
  RT_HIP(hipStreamSynchronize(rt->stream), "hipStreamSynchronize");
  for (auto& b : rt->buffers)
    if (b.kind == K_SOURCE && b.dev) {
      RT_HIP(hipFree(b.dev), "hipFree");
      b.dev = nullptr, b.freed = true;
    }
  rt->derived = true;
  return KERN_OK;
}

extern "C" int kern_rt_run(kern_runtime rt, const char* program, const char* const* var_names,
                           const uint64_t* var_values, int nvars) {
  RT_ENTER(rt);
  const RtProgram* pg = nullptr;
  if (int rc = find_program(*rt, program, &pg)) return rc;
  std::vector<uint64_t> dense;
  if (int rc = dense_vars(*rt, var_names, var_values, nvars, dense)) return rc;
  if (pg->graph) {
    hipGraphExec_t exec = nullptr;
    if (!rt->graphs.count(std::make_pair(rt->prog_index[pg->name], dense)))
      if (int rc = capture_program(*rt, *pg, dense)) return rc;
    if (int rc = graph_of(*rt, *pg, dense, &exec)) return rc;
    RT_HIP(hipGraphLaunch(exec, rt->stream), "hipGraphLaunch");
  } else if (int rc = issue_calls(*rt, *pg, dense)) {
    return rc;
  }
  RT_HIP(hipStreamSynchronize(rt->stream), "hipStreamSynchronize");
  return KERN_OK;
}

extern "C" int kern_rt_capture(kern_runtime rt, const char* program, const char* const* var_names,
                               const uint64_t* var_values, int nvars) {
  RT_ENTER(rt);
  const RtProgram* pg = nullptr;
  if (int rc = find_program(*rt, program, &pg)) return rc;
  std::vector<uint64_t> dense;
  if (int rc = dense_vars(*rt, var_names, var_values, nvars, dense)) return rc;
  return capture_program(*rt, *pg, dense);
}

extern "C" int kern_rt_run_captured(kern_runtime rt, const char* program, const char* const* var_names,
                                    const uint64_t* var_values, int nvars) {
  RT_ENTER(rt);
  const RtProgram* pg = nullptr;
  if (int rc = find_program(*rt, program, &pg)) return rc;
  std::vector<uint64_t> dense;
  if (int rc = dense_vars(*rt, var_names, var_values, nvars, dense)) return rc;
  hipGraphExec_t exec = nullptr;
  if (int rc = graph_of(*rt, *pg, dense, &exec)) return rc;
  RT_HIP(hipGraphLaunch(exec, rt->stream), "hipGraphLaunch");
  RT_HIP(hipStreamSynchronize(rt->stream), "hipStreamSynchronize");
  return KERN_OK;
}

extern "C" int kern_rt_time_captured(kern_runtime rt, const char* program, const char* const* var_names,
                                     const uint64_t* var_values, int nvars, int iters, float* ms_per_iter) {
  RT_ENTER(rt);
  if (iters <= 0 || !ms_per_iter) return kern_amd_fail(KERN_ERR_API, "time_captured: need iters > 0 and an out pointer");
  const RtProgram* pg = nullptr;
  if (int rc = find_program(*rt, program, &pg)) return rc;
  std::vector<uint64_t> dense;
  if (int rc = dense_vars(*rt, var_names, var_values, nvars, dense)) return rc;
  hipGraphExec_t exec = nullptr;
  if (int rc = graph_of(*rt, *pg, dense, &exec)) return rc;
  // back-to-back replays with an event between each, median replay (harness.rs:252-266)
  Events ev;
  if (int rc = ev.create((size_t)iters + 1)) return rc;
  RT_HIP(hipEventRecord(ev.ev[0], rt->stream), "hipEventRecord");
  for (int i = 0; i < iters; ++i) {
    RT_HIP(hipGraphLaunch(exec, rt->stream), "hipGraphLaunch");
    RT_HIP(hipEventRecord(ev.ev[i + 1], rt->stream), "hipEventRecord");
  }
  RT_HIP(hipEventSynchronize(ev.ev[iters]), "hipEventSynchronize");
  std::vector<float> t((size_t)iters);
  for (int i = 0; i < iters; ++i) RT_HIP(hipEventElapsedTime(&t[i], ev.ev[i], ev.ev[i + 1]), "hipEventElapsedTime");
  std::sort(t.begin(), t.end());
  *ms_per_iter = t[(size_t)iters / 2];
  return KERN_OK;
}

// Runtime::run_range (harness.rs:186-207): calls [lo, hi) of a program, eagerly, then synchronize.
extern "C" int kern_rt_run_range(kern_runtime rt, const char* program, const char* const* var_names,
                                 const uint64_t* var_values, int nvars, int lo, int hi) {
  RT_ENTER(rt);
  const RtProgram* pg = nullptr;
  if (int rc = find_program(*rt, program, &pg)) return rc;
  if (lo < 0 || lo > hi || (size_t)hi > pg->calls.size())
    return kern_amd_fail(KERN_ERR_API, "program `%s`: call range [%d, %d) outside 0..%zu", pg->name.c_str(), lo, hi,
                         pg->calls.size());
  std::vector<uint64_t> dense;
  if (int rc = dense_vars(*rt, var_names, var_values, nvars, dense)) return rc;
  if (int rc = issue_calls(*rt, *pg, dense, (size_t)lo, (size_t)hi)) return rc;
  RT_HIP(hipStreamSynchronize(rt->stream), "hipStreamSynchronize");
  return KERN_OK;
}

// Runtime::time_range (harness.rs:209-250): per-call GPU milliseconds of calls [lo, hi), issued eagerly and
// bracketed by events, each the minimum over iters runs of just that range; a launch gap counts towards the
// call after it.
extern "C" int kern_rt_time_range(kern_runtime rt, const char* program, const char* const* var_names,
                                  const uint64_t* var_values, int nvars, int lo, int hi, int iters, float* ms_per_call) {
  RT_ENTER(rt);
  const RtProgram* pg = nullptr;
  if (int rc = find_program(*rt, program, &pg)) return rc;
  if (lo < 0 || lo > hi || (size_t)hi > pg->calls.size())
    return kern_amd_fail(KERN_ERR_API, "program `%s`: call range [%d, %d) outside 0..%zu", pg->name.c_str(), lo, hi,
                         pg->calls.size());
  if (hi > lo && !ms_per_call) return kern_amd_fail(KERN_ERR_API, "time_range: null out pointer");
  std::vector<uint64_t> dense;
  if (int rc = dense_vars(*rt, var_names, var_values, nvars, dense)) return rc;
  const size_t n = (size_t)(hi - lo);
  Events ev;
  if (int rc = ev.create(n + 1)) return rc;
  std::vector<float> best(n, INFINITY);
  for (int it = 0; it < std::max(iters, 1); ++it) {
    RT_HIP(hipEventRecord(ev.ev[0], rt->stream), "hipEventRecord");
    if (int rc = issue_calls(*rt, *pg, dense, (size_t)lo, (size_t)hi, ev.ev.data() + 1)) return rc;
    RT_HIP(hipStreamSynchronize(rt->stream), "hipStreamSynchronize");
    for (size_t i = 0; i < n; ++i) {
      float ms = 0.f;
      RT_HIP(hipEventElapsedTime(&ms, ev.ev[i], ev.ev[i + 1]), "hipEventElapsedTime");
      best[i] = std::min(best[i], ms);
    }
  }
  for (size_t i = 0; i < n; ++i) ms_per_call[i] = best[i];
  return KERN_OK;
}

extern "C" int kern_rt_synchronize(kern_runtime rt) {
  RT_ENTER(rt);
  RT_HIP(hipStreamSynchronize(rt->stream), "hipStreamSynchronize");
  return KERN_OK;
}

extern "C" int kern_rt_buffer(kern_runtime rt, const char* name, void** device_ptr, size_t* bytes) {
  RT_ENTER(rt);
  RtBuffer* b = nullptr;
  if (int rc = buffer_of(*rt, name, &b)) return rc;
  if (device_ptr) *device_ptr = b->dev;
  if (bytes) *bytes = b->bytes;
  return KERN_OK;
}
