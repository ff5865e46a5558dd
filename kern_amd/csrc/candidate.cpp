// Candidates: other implementations of ops a manifest already has (crates/kern-manifest/src/candidate.rs).
//
// A candidate is a file holding the `modules` and `ops` sections of a manifest and nothing else, each op
// under the name and with the `params` of the op it stands in for. kern_candidate_splice puts one into a
// manifest the way candidate::splice does (candidate.rs:152-185): the interface is what is checked (an op
// the manifest lacks, one whose params differ, or a launch naming a module that neither side has is
// refused, every reason reported together); the candidate's modules are taken in, each under its own name
// or, when the manifest already pins other bytes under that name, as `<name>@<first 8 hex of its sha256>`
// (candidate.rs:116-131); the replaced ops' launches are renamed to match; and modules no launch names any
// more are dropped. Everything else in the manifest (vars, buffers, programs and their calls, the ops the
// candidate leaves alone) is carried over as the same JSON text.
//
// kern_candidate_of / _only / _join / _tile build candidates (candidate.rs:83-113, :231-300): a manifest's
// own implementation of some ops, a candidate cut down to some ops, candidates joined by op, and one op's
// implementation tiled from several candidates, each running in its own range of a var. A manifest has no
// control flow, so "this kernel up to 32 rows, that one above" is every launch of the first under `when` up
// to 32 and every launch of the second under `when` from 33. Their output is a candidate's JSON with
// modules and ops in name order; each op and launch keeps its own text except for the parts renamed or
// narrowed.
#include <algorithm>
#include <cstdio>
#include <cstring>
#include <map>
#include <set>
#include <string>
#include <vector>

#include "../../include/kern_amd.h"
#include "json.h"

int kern_amd_fail(int code, const char* fmt, ...);

namespace {

using kern_json::JVal;

std::string span(const std::string& src, const JVal& v) { return src.substr(v.off, v.len); }

std::string quote(const std::string& s) {
  std::string o = "\"";
  for (unsigned char c : s) {
    if (c == '"' || c == '\\') {
      o += '\\';
      o += (char)c;
    } else if (c < 0x20) {
      char b[8];
      snprintf(b, sizeof b, "\\u%04x", c);
      o += b;
    } else {
      o += (char)c;
    }
  }
  return o + "\"";
}

// the module names an op's kernel launches name (extern launches name none)
std::set<std::string> launched(const JVal& op) {
  std::set<std::string> out;
  const JVal* im = op.get("impl");
  const JVal* ls = im ? im->get("launches") : nullptr;
  if (ls && ls->kind == JVal::Arr)
    for (const JVal& l : ls->a)
      if (const JVal* m = l.get("module"))
        if (m->kind == JVal::Str) out.insert(m->s);
  return out;
}

// the op's params as the reference lists them in its error (types.rs ParamType display: the strings)
std::string param_list(const JVal* ps) {
  std::string o;
  if (!ps || ps->kind != JVal::Arr) return o;
  for (size_t i = 0; i < ps->a.size(); ++i) o += (i ? ", " : "") + (ps->a[i].kind == JVal::Str ? ps->a[i].s : "?");
  return o;
}

bool same_params(const JVal* a, const JVal* b) {
  if (!a || !b || a->kind != JVal::Arr || b->kind != JVal::Arr || a->a.size() != b->a.size()) return false;
  for (size_t i = 0; i < a->a.size(); ++i)
    if (a->a[i].kind != JVal::Str || b->a[i].kind != JVal::Str || a->a[i].s != b->a[i].s) return false;
  return true;
}

std::string module_sha(const JVal& m) {
  const JVal* s = m.get("sha256");
  return s && s->kind == JVal::Str ? s->s : std::string();
}

// the text of an op with its launches' modules renamed as `names` says (the rest of the text unchanged)
std::string renamed_op(const std::string& src, const JVal& op, const std::map<std::string, std::string>& names) {
  auto rename = [&](const JVal& l) {
    std::string o = "{";
    for (size_t i = 0; i < l.o.size(); ++i) {
      const auto& kv = l.o[i];
      o += (i ? ", " : "") + quote(kv.first) + ": ";
      auto it = kv.first == "module" && kv.second.kind == JVal::Str ? names.find(kv.second.s) : names.end();
      o += it != names.end() ? quote(it->second) : span(src, kv.second);
    }
    return o + "}";
  };
  std::string o = "{";
  for (size_t i = 0; i < op.o.size(); ++i) {
    const auto& kv = op.o[i];
    o += (i ? ", " : "") + quote(kv.first) + ": ";
    if (kv.first != "impl" || kv.second.kind != JVal::Obj) {
      o += span(src, kv.second);
      continue;
    }
    o += "{";
    for (size_t j = 0; j < kv.second.o.size(); ++j) {
      const auto& ikv = kv.second.o[j];
      o += (j ? ", " : "") + quote(ikv.first) + ": ";
      if (ikv.first != "launches" || ikv.second.kind != JVal::Arr) {
        o += span(src, ikv.second);
        continue;
      }
      o += "[";
      for (size_t k = 0; k < ikv.second.a.size(); ++k)
        o += (k ? ", " : "") + (ikv.second.a[k].kind == JVal::Obj ? rename(ikv.second.a[k]) : span(src, ikv.second.a[k]));
      o += "]";
    }
    o += "}";
  }
  return o + "}";
}

}  // namespace

extern "C" int kern_candidate_splice(const char* manifest_json, const char* candidate_json, char* out, size_t cap,
                                     size_t* out_len) {
  if (!manifest_json || !candidate_json || !out_len)
    return kern_amd_fail(KERN_ERR_API, "kern_candidate_splice: null argument");
  const std::string msrc = manifest_json, csrc = candidate_json;
  JVal m, c;
  std::string err;
  if (!kern_json::parse_json(manifest_json, m, err) || m.kind != JVal::Obj)
    return kern_amd_fail(KERN_ERR_MANIFEST, "manifest: %s", err.empty() ? "expected an object" : err.c_str());
  if (!kern_json::parse_json(candidate_json, c, err) || c.kind != JVal::Obj)
    return kern_amd_fail(KERN_ERR_MANIFEST, "candidate: %s", err.empty() ? "expected an object" : err.c_str());
  // Candidate { modules (default empty), ops }, unknown fields refused (candidate.rs:34-44)
  for (const auto& kv : c.o)
    if (kv.first != "modules" && kv.first != "ops")
      return kern_amd_fail(KERN_ERR_MANIFEST, "candidate: unknown field `%s` (expected `modules`, `ops`)",
                           kv.first.c_str());
  const JVal* cops = c.get("ops");
  const JVal* cmods = c.get("modules");
  const JVal* mops = m.get("ops");
  const JVal* mmods = m.get("modules");
  if (!cops || cops->kind != JVal::Obj) return kern_amd_fail(KERN_ERR_MANIFEST, "candidate: missing `ops` object");
  if (cmods && cmods->kind != JVal::Obj) return kern_amd_fail(KERN_ERR_MANIFEST, "candidate: `modules` must be an object");
  if (!mops || mops->kind != JVal::Obj || !mmods || mmods->kind != JVal::Obj)
    return kern_amd_fail(KERN_ERR_MANIFEST, "manifest: missing `ops` or `modules` object");

  // the interface check, every reason collected (candidate.rs:153-176)
  std::vector<std::string> errs;
  if (cops->o.empty()) errs.push_back("no ops");
  for (const auto& kv : cops->o) {
    const JVal* have = mops->get(kv.first.c_str());
    if (!have) {
      errs.push_back("op `" + kv.first + "`: the manifest has no such op");
    } else if (!same_params(kv.second.get("params"), have->get("params"))) {
      errs.push_back("op `" + kv.first + "`: params [" + param_list(kv.second.get("params")) +
                     "] are not the manifest's [" + param_list(have->get("params")) + "]");
    }
    for (const std::string& mod : launched(kv.second))
      if (!(cmods && cmods->get(mod.c_str())) && !mmods->get(mod.c_str()))
        errs.push_back("op `" + kv.first + "`: module `" + mod + "` is in neither the candidate nor the manifest");
  }
  if (!errs.empty()) {
    std::string msg = "candidate does not fit:";
    for (const auto& e : errs) msg += "\n  - " + e;
    return kern_amd_fail(KERN_ERR_MANIFEST, "%s", msg.c_str());
  }

  // modules: the manifest's, then the candidate's under their own name or <name>@<hash prefix> when the
  // manifest has that name for other bytes (adopt, candidate.rs:116-131; the candidate's in name order, as
  // its BTreeMap iterates)
  std::vector<std::pair<std::string, std::string>> modules;  // name -> JSON text, manifest order first
  std::map<std::string, std::string> mod_sha, names;
  for (const auto& kv : mmods->o) modules.emplace_back(kv.first, span(msrc, kv.second)), mod_sha[kv.first] = module_sha(kv.second);
  if (cmods) {
    std::vector<const std::pair<std::string, JVal>*> sorted;
    for (const auto& kv : cmods->o) sorted.push_back(&kv);
    std::sort(sorted.begin(), sorted.end(), [](auto* a, auto* b) { return a->first < b->first; });
    for (const auto* kv : sorted) {
      const std::string sha = module_sha(kv->second);
      const bool taken = mod_sha.count(kv->first) && mod_sha[kv->first] != sha;
      const std::string as_name = taken ? kv->first + "@" + sha.substr(0, 8) : kv->first;
      if (!mod_sha.count(as_name)) modules.emplace_back(as_name, span(csrc, kv->second)), mod_sha[as_name] = sha;
      names[kv->first] = as_name;
    }
  }
  // ops: the manifest's, each the candidate listed replaced by its (renamed) implementation
  std::vector<std::pair<std::string, std::string>> ops;
  std::set<std::string> used;
  for (const auto& kv : mops->o) {
    if (const JVal* rep = cops->get(kv.first.c_str())) {
      ops.emplace_back(kv.first, renamed_op(csrc, *rep, names));
      for (const std::string& mod : launched(*rep)) used.insert(names.count(mod) ? names[mod] : mod);
    } else {
      ops.emplace_back(kv.first, span(msrc, kv.second));
      for (const std::string& mod : launched(kv.second)) used.insert(mod);
    }
  }
  // the manifest, with modules nothing launches any more dropped (candidate.rs:182-183)
  std::string o = "{";
  for (size_t i = 0; i < m.o.size(); ++i) {
    const auto& kv = m.o[i];
    o += (i ? ",\n" : "\n") + quote(kv.first) + ": ";
    if (kv.first == "modules") {
      o += "{";
      bool first = true;
      for (const auto& mk : modules)
        if (used.count(mk.first)) o += (first ? "\n  " : ",\n  ") + quote(mk.first) + ": " + mk.second, first = false;
      o += "}";
    } else if (kv.first == "ops") {
      o += "{";
      for (size_t j = 0; j < ops.size(); ++j) o += (j ? ",\n  " : "\n  ") + quote(ops[j].first) + ": " + ops[j].second;
      o += "}";
    } else {
      o += span(msrc, kv.second);
    }
  }
  o += "\n}\n";
  *out_len = o.size();
  if (!out) return KERN_OK;  // size query
  if (cap < o.size() + 1)
    return kern_amd_fail(KERN_ERR_API, "kern_candidate_splice: output needs %zu bytes, buffer has %zu", o.size() + 1, cap);
  memcpy(out, o.c_str(), o.size() + 1);
  return KERN_OK;
}

// ================================================================================== building candidates
namespace {

typedef std::map<std::string, std::string> Names;

// a candidate under construction: modules and ops as JSON text by name (name order, as the reference's
// BTreeMaps), and each module's sha256
struct Cand {
  std::map<std::string, std::string> modules, sha, ops;
};

// one parsed input, its text kept for the spans
struct Doc {
  std::string src;
  JVal v;
};

// compact JSON of a value, to compare two values independently of their spacing
std::string canon(const JVal& v) {
  switch (v.kind) {
    case JVal::Null: return "null";
    case JVal::Bool: return v.b ? "true" : "false";
    case JVal::Int: return v.is_u64 ? std::to_string(v.u) : std::to_string(v.i);
    case JVal::Float: {
      char b[40];
      snprintf(b, sizeof b, "%.17g", v.f);
      return b;
    }
    case JVal::Str: return quote(v.s);
    case JVal::Arr: {
      std::string o = "[";
      for (size_t i = 0; i < v.a.size(); ++i) o += (i ? "," : "") + canon(v.a[i]);
      return o + "]";
    }
    case JVal::Obj: {
      std::string o = "{";
      for (size_t i = 0; i < v.o.size(); ++i) o += (i ? "," : "") + quote(v.o[i].first) + ":" + canon(v.o[i].second);
      return o + "}";
    }
  }
  return "null";
}

std::string fit_errors(const std::vector<std::string>& errs) {
  std::string msg = "candidate does not fit:";
  for (const auto& e : errs) msg += "\n  - " + e;
  return msg;
}

int emit(const std::string& o, char* out, size_t cap, size_t* out_len, const char* fn) {
  *out_len = o.size();
  if (!out) return KERN_OK;  // size query
  if (cap < o.size() + 1)
    return kern_amd_fail(KERN_ERR_API, "%s: output needs %zu bytes, buffer has %zu", fn, o.size() + 1, cap);
  memcpy(out, o.c_str(), o.size() + 1);
  return KERN_OK;
}

std::string cand_json(const Cand& c) {
  std::string o = "{\n\"modules\": {";
  bool first = true;
  for (const auto& kv : c.modules) o += (first ? "\n  " : ",\n  ") + quote(kv.first) + ": " + kv.second, first = false;
  o += "},\n\"ops\": {";
  first = true;
  for (const auto& kv : c.ops) o += (first ? "\n  " : ",\n  ") + quote(kv.first) + ": " + kv.second, first = false;
  return o + "}\n}\n";
}

// a candidate's text: an object of `modules` (optional) and `ops` objects and nothing else (candidate.rs:34-44)
bool parse_candidate(const char* text, Doc& d, std::string& err) {
  d.src = text;
  if (!kern_json::parse_json(text, d.v, err) || d.v.kind != JVal::Obj)
    return err = "candidate: " + (err.empty() ? std::string("expected an object") : err), false;
  for (const auto& kv : d.v.o)
    if (kv.first != "modules" && kv.first != "ops")
      return err = "candidate: unknown field `" + kv.first + "` (expected `modules`, `ops`)", false;
  const JVal* ops = d.v.get("ops");
  const JVal* mods = d.v.get("modules");
  if (!ops || ops->kind != JVal::Obj) return err = "candidate: missing `ops` object", false;
  if (mods && mods->kind != JVal::Obj) return err = "candidate: `modules` must be an object", false;
  return true;
}

// `more`'s modules taken into `into` (adopt, candidate.rs:116-131): each under its own name, or under
// `<name>@<sha256[0:8]>` when `into` has that name for other bytes; returns what each name became
Names adopt(Cand& into, const Doc& d, const JVal* more) {
  Names names;
  if (!more) return names;
  std::vector<const std::pair<std::string, JVal>*> sorted;
  for (const auto& kv : more->o) sorted.push_back(&kv);
  std::sort(sorted.begin(), sorted.end(), [](auto* a, auto* b) { return a->first < b->first; });
  for (const auto* kv : sorted) {
    const std::string sha = module_sha(kv->second);
    const bool taken = into.sha.count(kv->first) && into.sha[kv->first] != sha;
    const std::string as_name = taken ? kv->first + "@" + sha.substr(0, 8) : kv->first;
    if (!into.modules.count(as_name)) into.modules[as_name] = span(d.src, kv->second), into.sha[as_name] = sha;
    names[kv->first] = as_name;
  }
  return names;
}

// Candidate::only (candidate.rs:89-97): the ops named that `ops_obj` has, with the modules (of `mods_obj`)
// their launches name
Cand only(const Doc& d, const JVal* ops_obj, const JVal* mods_obj, const char* const* names, int n) {
  Cand c;
  std::set<std::string> used;
  for (int i = 0; i < n; ++i) {
    const JVal* op = names[i] ? ops_obj->get(names[i]) : nullptr;
    if (!op) continue;
    c.ops[names[i]] = span(d.src, *op);
    for (const std::string& m : launched(*op)) used.insert(m);
  }
  for (const std::string& m : used)
    if (const JVal* mv = mods_obj ? mods_obj->get(m.c_str()) : nullptr)
      c.modules[m] = span(d.src, *mv), c.sha[m] = module_sha(*mv);
  return c;
}

// `v` with every string member named "scratch" renamed as `names` says (launch args and pack fields); the
// names it refers to afterwards go to `wired`
std::string rescratch(const std::string& src, const JVal& v, const Names& names, std::set<std::string>& wired) {
  if (v.kind == JVal::Arr) {
    std::string o = "[";
    for (size_t i = 0; i < v.a.size(); ++i) o += (i ? ", " : "") + rescratch(src, v.a[i], names, wired);
    return o + "]";
  }
  if (v.kind != JVal::Obj) return span(src, v);
  std::string o = "{";
  for (size_t i = 0; i < v.o.size(); ++i) {
    const auto& kv = v.o[i];
    o += (i ? ", " : "") + quote(kv.first) + ": ";
    if (kv.first == "scratch" && kv.second.kind == JVal::Str) {
      auto it = names.find(kv.second.s);
      const std::string to = it != names.end() ? it->second : kv.second.s;
      wired.insert(to);
      o += quote(to);
    } else {
      o += rescratch(src, kv.second, names, wired);
    }
  }
  return o + "}";
}

bool u64_of(const JVal* v, uint64_t& out) {
  if (!v || v->kind != JVal::Int || (v->i < 0 && !v->is_u64)) return false;
  out = v->u;
  return true;
}

}  // namespace

extern "C" int kern_candidate_of(const char* manifest_json, const char* const* ops, int n_ops, char* out, size_t cap,
                                 size_t* out_len) {
  if (!manifest_json || (n_ops > 0 && !ops) || n_ops < 0 || !out_len)
    return kern_amd_fail(KERN_ERR_API, "kern_candidate_of: null argument");
  Doc d;
  std::string err;
  d.src = manifest_json;
  if (!kern_json::parse_json(manifest_json, d.v, err) || d.v.kind != JVal::Obj)
    return kern_amd_fail(KERN_ERR_MANIFEST, "manifest: %s", err.empty() ? "expected an object" : err.c_str());
  const JVal* mops = d.v.get("ops");
  const JVal* mmods = d.v.get("modules");
  if (!mops || mops->kind != JVal::Obj || !mmods || mmods->kind != JVal::Obj)
    return kern_amd_fail(KERN_ERR_MANIFEST, "manifest: missing `ops` or `modules` object");
  return emit(cand_json(only(d, mops, mmods, ops, n_ops)), out, cap, out_len, "kern_candidate_of");
}

extern "C" int kern_candidate_only(const char* candidate_json, const char* const* ops, int n_ops, char* out,
                                   size_t cap, size_t* out_len) {
  if (!candidate_json || (n_ops > 0 && !ops) || n_ops < 0 || !out_len)
    return kern_amd_fail(KERN_ERR_API, "kern_candidate_only: null argument");
  Doc d;
  std::string err;
  if (!parse_candidate(candidate_json, d, err)) return kern_amd_fail(KERN_ERR_MANIFEST, "%s", err.c_str());
  return emit(cand_json(only(d, d.v.get("ops"), d.v.get("modules"), ops, n_ops)), out, cap, out_len,
              "kern_candidate_only");
}

extern "C" int kern_candidate_join(const char* const* candidates, int n, char* out, size_t cap, size_t* out_len) {
  if ((n > 0 && !candidates) || n < 0 || !out_len) return kern_amd_fail(KERN_ERR_API, "kern_candidate_join: null argument");
  std::vector<Doc> docs(n);
  Cand all;
  std::vector<std::string> errs;
  for (int i = 0; i < n; ++i) {
    std::string err;
    if (!candidates[i]) return kern_amd_fail(KERN_ERR_API, "kern_candidate_join: candidate %d is null", i);
    if (!parse_candidate(candidates[i], docs[i], err))
      return kern_amd_fail(KERN_ERR_MANIFEST, "candidate %d: %s", i, err.c_str());
    const Names names = adopt(all, docs[i], docs[i].v.get("modules"));
    std::vector<const std::pair<std::string, JVal>*> sorted;
    for (const auto& kv : docs[i].v.get("ops")->o) sorted.push_back(&kv);
    std::sort(sorted.begin(), sorted.end(), [](auto* a, auto* b) { return a->first < b->first; });
    for (const auto* kv : sorted) {
      if (all.ops.count(kv->first)) errs.push_back("op `" + kv->first + "` is implemented twice");
      else all.ops[kv->first] = renamed_op(docs[i].src, kv->second, names);
    }
  }
  if (!errs.empty()) return kern_amd_fail(KERN_ERR_MANIFEST, "%s", fit_errors(errs).c_str());
  return emit(cand_json(all), out, cap, out_len, "kern_candidate_join");
}

extern "C" int kern_candidate_tile(const char* op, const char* var, const kern_candidate_piece* pieces, int n,
                                   char* out, size_t cap, size_t* out_len) {
  if (!op || !var || (n > 0 && !pieces) || n < 0 || !out_len)
    return kern_amd_fail(KERN_ERR_API, "kern_candidate_tile: null argument");
  std::vector<Doc> docs(n);
  Cand c;
  std::vector<std::string> errs, launches;
  std::map<std::string, std::pair<std::string, std::string>> scratch;  // name -> (canonical, text)
  std::set<std::string> wired, used;
  const JVal* params = nullptr;
  std::string params_text;
  const std::string sop = op, svar = var;
  for (int i = 0; i < n; ++i) {
    std::string err;
    if (!pieces[i].candidate_json) return kern_amd_fail(KERN_ERR_API, "kern_candidate_tile: piece %d is null", i);
    if (!parse_candidate(pieces[i].candidate_json, docs[i], err))
      return kern_amd_fail(KERN_ERR_MANIFEST, "piece %d: %s", i, err.c_str());
    const Doc& d = docs[i];
    const std::string pi = "piece " + std::to_string(i);
    const JVal* have = d.v.get("ops")->get(op);
    if (!have) {
      errs.push_back(pi + ": no op `" + sop + "`");
      continue;
    }
    if (!params) params = have->get("params"), params_text = params ? span(d.src, *params) : "[]";
    else if (!same_params(params, have->get("params")))
      errs.push_back(pi + ": op `" + sop + "` has other params than piece 0");
    const Names modules = adopt(c, d, d.v.get("modules"));
    const JVal* im = have->get("impl");
    // the piece's scratch: under its own name, or <name>@<piece> where an earlier piece has the name for
    // another dtype or shape
    Names sn;
    if (const JVal* sc = im ? im->get("scratch") : nullptr) {
      if (sc->kind != JVal::Obj) return kern_amd_fail(KERN_ERR_MANIFEST, "%s: op `%s`: `scratch` must be an object", pi.c_str(), op);
      std::vector<const std::pair<std::string, JVal>*> sorted;
      for (const auto& kv : sc->o) sorted.push_back(&kv);
      std::sort(sorted.begin(), sorted.end(), [](auto* a, auto* b) { return a->first < b->first; });
      for (const auto* kv : sorted) {
        const std::string key = canon(kv->second);
        auto it = scratch.find(kv->first);
        const std::string as_name = it != scratch.end() && it->second.first != key ? kv->first + "@" + std::to_string(i) : kv->first;
        if (!scratch.count(as_name)) scratch[as_name] = {key, span(d.src, kv->second)};
        sn[kv->first] = as_name;
      }
    }
    const JVal* ls = im ? im->get("launches") : nullptr;
    if (!ls || ls->kind != JVal::Arr) return kern_amd_fail(KERN_ERR_MANIFEST, "%s: op `%s`: missing `launches`", pi.c_str(), op);
    for (const JVal& l : ls->a) {
      if (l.kind != JVal::Obj) return kern_amd_fail(KERN_ERR_MANIFEST, "%s: op `%s`: a launch must be an object", pi.c_str(), op);
      // narrow (candidate.rs:189-212): the launch's own range of the var, cut to the piece's
      bool has_lo = pieces[i].has_min != 0, has_hi = pieces[i].has_max != 0;
      uint64_t lo = pieces[i].min, hi = pieces[i].max;
      if (const JVal* w = l.get("when")) {
        const JVal* wv = w->get("var");
        const JVal* en = l.get("entry");
        const std::string entry = en && en->kind == JVal::Str ? en->s : "?";
        if (!wv || wv->kind != JVal::Str) return kern_amd_fail(KERN_ERR_MANIFEST, "%s: launch `%s`: `when` needs a var", pi.c_str(), entry.c_str());
        if (wv->s != svar) {
          errs.push_back(pi + ": op `" + sop + "`: launch `" + entry + "` runs in a range of `" + wv->s + "`, not of `" + svar + "`");
          continue;
        }
        uint64_t x;
        for (const char* end : {"min", "max"})
          if (w->get(end) && !u64_of(w->get(end), x))
            return kern_amd_fail(KERN_ERR_MANIFEST, "%s: launch `%s`: when.%s must be a non-negative integer",
                                 pi.c_str(), entry.c_str(), end);
        if (u64_of(w->get("min"), x)) lo = has_lo ? std::max(lo, x) : x, has_lo = true;
        if (u64_of(w->get("max"), x)) hi = has_hi ? std::min(hi, x) : x, has_hi = true;
      }
      if (has_lo && has_hi && lo > hi) continue;  // never runs in the piece's range
      if (has_lo && lo <= 1) has_lo = false;      // a var is at least 1: a lower end of 1 is no bound
      std::string when;
      if (has_lo || has_hi) {
        when = "{\"var\": " + quote(svar);
        if (has_lo) when += ", \"min\": " + std::to_string(lo);
        if (has_hi) when += ", \"max\": " + std::to_string(hi);
        when += "}";
      }
      // the launch's text: module renamed, `when` replaced, scratch arguments renamed
      std::string o = "{";
      bool first = true, put_when = false;
      for (const auto& kv : l.o) {
        std::string val;
        if (kv.first == "when") {
          if (when.empty()) continue;
          val = when, put_when = true;
        } else if (kv.first == "module" && kv.second.kind == JVal::Str) {
          auto it = modules.find(kv.second.s);
          const std::string mod = it != modules.end() ? it->second : kv.second.s;
          used.insert(mod);
          val = quote(mod);
        } else if (kv.first == "args") {
          val = rescratch(d.src, kv.second, sn, wired);
        } else {
          val = span(d.src, kv.second);
        }
        o += (first ? "" : ", ") + quote(kv.first) + ": " + val, first = false;
      }
      if (!when.empty() && !put_when) o += (first ? "" : ", ") + std::string("\"when\": ") + when;
      launches.push_back(o + "}");
    }
  }
  if (errs.empty() && launches.empty())
    errs.push_back("op `" + sop + "`: no launch of any piece runs in its range of `" + svar + "`");
  if (!errs.empty() || !params) {
    if (errs.empty()) errs.push_back("no pieces");
    return kern_amd_fail(KERN_ERR_MANIFEST, "%s", fit_errors(errs).c_str());
  }
  for (auto it = c.modules.begin(); it != c.modules.end();) it = used.count(it->first) ? std::next(it) : c.modules.erase(it);
  std::string o = "{\"params\": " + params_text + ", \"impl\": {";
  std::string sc;
  for (const auto& kv : scratch)
    if (wired.count(kv.first)) sc += (sc.empty() ? "" : ", ") + quote(kv.first) + ": " + kv.second.second;
  if (!sc.empty()) o += "\"scratch\": {" + sc + "}, ";
  o += "\"launches\": [";
  for (size_t j = 0; j < launches.size(); ++j) o += (j ? ",\n    " : "\n    ") + launches[j];
  o += "]}}";
  c.ops[sop] = o;
  return emit(cand_json(c), out, cap, out_len, "kern_candidate_tile");
}
