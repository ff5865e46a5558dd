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
