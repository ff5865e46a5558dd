// Reads the explicit kernel-argument sizes of every entry from the AMDGPU metadata note
// (NT_AMDGPU_METADATA, msgpack) of a code object this project built itself. This is the data the
// launch ABI check compares against a manifest launch's declared params.
#pragma once
#include <stddef.h>
#include <stdint.h>
#include <string.h>

#include <map>
#include <string>
#include <vector>

namespace kern {

struct MsgPack {
  const uint8_t* p;
  const uint8_t* end;
  bool ok = true;

  uint64_t be(int n) {
    if (!ok || p > end || end - p < n) { ok = false; return 0; }
    uint64_t v = 0;
    for (int i = 0; i < n; ++i) v = (v << 8) | p[i];
    p += n;
    return v;
  }
  // kinds: 0 nil/bool/number, 1 string, 2 array, 3 map
  int head(uint64_t& n, int64_t& ival, std::string& s) {
    if (!ok || p >= end) { ok = false; return -1; }
    uint8_t t = *p++;
    if (t <= 0x7f) { ival = t; return 0; }
    if (t >= 0xe0) { ival = (int8_t)t; return 0; }
    if ((t & 0xf0) == 0x80) { n = t & 15; return 3; }
    if ((t & 0xf0) == 0x90) { n = t & 15; return 2; }
    if ((t & 0xe0) == 0xa0) { n = t & 31; return str(n, s); }
    switch (t) {
      case 0xc0: case 0xc2: case 0xc3: ival = t == 0xc3; return 0;
      case 0xc4: n = be(1); return bin(n);
      case 0xc5: n = be(2); return bin(n);
      case 0xc6: n = be(4); return bin(n);
      case 0xca: be(4); return 0;
      case 0xcb: be(8); return 0;
      case 0xcc: ival = (int64_t)be(1); return 0;
      case 0xcd: ival = (int64_t)be(2); return 0;
      case 0xce: ival = (int64_t)be(4); return 0;
      case 0xcf: ival = (int64_t)be(8); return 0;
      case 0xd0: ival = (int8_t)be(1); return 0;
      case 0xd1: ival = (int16_t)be(2); return 0;
      case 0xd2: ival = (int32_t)be(4); return 0;
      case 0xd3: ival = (int64_t)be(8); return 0;
      case 0xd9: n = be(1); return str(n, s);
      case 0xda: n = be(2); return str(n, s);
      case 0xdb: n = be(4); return str(n, s);
      case 0xdc: n = be(2); return 2;
      case 0xdd: n = be(4); return 2;
      case 0xde: n = be(2); return 3;
      case 0xdf: n = be(4); return 3;
    }
    ok = false;
    return -1;
  }
  // bytes left before `end` (0 once a read has failed or run past it)
  uint64_t left() const { return ok && p <= end ? (uint64_t)(end - p) : 0; }
  int str(uint64_t n, std::string& s) {
    if (!ok || left() < n) { ok = false; return -1; }
    s.assign(reinterpret_cast<const char*>(p), n);
    p += n;
    return 1;
  }
  // a bin8/16/32 payload, skipped
  int bin(uint64_t n) {
    if (!ok || left() < n) { ok = false; return -1; }
    p += n;
    return 0;
  }
  // skip one value; nesting deeper than any metadata this build writes is refused, not recursed into
  void skip(int depth = 0) {
    uint64_t n = 0; int64_t iv = 0; std::string s;
    int k = head(n, iv, s);
    if ((k == 2 || k == 3) && depth >= 32) { ok = false; return; }
    if (k == 2) for (uint64_t i = 0; i < n && ok; ++i) skip(depth + 1);
    if (k == 3) for (uint64_t i = 0; i < n && ok; ++i) { skip(depth + 1); if (ok) skip(depth + 1); }
  }
};

// one kernel map: collect .name and the explicit .args sizes and byte offsets
inline bool parse_kernel(MsgPack& m, uint64_t nkeys, std::string& name, std::vector<uint32_t>& sizes,
                         std::vector<uint32_t>& offsets) {
  for (uint64_t i = 0; i < nkeys && m.ok; ++i) {
    uint64_t n = 0; int64_t iv = 0; std::string key, val;
    if (m.head(n, iv, key) != 1) return false;
    if (key == ".name") {
      if (m.head(n, iv, val) != 1) return false;
      name = val;
    } else if (key == ".args") {
      uint64_t na = 0;
      if (m.head(na, iv, val) != 2) return false;
      for (uint64_t a = 0; a < na && m.ok; ++a) {
        uint64_t nk = 0;
        if (m.head(nk, iv, val) != 3) return false;
        int64_t size = -1, offset = -1;
        std::string kind;
        for (uint64_t q = 0; q < nk && m.ok; ++q) {
          std::string k2;
          if (m.head(n, iv, k2) != 1) return false;
          if (k2 == ".size") {
            std::string t;
            m.head(n, size, t);
          } else if (k2 == ".offset") {
            std::string t;
            m.head(n, offset, t);
          } else if (k2 == ".value_kind") {
            if (m.head(n, iv, kind) != 1) return false;
          } else {
            m.skip();
          }
        }
        if (kind.compare(0, 7, "hidden_") != 0) {
          // an explicit argument must state its size and offset, each within the kernarg segment's range
          if (size < 0 || offset < 0 || size > 4096 || offset > 65536) return false;
          sizes.push_back((uint32_t)size);
          offsets.push_back((uint32_t)offset);
        }
      }
    } else {
      m.skip();
    }
  }
  return m.ok;
}

inline bool read_kernel_params(const uint8_t* img, size_t len, std::map<std::string, std::vector<uint32_t>>& out,
                               std::string& err,
                               std::map<std::string, std::vector<uint32_t>>* offsets_out = nullptr) {
  if (len < 64 || memcmp(img, "\x7f" "ELF", 4) != 0 || img[4] != 2) { err = "not a 64-bit ELF"; return false; }
  uint64_t shoff; uint16_t shentsize, shnum;
  memcpy(&shoff, img + 0x28, 8);
  memcpy(&shentsize, img + 0x3a, 2);
  memcpy(&shnum, img + 0x3c, 2);
  // overflow-safe range checks throughout: an offset past the image, or a size past what is left after it
  if (shentsize < 0x28 || shoff > len || (uint64_t)shentsize * shnum > len - shoff) {
    err = "section headers out of range";
    return false;
  }
  for (int i = 0; i < shnum; ++i) {
    const uint8_t* sh = img + shoff + (uint64_t)i * shentsize;
    uint32_t type; uint64_t off, size;
    memcpy(&type, sh + 4, 4);
    memcpy(&off, sh + 0x18, 8);
    memcpy(&size, sh + 0x20, 8);
    if (type != 7 /* SHT_NOTE */ || off > len || size > len - off) continue;
    const uint8_t* p = img + off;
    const uint8_t* e = p + size;
    while (e - p >= 12) {
      uint32_t namesz, descsz, ntype;
      memcpy(&namesz, p, 4); memcpy(&descsz, p + 4, 4); memcpy(&ntype, p + 8, 4);
      const uint64_t name_pad = ((uint64_t)namesz + 3) & ~3ull, desc_pad = ((uint64_t)descsz + 3) & ~3ull;
      if (name_pad > (uint64_t)(e - p) - 12 || descsz > (uint64_t)(e - p) - 12 - name_pad) break;
      const uint8_t* name = p + 12;
      const uint8_t* desc = name + name_pad;
      if (ntype == 32 && namesz >= 6 && memcmp(name, "AMDGPU", 6) == 0) {
        MsgPack m{desc, desc + descsz};
        uint64_t nmap = 0, n = 0; int64_t iv = 0; std::string s;
        if (m.head(nmap, iv, s) != 3) { err = "metadata is not a map"; return false; }
        for (uint64_t k = 0; k < nmap && m.ok; ++k) {
          std::string key;
          if (m.head(n, iv, key) != 1) { err = "bad metadata key"; return false; }
          if (key == "amdhsa.kernels") {
            uint64_t nk = 0; std::string t;
            if (m.head(nk, iv, t) != 2) { err = "amdhsa.kernels is not an array"; return false; }
            for (uint64_t q = 0; q < nk && m.ok; ++q) {
              uint64_t nkeys = 0;
              if (m.head(nkeys, iv, t) != 3) { err = "kernel entry is not a map"; return false; }
              std::string name; std::vector<uint32_t> sizes, offsets;
              if (!parse_kernel(m, nkeys, name, sizes, offsets)) { err = "malformed kernel entry"; return false; }
              out[name] = sizes;
              if (offsets_out) (*offsets_out)[name] = offsets;
            }
          } else {
            m.skip();
          }
        }
        if (!m.ok) { err = "truncated metadata"; return false; }
        return true;
      }
      if (desc_pad > (uint64_t)(e - desc)) break;
      p = desc + desc_pad;
    }
  }
  err = "no NT_AMDGPU_METADATA note";
  return false;
}

}  // namespace kern
