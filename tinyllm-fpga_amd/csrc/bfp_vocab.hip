// Token-id -> text: the "BFPV" vocabulary table and the decoder that turns a
// generated id sequence into readable UTF-8.  Host code only.
//
// File format (written by rtl/vc707/host/gen_bfp_vocab_bin.py:10-17,69-74,
// read by rtl/vc707/host/bfp_client.cpp:876-903), little-endian:
//   "BFPV", u32 version (1), u32 n_tokens, u32 blob_size,
//   n_tokens x {u32 offset, u32 length}, blob_size bytes of raw token bytes.
//
// Decoding (bfp_client.cpp:905-1027): concatenate the tokens' raw bytes,
// read them as UTF-8 leniently (a byte that starts no complete sequence
// stands for itself as a code point), then repair "web mojibake": a run of
// code points that Windows-1252 maps to single bytes >= 0x80 is re-read as
// UTF-8 bytes, and replaced by that reading when every byte forms part of a
// sequence and at least one decoded code point lies above U+00FF.

#include <stdio.h>
#include <string.h>

#include <new>
#include <string>
#include <vector>

#include "bfp_internal.h"

struct bfp_vocab {
  std::vector<uint32_t> off, len;
  std::vector<uint8_t> blob;
};

namespace bfp {
namespace {

// One code point of s starting at *i (bfp_client.cpp:913-931).
uint32_t next_cp(const uint8_t *s, size_t n, size_t *i) {
  const uint32_t b = s[*i];
  int extra;
  uint32_t cp;
  if (b < 0x80) {
    ++*i;
    return b;
  } else if ((b & 0xe0) == 0xc0) {
    extra = 1, cp = b & 0x1f;
  } else if ((b & 0xf0) == 0xe0) {
    extra = 2, cp = b & 0x0f;
  } else if ((b & 0xf8) == 0xf0) {
    extra = 3, cp = b & 0x07;
  } else {
    ++*i;
    return b;
  }
  if (*i + extra + 1 > n) {  // sequence runs past the end
    ++*i;
    return b;
  }
  for (int k = 1; k <= extra; ++k) {
    const uint32_t c = s[*i + k];
    if ((c & 0xc0) != 0x80) {
      ++*i;
      return b;
    }
    cp = (cp << 6) | (c & 0x3f);
  }
  *i += extra + 1;
  return cp;
}

// UTF-8 encoding of a code point of up to 21 bits (bfp_client.cpp:933-944).
void put_cp(uint32_t cp, std::string &out) {
  if (cp < 0x80) {
    out.push_back((char)cp);
  } else if (cp < 0x800) {
    out.push_back((char)(0xc0 | (cp >> 6)));
    out.push_back((char)(0x80 | (cp & 0x3f)));
  } else if (cp < 0x10000) {
    out.push_back((char)(0xe0 | (cp >> 12)));
    out.push_back((char)(0x80 | ((cp >> 6) & 0x3f)));
    out.push_back((char)(0x80 | (cp & 0x3f)));
  } else {
    out.push_back((char)(0xf0 | (cp >> 18)));
    out.push_back((char)(0x80 | ((cp >> 12) & 0x3f)));
    out.push_back((char)(0x80 | ((cp >> 6) & 0x3f)));
    out.push_back((char)(0x80 | (cp & 0x3f)));
  }
}

// Windows-1252 byte of a code point, or -1 (bfp_client.cpp:950-969): the
// identity on U+0000..U+007F and U+00A0..U+00FF, and the 27 characters the
// code page places in 0x80..0x9F.
struct W1252 {
  uint16_t cp;
  uint8_t byte;
};
constexpr W1252 kW1252[] = {
    {0x0152, 0x8C}, {0x0153, 0x9C}, {0x0160, 0x8A}, {0x0161, 0x9A}, {0x0178, 0x9F},
    {0x017D, 0x8E}, {0x017E, 0x9E}, {0x0192, 0x83}, {0x02C6, 0x88}, {0x02DC, 0x98},
    {0x2013, 0x96}, {0x2014, 0x97}, {0x2018, 0x91}, {0x2019, 0x92}, {0x201A, 0x82},
    {0x201C, 0x93}, {0x201D, 0x94}, {0x201E, 0x84}, {0x2020, 0x86}, {0x2021, 0x87},
    {0x2022, 0x95}, {0x2026, 0x85}, {0x2030, 0x89}, {0x2039, 0x8B}, {0x203A, 0x9B},
    {0x20AC, 0x80}, {0x2122, 0x99}};

int w1252_byte(uint32_t cp) {
  if (cp < 0x80 || (cp >= 0xA0 && cp <= 0xFF)) return (int)cp;
  for (const W1252 &w : kW1252)
    if (w.cp == cp) return w.byte;
  return -1;
}

std::string repair(const std::string &raw) {
  const uint8_t *s = reinterpret_cast<const uint8_t *>(raw.data());
  std::vector<uint32_t> cps;
  for (size_t i = 0; i < raw.size();) cps.push_back(next_cp(s, raw.size(), &i));
  std::string out, bytes, dec;
  size_t i = 0;
  while (i < cps.size()) {
    if (w1252_byte(cps[i]) < 0x80) {  // ASCII, or no single-byte form
      put_cp(cps[i++], out);
      continue;
    }
    size_t j = i;
    bytes.clear();
    for (int b; j < cps.size() && (b = w1252_byte(cps[j])) >= 0x80; ++j) bytes.push_back((char)b);
    const uint8_t *bs = reinterpret_cast<const uint8_t *>(bytes.data());
    dec.clear();
    bool whole = true, wider = false;
    for (size_t k = 0; k < bytes.size();) {
      const size_t k0 = k;
      const uint32_t cp = next_cp(bs, bytes.size(), &k);
      if (k == k0 + 1 && bs[k0] >= 0x80) {  // a byte that starts no sequence
        whole = false;
        break;
      }
      wider |= cp > 0xFF;
      put_cp(cp, dec);
    }
    if (whole && wider)
      out += dec;
    else
      for (size_t k = i; k < j; ++k) put_cp(cps[k], out);
    i = j;
  }
  return out;
}

uint32_t rd32(const uint8_t *p) {
  return (uint32_t)p[0] | ((uint32_t)p[1] << 8) | ((uint32_t)p[2] << 16) | ((uint32_t)p[3] << 24);
}

}  // namespace
}  // namespace bfp

using namespace bfp;

extern "C" {

int bfp_vocab_parse(const void *buf, size_t n, bfp_vocab **out) {
  if (!buf || !out) return set_err(BFP_EINVAL, "vocab: null argument");
  *out = nullptr;
  const uint8_t *p = static_cast<const uint8_t *>(buf);
  if (n < 16 || memcmp(p, "BFPV", 4) != 0) return set_err(BFP_EINVAL, "vocab: bad magic");
  const uint32_t version = rd32(p + 4), nt = rd32(p + 8), nb = rd32(p + 12);
  if (version != 1) return set_err(BFP_EINVAL, "vocab: unsupported version %u", version);
  if ((n - 16) / 8 < nt || n - 16 - (size_t)nt * 8 < nb)
    return set_err(BFP_EINVAL, "vocab: truncated (%zu bytes for %u tokens, %u-byte blob)", n, nt,
                   nb);
  bfp_vocab *v = new (std::nothrow) bfp_vocab;
  if (!v) return set_err(BFP_ENOMEM, "vocab: out of host memory");
  try {
    v->off.resize(nt);
    v->len.resize(nt);
    for (uint32_t t = 0; t < nt; ++t) {
      v->off[t] = rd32(p + 16 + 8 * (size_t)t);
      v->len[t] = rd32(p + 20 + 8 * (size_t)t);
    }
    const uint8_t *b = p + 16 + 8 * (size_t)nt;
    v->blob.assign(b, b + nb);
  } catch (...) {
    delete v;
    return set_err(BFP_ENOMEM, "vocab: out of host memory");
  }
  *out = v;
  return BFP_OK;
}

int bfp_vocab_open(const char *path, bfp_vocab **out) {
  if (!path || !out) return set_err(BFP_EINVAL, "vocab: null argument");
  *out = nullptr;
  FILE *f = fopen(path, "rb");
  if (!f) return set_err(BFP_EINVAL, "vocab: cannot open %s", path);
  std::vector<uint8_t> buf;
  try {
    uint8_t chunk[1 << 16];
    size_t got;
    while ((got = fread(chunk, 1, sizeof chunk, f)) > 0) buf.insert(buf.end(), chunk, chunk + got);
  } catch (...) {
    fclose(f);
    return set_err(BFP_ENOMEM, "vocab: out of host memory");
  }
  const bool err = ferror(f);
  fclose(f);
  if (err) return set_err(BFP_EIO, "vocab: read error on %s", path);
  return bfp_vocab_parse(buf.data(), buf.size(), out);
}

void bfp_vocab_close(bfp_vocab *v) { delete v; }

int bfp_vocab_size(const bfp_vocab *v) { return v ? (int)v->off.size() : 0; }

int bfp_vocab_token(const bfp_vocab *v, int id, const char **bytes, size_t *len) {
  if (!v || !bytes || !len) return set_err(BFP_EINVAL, "vocab: null argument");
  *bytes = "";
  *len = 0;
  if (id < 0 || (size_t)id >= v->off.size()) return BFP_OK;
  const uint64_t o = v->off[id], l = v->len[id];
  if (o + l > v->blob.size()) return BFP_OK;
  *bytes = reinterpret_cast<const char *>(v->blob.data() + o);
  *len = (size_t)l;
  return BFP_OK;
}

long long bfp_vocab_decode(const bfp_vocab *v, const int32_t *ids, int n, char *out, size_t cap) {
  if (!v || n < 0 || (n > 0 && !ids)) return set_err(BFP_EINVAL, "vocab: bad arguments");
  try {
    std::string raw;
    for (int k = 0; k < n; ++k) {
      const char *b;
      size_t l;
      bfp_vocab_token(v, ids[k], &b, &l);
      raw.append(b, l);
    }
    const std::string text = repair(raw);
    if (out && cap > 0) {
      const size_t w = text.size() < cap - 1 ? text.size() : cap - 1;
      memcpy(out, text.data(), w);
      out[w] = '\0';
    }
    return (long long)text.size();
  } catch (...) {
    return set_err(BFP_ENOMEM, "vocab: out of host memory");
  }
}

}  // extern "C"
