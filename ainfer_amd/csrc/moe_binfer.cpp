// moe_binfer.cpp - reader, validator and layer loader of `.binfer` containers
// holding INT4 mixture-of-experts layers (host code).
//
// The container is the reference's v1 format (docs/binfer_spec.md): a
// 128-byte header, a section table of 32-byte entries, sections 1-4
// (identity, architecture, tokenizer, quantization policy) stored as a u64
// length and a body, section 5 the tensor directory (raw 192-byte entries),
// a scale pool, 64-byte aligned payloads and a trailing SHA-256 of every byte
// before it.  Validation follows the reference's loader rules
// (docs/binfer_spec.md:112-116, tools/binfer.py:383-499) and runs in full
// before anything is allocated; the first failure is reported with the
// tensor name and the expected and actual values.
//
// Additions, in fields the v1 spec reserves (docs/binfer_spec.md:118-121):
//  - layout_id 32 (the spec's experimental range, which a v1 reference loader
//    rejects): an INT4 tensor of shape [E][rows][K] holding the E experts'
//    [rows][K] matrices back to back, each row-major and packed as layout 0
//    (two nibbles per byte, low nibble = even k), its scales [E][rows][K/128]
//    contiguous in the scale pool.  This is the weight layout of
//    include/ainfer_moe.h, so a layer loads with one copy per tensor;
//  - byte 180 of a directory entry (the first reserved byte): the scale
//    dtype of an INT4 tensor, 0 = BF16 (the v1 default), 1 = FP16.
#include <hip/hip_runtime.h>
#include <stdio.h>
#include <string.h>

#include <algorithm>
#include <string>
#include <vector>

#include "../../include/ainfer_moe.h"

namespace {

constexpr uint8_t MAGIC[8] = {'B', 'I', 'N', 'F', 'E', 'R', 0, 1};
constexpr uint32_t VERSION = 1, ALIGN = 64, GROUP = 128;
constexpr int DIR_ENTRY = 192, SECT_ENTRY = 32;
enum { DT_BF16 = 0, DT_FP16 = 1, DT_FP32 = 2, DT_INT4 = 3, DT_INT8 = 4, DT_FP8 = 5 };
enum { LAYOUT_ROW_MAJOR = 0, LAYOUT_EXPERT_STACKED = AINFER_BINFER_LAYOUT_EXPERTS };

// ---- CRC-32 (IEEE 802.3, reflected polynomial 0xEDB88320), as zlib -------
uint32_t g_crc_table[256];
bool g_crc_init = false;
void crc_init() {
  if (g_crc_init) return;
  for (uint32_t i = 0; i < 256; ++i) {
    uint32_t c = i;
    for (int k = 0; k < 8; ++k) c = (c & 1) ? 0xEDB88320u ^ (c >> 1) : c >> 1;
    g_crc_table[i] = c;
  }
  g_crc_init = true;
}
uint32_t crc32_update(uint32_t crc, const uint8_t *p, size_t n) {
  crc = ~crc;
  for (size_t i = 0; i < n; ++i) crc = g_crc_table[(crc ^ p[i]) & 0xFF] ^ (crc >> 8);
  return ~crc;
}

// ---- SHA-256 (FIPS 180-4) ---------------------------------------------------
struct Sha256 {
  uint32_t h[8] = {0x6a09e667, 0xbb67ae85, 0x3c6ef372, 0xa54ff53a,
                   0x510e527f, 0x9b05688c, 0x1f83d9ab, 0x5be0cd19};
  uint8_t buf[64];
  size_t nbuf = 0;
  uint64_t len = 0;
  static uint32_t rotr(uint32_t x, int n) { return (x >> n) | (x << (32 - n)); }
  void block(const uint8_t *p) {
    static const uint32_t K[64] = {
        0x428a2f98, 0x71374491, 0xb5c0fbcf, 0xe9b5dba5, 0x3956c25b, 0x59f111f1, 0x923f82a4,
        0xab1c5ed5, 0xd807aa98, 0x12835b01, 0x243185be, 0x550c7dc3, 0x72be5d74, 0x80deb1fe,
        0x9bdc06a7, 0xc19bf174, 0xe49b69c1, 0xefbe4786, 0x0fc19dc6, 0x240ca1cc, 0x2de92c6f,
        0x4a7484aa, 0x5cb0a9dc, 0x76f988da, 0x983e5152, 0xa831c66d, 0xb00327c8, 0xbf597fc7,
        0xc6e00bf3, 0xd5a79147, 0x06ca6351, 0x14292967, 0x27b70a85, 0x2e1b2138, 0x4d2c6dfc,
        0x53380d13, 0x650a7354, 0x766a0abb, 0x81c2c92e, 0x92722c85, 0xa2bfe8a1, 0xa81a664b,
        0xc24b8b70, 0xc76c51a3, 0xd192e819, 0xd6990624, 0xf40e3585, 0x106aa070, 0x19a4c116,
        0x1e376c08, 0x2748774c, 0x34b0bcb5, 0x391c0cb3, 0x4ed8aa4a, 0x5b9cca4f, 0x682e6ff3,
        0x748f82ee, 0x78a5636f, 0x84c87814, 0x8cc70208, 0x90befffa, 0xa4506ceb, 0xbef9a3f7,
        0xc67178f2};
    uint32_t w[64];
    for (int i = 0; i < 16; ++i)
      w[i] = (uint32_t)p[4 * i] << 24 | (uint32_t)p[4 * i + 1] << 16 | (uint32_t)p[4 * i + 2] << 8 |
             p[4 * i + 3];
    for (int i = 16; i < 64; ++i) {
      const uint32_t s0 = rotr(w[i - 15], 7) ^ rotr(w[i - 15], 18) ^ (w[i - 15] >> 3);
      const uint32_t s1 = rotr(w[i - 2], 17) ^ rotr(w[i - 2], 19) ^ (w[i - 2] >> 10);
      w[i] = w[i - 16] + s0 + w[i - 7] + s1;
    }
    uint32_t a = h[0], b = h[1], c = h[2], d = h[3], e = h[4], f = h[5], g = h[6], hh = h[7];
    for (int i = 0; i < 64; ++i) {
      const uint32_t S1 = rotr(e, 6) ^ rotr(e, 11) ^ rotr(e, 25);
      const uint32_t ch = (e & f) ^ (~e & g);
      const uint32_t t1 = hh + S1 + ch + K[i] + w[i];
      const uint32_t S0 = rotr(a, 2) ^ rotr(a, 13) ^ rotr(a, 22);
      const uint32_t mj = (a & b) ^ (a & c) ^ (b & c);
      const uint32_t t2 = S0 + mj;
      hh = g; g = f; f = e; e = d + t1; d = c; c = b; b = a; a = t1 + t2;
    }
    h[0] += a; h[1] += b; h[2] += c; h[3] += d; h[4] += e; h[5] += f; h[6] += g; h[7] += hh;
  }
  void update(const uint8_t *p, size_t n) {
    len += n;
    while (n > 0) {
      const size_t take = std::min(n, (size_t)64 - nbuf);
      memcpy(buf + nbuf, p, take);
      nbuf += take;
      p += take;
      n -= take;
      if (nbuf == 64) {
        block(buf);
        nbuf = 0;
      }
    }
  }
  void finish(uint8_t out[32]) {
    const uint64_t bits = len * 8;
    const uint8_t pad = 0x80;
    update(&pad, 1);
    const uint8_t zero = 0;
    while (nbuf != 56) update(&zero, 1);
    uint8_t lb[8];
    for (int i = 0; i < 8; ++i) lb[i] = (uint8_t)(bits >> (56 - 8 * i));
    update(lb, 8);
    for (int i = 0; i < 8; ++i)
      for (int j = 0; j < 4; ++j) out[4 * i + j] = (uint8_t)(h[i] >> (24 - 8 * j));
  }
};

template <typename T>
T rd(const uint8_t *p) {
  T v;
  memcpy(&v, p, sizeof v);
  return v;
}

struct Entry {
  std::string name;
  int ndim = 0;
  uint64_t shape[8] = {};
  int logical = 0, storage = 0, layout = 0, scale_dtype = 0;
  uint32_t group = 0;
  uint64_t sc_off = 0, sc_bytes = 0, d_off = 0, d_bytes = 0;
  uint32_t crc = 0;
  // Element count, or UINT64_MAX when the product of the dims overflows 64 bits
  // (every caller then rejects the shape as implausible).
  uint64_t numel() const {
    uint64_t n = 1;
    for (int i = 0; i < ndim; ++i)
      if (__builtin_mul_overflow(n, shape[i], &n)) return UINT64_MAX;
    return n;
  }
};

bool is_visual(const std::string &n) {
  return n.find(".visual.") != std::string::npos || n.find(".merger.") != std::string::npos ||
         n.find("patch_embed") != std::string::npos || n.find("pos_embed") != std::string::npos;
}

int dtype_bytes(int dt) {
  switch (dt) {
  case DT_BF16: case DT_FP16: return 2;
  case DT_FP32: return 4;
  case DT_INT8: case DT_FP8: return 1;
  default: return 0;
  }
}

}  // namespace

struct ainfer_binfer {
  FILE *f = nullptr;
  uint64_t size = 0;
  std::vector<Entry> entries;
  std::string arch;  // section 2 body (JSON)
  std::string err;
};

namespace {

int fail(ainfer_binfer *b, const std::string &msg) {
  if (b->err.empty()) b->err = msg;
  return AINFER_ERR_FORMAT;
}

bool read_at(FILE *f, uint64_t off, void *dst, size_t n) {
  if (fseeko(f, (off_t)off, SEEK_SET) != 0) return false;
  return fread(dst, 1, n, f) == n;
}

// Every rule before anything is allocated (docs/binfer_spec.md:112-116).
int validate(ainfer_binfer *b) {
  crc_init();
  uint8_t hdr[128];
  if (b->size < 128 + 32 || !read_at(b->f, 0, hdr, 128))
    return fail(b, "truncated: file shorter than the 128-byte header and trailing SHA-256");
  if (memcmp(hdr, MAGIC, 8) != 0) return fail(b, "bad magic");
  if (rd<uint32_t>(hdr + 8) != VERSION)
    return fail(b, "bad version: expected 1, got " + std::to_string(rd<uint32_t>(hdr + 8)));
  const uint32_t flags = rd<uint32_t>(hdr + 12);
  if (flags & ~1u) return fail(b, "reserved flags set: " + std::to_string(flags));
  const uint64_t n = rd<uint64_t>(hdr + 16), table_off = rd<uint64_t>(hdr + 24);
  const uint32_t scount = rd<uint32_t>(hdr + 32);
  if (rd<uint32_t>(hdr + 36) != ALIGN)
    return fail(b, "bad alignment field: expected 64, got " + std::to_string(rd<uint32_t>(hdr + 36)));
  const uint64_t total = rd<uint64_t>(hdr + 40);
  if (total != b->size)
    return fail(b, "total mismatch: header " + std::to_string(total) + ", file " +
                       std::to_string(b->size));
  if (scount == 0 || scount > 64 || table_off + (uint64_t)scount * SECT_ENTRY > b->size - 32)
    return fail(b, "section table out of range");
  std::vector<uint8_t> st((size_t)scount * SECT_ENTRY);
  if (!read_at(b->f, table_off, st.data(), st.size())) return fail(b, "truncated section table");
  uint64_t soff[6] = {}, sbytes[6] = {};
  uint32_t scrc[6] = {};
  bool have[6] = {};
  for (uint32_t i = 0; i < scount; ++i) {
    const uint8_t *e = st.data() + i * SECT_ENTRY;
    const uint32_t id = rd<uint32_t>(e);
    if (id < 1 || id > 5) continue;  // unknown sections are not v1's to check
    have[id] = true;
    soff[id] = rd<uint64_t>(e + 4);
    sbytes[id] = rd<uint64_t>(e + 12);
    scrc[id] = rd<uint32_t>(e + 20);
  }
  for (int id = 1; id <= 5; ++id) {
    if (!have[id]) return fail(b, "missing section " + std::to_string(id));
    if (soff[id] > b->size - 32 || sbytes[id] > b->size - 32 - soff[id])
      return fail(b, "section " + std::to_string(id) + " out of range");
  }
  // sections 1-4: u64 length + body, CRC over both; 5: raw directory entries
  for (int id = 1; id <= 4; ++id) {
    uint8_t lb[8];
    if (sbytes[id] < 8 || !read_at(b->f, soff[id], lb, 8))
      return fail(b, "section " + std::to_string(id) + " truncated");
    const uint64_t ln = rd<uint64_t>(lb);
    if (ln + 8 > sbytes[id] || ln > (1ull << 26))
      return fail(b, "section " + std::to_string(id) + " length implausible");
    std::vector<uint8_t> body(ln);
    if (ln && !read_at(b->f, soff[id] + 8, body.data(), ln))
      return fail(b, "section " + std::to_string(id) + " truncated");
    uint32_t c = crc32_update(0, lb, 8);
    c = crc32_update(c, body.data(), ln);
    if (c != scrc[id]) return fail(b, "section " + std::to_string(id) + " CRC mismatch");
    if (id == 2) b->arch.assign(body.begin(), body.end());
  }
  // n is checked against the section size before it is multiplied, so a crafted count
  // cannot wrap n * 192 onto the section's byte count.
  if (n > sbytes[5] / DIR_ENTRY || sbytes[5] != n * DIR_ENTRY)
    return fail(b, "dir size mismatch: tensor_count " + std::to_string(n) + " x 192 != " +
                       std::to_string(sbytes[5]));
  std::vector<uint8_t> dir(sbytes[5]);
  if (!dir.empty() && !read_at(b->f, soff[5], dir.data(), dir.size()))
    return fail(b, "truncated dir");
  if (crc32_update(0, dir.data(), dir.size()) != scrc[5]) return fail(b, "section 5 (dir) CRC mismatch");
  b->entries.resize(n);
  for (uint64_t i = 0; i < n; ++i) {
    const uint8_t *e = dir.data() + i * DIR_ENTRY;
    Entry &t = b->entries[i];
    const void *nul = memchr(e, 0, 64);
    if (!nul) return fail(b, "entry " + std::to_string(i) + ": name not NUL-terminated");
    t.name.assign((const char *)e, (const char *)nul);
    t.ndim = e[64];
    if (t.ndim > 8) return fail(b, t.name + ": ndim " + std::to_string(t.ndim) + " > 8");
    for (int d = 0; d < 8; ++d) t.shape[d] = rd<uint64_t>(e + 72 + 8 * d);
    t.logical = e[136];
    t.storage = e[137];
    t.layout = rd<uint16_t>(e + 138);
    t.group = rd<uint32_t>(e + 140);
    t.sc_off = rd<uint64_t>(e + 144);
    t.sc_bytes = rd<uint64_t>(e + 152);
    t.d_off = rd<uint64_t>(e + 160);
    t.d_bytes = rd<uint64_t>(e + 168);
    t.crc = rd<uint32_t>(e + 176);
    t.scale_dtype = e[180];
  }
  // names, namespaces, dtypes, layouts, sizes
  std::vector<std::string> names;
  for (const Entry &t : b->entries) names.push_back(t.name);
  std::sort(names.begin(), names.end());
  for (size_t i = 1; i < names.size(); ++i)
    if (names[i] == names[i - 1]) return fail(b, "duplicate name " + names[i]);
  struct Span { uint64_t a, z; std::string what; };
  std::vector<Span> spans;
  for (const Entry &t : b->entries) {
    if (is_visual(t.name)) return fail(b, "visual tensor present: " + t.name);
    if (t.logical > DT_FP8 || t.storage > DT_FP8)
      return fail(b, t.name + ": unsupported dtype enum " + std::to_string(t.storage));
    for (int d = 0; d < t.ndim; ++d)
      if (t.shape[d] == 0 || t.shape[d] > (1ull << 40))
        return fail(b, t.name + ": implausible shape");
    if (t.numel() > (1ull << 48)) return fail(b, t.name + ": implausible shape");
    if (t.layout == LAYOUT_EXPERT_STACKED) {
      if (t.storage != DT_INT4 || t.ndim != 3)
        return fail(b, t.name + ": layout_id 32 needs a 3-D INT4 tensor");
    } else if (t.layout != LAYOUT_ROW_MAJOR) {
      return fail(b, t.name + ": unknown layout_id " + std::to_string(t.layout));
    }
    const uint64_t ne = t.numel();
    if (t.storage == DT_INT4) {
      const uint64_t ng = (ne + GROUP - 1) / GROUP;
      if (t.group != GROUP || t.sc_bytes != ng * 2)
        return fail(b, "bad quant params " + t.name + ": group " + std::to_string(t.group) +
                           ", scale bytes " + std::to_string(t.sc_bytes) + " (expected " +
                           std::to_string(ng * 2) + ")");
      if (t.d_bytes != ng * GROUP / 2)
        return fail(b, "bad packed size " + t.name + ": " + std::to_string(t.d_bytes) +
                           " (expected " + std::to_string(ng * GROUP / 2) + ")");
      if (t.scale_dtype > 1) return fail(b, t.name + ": unknown scale dtype " + std::to_string(t.scale_dtype));
    } else {
      // scale_offset is not looked at when there are no scale bytes: the reference's own
      // valid test file (tools/binfer.py:541-544) leaves the scale-pool cursor there
      if (t.sc_bytes || t.group)
        return fail(b, t.name + ": quant fields set on an unquantized tensor");
      if (t.d_bytes != ne * dtype_bytes(t.storage))
        return fail(b, "bad payload size " + t.name + ": " + std::to_string(t.d_bytes) +
                           " (expected " + std::to_string(ne * dtype_bytes(t.storage)) + ")");
    }
    if (t.d_off % ALIGN) return fail(b, t.name + ": payload not 64-byte aligned");
    spans.push_back({t.d_off, t.d_off + t.d_bytes, t.name});
    if (t.sc_bytes) spans.push_back({t.sc_off, t.sc_off + t.sc_bytes, t.name + "#scales"});
  }
  for (const Span &s : spans)
    if (s.z < s.a || s.z > b->size - 32) return fail(b, "span out of range: " + s.what);
  std::sort(spans.begin(), spans.end(), [](const Span &x, const Span &y) { return x.a < y.a; });
  for (size_t i = 1; i < spans.size(); ++i)
    if (spans[i].a < spans[i - 1].z)
      return fail(b, "overlap " + spans[i - 1].what + " vs " + spans[i].what);
  // payload CRCs, then the trailing SHA-256 of everything before it
  std::vector<uint8_t> chunk(1 << 20);
  for (const Entry &t : b->entries) {
    uint32_t c = 0;
    for (uint64_t o = 0; o < t.d_bytes; o += chunk.size()) {
      const size_t m = (size_t)std::min<uint64_t>(chunk.size(), t.d_bytes - o);
      if (!read_at(b->f, t.d_off + o, chunk.data(), m)) return fail(b, "truncated payload " + t.name);
      c = crc32_update(c, chunk.data(), m);
    }
    if (c != t.crc) return fail(b, "payload CRC " + t.name);
  }
  Sha256 sha;
  if (fseeko(b->f, 0, SEEK_SET) != 0) return fail(b, "seek failed");
  for (uint64_t left = b->size - 32; left > 0;) {
    const size_t m = (size_t)std::min<uint64_t>(chunk.size(), left);
    if (fread(chunk.data(), 1, m, b->f) != m) return fail(b, "truncated");
    sha.update(chunk.data(), m);
    left -= m;
  }
  uint8_t want[32], got[32];
  sha.finish(got);
  if (fread(want, 1, 32, b->f) != 32 || memcmp(want, got, 32) != 0)
    return fail(b, "trailing sha256 mismatch");
  return AINFER_OK;
}

// integer value of "key": in the architecture section's compact JSON
bool arch_int(const std::string &js, const char *key, long long *v) {
  const std::string k = std::string("\"") + key + "\":";
  const size_t p = js.find(k);
  if (p == std::string::npos) return false;
  char *end = nullptr;
  *v = strtoll(js.c_str() + p + k.size(), &end, 10);
  return end != js.c_str() + p + k.size();
}
bool arch_num(const std::string &js, const char *key, double *v) {
  const std::string k = std::string("\"") + key + "\":";
  const size_t p = js.find(k);
  if (p == std::string::npos) return false;
  char *end = nullptr;
  *v = strtod(js.c_str() + p + k.size(), &end);
  return end != js.c_str() + p + k.size();
}

const Entry *find(const ainfer_binfer *b, const std::string &name) {
  for (const Entry &t : b->entries)
    if (t.name == name) return &t;
  return nullptr;
}

std::string lname(int layer, const char *suffix) {
  return "model.layers." + std::to_string(layer) + "." + suffix;
}

size_t al256(size_t v) { return (v + 255) & ~(size_t)255; }

// One layer's tensors in the order they go into the device arena.
struct Part {
  const char *suffix;
  bool scales;  // the INT4 tensor's scales (else its payload)
  bool optional;
};
constexpr Part PARTS[] = {
    {"mlp.gate.weight", false, false},
    {"mlp.gate.bias", false, true},
    {"mlp.shared_expert_gate.weight", false, true},
    {"mlp.experts.gate_proj.weight", false, false},
    {"mlp.experts.gate_proj.weight", true, false},
    {"mlp.experts.up_proj.weight", false, false},
    {"mlp.experts.up_proj.weight", true, false},
    {"mlp.experts.down_proj.weight", false, false},
    {"mlp.experts.down_proj.weight", true, false},
    {"mlp.shared_expert.gate_proj.weight", false, true},
    {"mlp.shared_expert.gate_proj.weight", true, true},
    {"mlp.shared_expert.up_proj.weight", false, true},
    {"mlp.shared_expert.up_proj.weight", true, true},
    {"mlp.shared_expert.down_proj.weight", false, true},
    {"mlp.shared_expert.down_proj.weight", true, true},
    {"post_attention_layernorm.weight", false, true},
};
constexpr int NPARTS = sizeof(PARTS) / sizeof(PARTS[0]);

// Check the layer's tensors against the file's MoE shape.
int check_layer(const ainfer_binfer *b, int layer, const ainfer_moe_shape &s) {
  auto bad = [&](const std::string &m) {
    const_cast<ainfer_binfer *>(b)->err = m;
    return AINFER_ERR_FORMAT;
  };
  const uint64_t H = s.hidden, E = s.n_experts, I = s.inter, Is = s.shared_inter;
  struct Want {
    const char *suffix;
    int storage, layout, ndim;
    uint64_t d0, d1, d2;
    bool optional;
  };
  const Want want[] = {
      {"mlp.gate.weight", DT_BF16, 0, 2, E, H, 0, false},
      {"mlp.gate.bias", DT_FP32, 0, 1, E, 0, 0, true},
      {"mlp.shared_expert_gate.weight", DT_BF16, 0, 2, 1, H, 0, true},
      {"mlp.experts.gate_proj.weight", DT_INT4, LAYOUT_EXPERT_STACKED, 3, E, I, H, false},
      {"mlp.experts.up_proj.weight", DT_INT4, LAYOUT_EXPERT_STACKED, 3, E, I, H, false},
      {"mlp.experts.down_proj.weight", DT_INT4, LAYOUT_EXPERT_STACKED, 3, E, H, I, false},
      {"mlp.shared_expert.gate_proj.weight", DT_INT4, 0, 2, Is, H, 0, Is == 0},
      {"mlp.shared_expert.up_proj.weight", DT_INT4, 0, 2, Is, H, 0, Is == 0},
      {"mlp.shared_expert.down_proj.weight", DT_INT4, 0, 2, H, Is, 0, Is == 0},
      {"post_attention_layernorm.weight", DT_BF16, 0, 1, H, 0, 0, true},
  };
  for (const Want &w : want) {
    const std::string nm = lname(layer, w.suffix);
    const Entry *t = find(b, nm);
    if (!t) {
      if (w.optional) continue;
      return bad("missing tensor " + nm);
    }
    const uint64_t dims[3] = {w.d0, w.d1, w.d2};
    bool ok = t->storage == w.storage && t->layout == w.layout && t->ndim == w.ndim;
    for (int d = 0; ok && d < w.ndim; ++d) ok = t->shape[d] == dims[d];
    if (!ok) return bad(nm + ": dtype/layout/shape do not match the MoE shape");
    if (w.storage == DT_INT4 && t->scale_dtype != (s.scale_dtype == AINFER_SCALE_FP16 ? 1 : 0))
      return bad(nm + ": scale dtype differs from the layer's");
  }
  return AINFER_OK;
}

}  // namespace

extern "C" {

int ainfer_binfer_open(const char *path, ainfer_binfer **out, char *err, size_t err_len) {
  if (!path || !out) return AINFER_ERR_NULL;
  *out = nullptr;
  ainfer_binfer *b = new ainfer_binfer();
  b->f = fopen(path, "rb");
  int rc = AINFER_OK;
  if (!b->f) {
    b->err = std::string("cannot open ") + path;
    rc = AINFER_ERR_IO;
  } else {
    fseeko(b->f, 0, SEEK_END);
    b->size = (uint64_t)ftello(b->f);
    // The validator reports a bad file through its return code; an exception from it
    // (an allocation a damaged file would size) must not cross the C ABI.
    try {
      rc = validate(b);
    } catch (...) {
      rc = fail(b, "file rejected: a directory or section size the validator cannot hold");
    }
  }
  if (rc != AINFER_OK) {
    if (err && err_len) snprintf(err, err_len, "%s", b->err.c_str());
    if (b->f) fclose(b->f);
    delete b;
    return rc;
  }
  if (err && err_len) err[0] = 0;
  *out = b;
  return AINFER_OK;
}

void ainfer_binfer_close(ainfer_binfer *b) {
  if (!b) return;
  if (b->f) fclose(b->f);
  delete b;
}

int ainfer_binfer_moe_info(const ainfer_binfer *b, ainfer_moe_shape *s, int32_t *n_layers,
                           float *eps) {
  if (!b || !s) return AINFER_ERR_NULL;
  long long H, E, k, I, Is, L, sd;
  if (!arch_int(b->arch, "hidden", &H) || !arch_int(b->arch, "n_experts", &E) ||
      !arch_int(b->arch, "top_k", &k) || !arch_int(b->arch, "inter", &I) ||
      !arch_int(b->arch, "shared_inter", &Is) || !arch_int(b->arch, "layers", &L) ||
      !arch_int(b->arch, "scale_fp16", &sd))
    return AINFER_ERR_FORMAT;
  memset(s, 0, sizeof *s);
  s->hidden = (int32_t)H;
  s->n_experts = (int32_t)E;
  s->top_k = (int32_t)k;
  s->inter = (int32_t)I;
  s->shared_inter = (int32_t)Is;
  s->group = GROUP;
  s->scale_dtype = sd ? AINFER_SCALE_FP16 : AINFER_SCALE_BF16;
  if (ainfer_moe_validate(s) != AINFER_OK) return AINFER_ERR_SHAPE;
  if (n_layers) *n_layers = (int32_t)L;
  double e = 1e-6;
  arch_num(b->arch, "rms_eps", &e);
  if (eps) *eps = (float)e;
  return AINFER_OK;
}

size_t ainfer_binfer_moe_layer_bytes(const ainfer_binfer *b, int32_t layer) {
  if (!b) return 0;
  size_t total = 0;
  for (int i = 0; i < NPARTS; ++i) {
    const Entry *t = find(b, lname(layer, PARTS[i].suffix));
    if (!t) continue;
    total += al256(PARTS[i].scales ? t->sc_bytes : t->d_bytes);
  }
  return total;
}

const char *ainfer_binfer_error(const ainfer_binfer *b) { return b ? b->err.c_str() : ""; }

int ainfer_binfer_load_moe_layer(const ainfer_binfer *b, int32_t layer, void *arena,
                                 size_t arena_bytes, ainfer_moe_weights *w, const void **norm_w,
                                 void *stream) {
  if (!b || !arena || !w) return AINFER_ERR_NULL;
  ainfer_moe_shape s;
  int32_t L = 0;
  int rc = ainfer_binfer_moe_info(b, &s, &L, nullptr);
  if (rc) return rc;
  if (layer < 0 || layer >= L) return AINFER_ERR_ARG;
  if ((rc = check_layer(b, layer, s))) return rc;
  if (((uintptr_t)arena & 255) || arena_bytes < ainfer_binfer_moe_layer_bytes(b, layer))
    return AINFER_ERR_WORKSPACE;
  memset(w, 0, sizeof *w);
  if (norm_w) *norm_w = nullptr;
  const void **dst[NPARTS] = {
      (const void **)&w->router_w, (const void **)&w->router_bias,
      (const void **)&w->shared_gate_w, (const void **)&w->w_gate, &w->s_gate,
      (const void **)&w->w_up, &w->s_up, (const void **)&w->w_down, &w->s_down,
      (const void **)&w->ws_gate, &w->ss_gate, (const void **)&w->ws_up, &w->ss_up,
      (const void **)&w->ws_down, &w->ss_down, norm_w};
  hipStream_t st = (hipStream_t)stream;
  std::vector<uint8_t> host;
  size_t off = 0;
  for (int i = 0; i < NPARTS; ++i) {
    const Entry *t = find(b, lname(layer, PARTS[i].suffix));
    if (!t) continue;
    const uint64_t src = PARTS[i].scales ? t->sc_off : t->d_off;
    const uint64_t n = PARTS[i].scales ? t->sc_bytes : t->d_bytes;
    host.resize(n);
    if (n && !read_at(b->f, src, host.data(), n)) return AINFER_ERR_IO;
    uint8_t *d = (uint8_t *)arena + off;
    if (n && hipMemcpyAsync(d, host.data(), n, hipMemcpyHostToDevice, st) != hipSuccess)
      return AINFER_ERR_HIP;
    if (hipStreamSynchronize(st) != hipSuccess) return AINFER_ERR_HIP;  // host is reused
    if (dst[i]) *dst[i] = d;
    off += al256(n);
  }
  if (!s.shared_inter) {
    w->ws_gate = w->ws_up = w->ws_down = nullptr;
    w->ss_gate = w->ss_up = w->ss_down = nullptr;
  }
  return AINFER_OK;
}

}  // extern "C"
