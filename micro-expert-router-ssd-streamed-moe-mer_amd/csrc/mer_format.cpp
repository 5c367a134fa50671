// mer_format.cpp -- on-disk expert formats (host only): the UTH expert-blob
// headers and the GGUF reader that cuts per-expert blobs out of a model's
// MoE tensors, so real checkpoints feed the device path unchanged.
//
// UTH (reference tensor_header.rs):
//   UTH1: 64-byte header "UTH1", u16 version (1), u8 dtype id, u8 rank
//         (1..4), u32 shape[4], u32 quant_scale_offset, u32
//         quant_scale_count, u32 tile hints m/n/k, u32 flags (bit 0: the
//         payload starts at the next multiple of the block alignment),
//         16 reserved bytes (tensor_header.rs:11-27, :476-536).
//   UTH2: 128-byte mixed-projection header "UTH2", u16 version (2), u16
//         projection count (3), u32 d_model, u32 d_ff, u32 flags, then at
//         24 + 24 i for gate/up/down: u8 dtype, u8 role (= i), u64 offset,
//         u64 len, u32 weights; ranges are payload-relative, non-empty,
//         inside the payload and non-overlapping (tensor_header.rs:189-391).
//   A blob is stripped as ExpertResident::new_with_block_align does
//   (expert_cache.rs:110-143): UTH2 first, then UTH1, else it is a
//   headerless (legacy) blob used as is.
//
// GGUF (reference gguf.rs:207-295, gguf_loader.rs:136-200, :2255-2330,
// :2940-3010): magic "GGUF", u32 version 1..3, tensor and KV counts (u32 in
// v1, u64 after), KV pairs, tensor infos (name, n_dims, dims (u32 in v1),
// ggml type, data offset); tensor data starts at the next multiple of
// general.alignment (default 32).  A layer's experts are either stacked --
// blk.L.ffn_{gate,up}_exps.weight with GGML dims [d_model, d_ff, E] and
// blk.L.ffn_down_exps.weight [d_ff, d_model, E] -- or per expert --
// blk.L.ffn_{gate,up,down}.e.weight.  For Q4_0 / Q8_0 with d_model * d_ff a
// multiple of 32, expert e's quantised bytes are the contiguous run at
// e * projection_bytes of each stacked tensor, copied byte for byte into
// MER's gate || up || down blob.
#include <errno.h>
#include <fcntl.h>
#include <stdio.h>
#include <string.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <map>
#include <string>
#include <vector>

#include "../../include/mer_hip.h"
#include "mer_internal.hpp"

using namespace mer;

namespace {

uint16_t rd16(const uint8_t *p) { return (uint16_t)(p[0] | (p[1] << 8)); }
uint32_t rd32(const uint8_t *p) { return (uint32_t)p[0] | ((uint32_t)p[1] << 8) | ((uint32_t)p[2] << 16) | ((uint32_t)p[3] << 24); }
uint64_t rd64(const uint8_t *p) { return (uint64_t)rd32(p) | ((uint64_t)rd32(p + 4) << 32); }
void wr16(uint8_t *p, uint16_t v) { p[0] = (uint8_t)v; p[1] = (uint8_t)(v >> 8); }
void wr32(uint8_t *p, uint32_t v) { for (int i = 0; i < 4; ++i) p[i] = (uint8_t)(v >> (8 * i)); }

constexpr size_t kUth1Bytes = 64;
constexpr size_t kUth2Bytes = 128;
constexpr uint32_t kUthPageAligned = 1u;
constexpr int kUthMaxDtype = 10;  // UthDtypeId::Mixed

size_t padded_prefix(size_t header, uint32_t flags, size_t block_align) {
  if ((flags & kUthPageAligned) && block_align > 0) return header + (block_align - header % block_align) % block_align;
  return header;
}

// MixedExpertHeader::probe + strip + validate
bool probe_uth2(const uint8_t *b, size_t len, size_t block_align, mer_uth_info *o) {
  if (len < kUth2Bytes || memcmp(b, "UTH2", 4) != 0) return false;
  if (rd16(b + 4) != 2 || rd16(b + 6) != 3) return false;
  mer_uth_info h{};
  h.kind = 2;
  h.version = 2;
  h.dtype = kUthMaxDtype;
  h.d_model = rd32(b + 8);
  h.d_ff = rd32(b + 12);
  h.flags = rd32(b + 16);
  for (int i = 0; i < 3; ++i) {
    const uint8_t *q = b + 24 + 24 * i;
    if (q[1] != (uint8_t)i || q[0] > kUthMaxDtype) return false;
    h.proj[i].dtype = q[0];
    h.proj[i].offset = rd64(q + 4);
    h.proj[i].len = rd64(q + 12);
    h.proj[i].weights = rd32(q + 20);
  }
  const size_t prefix = padded_prefix(kUth2Bytes, h.flags, block_align);
  if (prefix > len) return false;
  const uint64_t payload = len - prefix;
  // validate (tensor_header.rs:197-240)
  if (h.d_model == 0 || h.d_ff == 0) return false;
  uint64_t start[3], end[3];
  for (int i = 0; i < 3; ++i) {
    const mer_uth_projection &r = h.proj[i];
    if (r.dtype == kUthMaxDtype || r.len == 0 || r.offset > UINT64_MAX - r.len) return false;
    start[i] = r.offset;
    end[i] = r.offset + r.len;
    if (end[i] > payload) return false;
  }
  for (int i = 0; i < 3; ++i)
    for (int j = 0; j < 3; ++j)
      if (i != j && start[i] <= start[j] && end[i] > start[j]) return false;  // overlap
  h.payload_offset = prefix;
  h.payload_len = payload;
  *o = h;
  return true;
}

// TensorHeader::probe + strip
bool probe_uth1(const uint8_t *b, size_t len, size_t block_align, mer_uth_info *o) {
  if (len < kUth1Bytes || memcmp(b, "UTH1", 4) != 0) return false;
  const uint16_t version = rd16(b + 4);
  if (version == 0 || version > 1) return false;
  if (b[6] > kUthMaxDtype) return false;
  const uint8_t rank = b[7];
  if (rank == 0 || rank > 4) return false;
  mer_uth_info h{};
  h.kind = 1;
  h.version = version;
  h.dtype = b[6];
  h.shape_rank = rank;
  for (int i = 0; i < 4; ++i) h.shape[i] = rd32(b + 8 + 4 * i);
  h.quant_scale_offset = rd32(b + 24);
  h.quant_scale_count = rd32(b + 28);
  h.flags = rd32(b + 44);
  const size_t prefix = padded_prefix(kUth1Bytes, h.flags, block_align);
  if (prefix > len) return false;  // treated as a legacy blob
  // A SwiGLU expert header records [d_ff, d_model, 3] (for_swiglu_expert).
  if (rank == 3 && h.shape[2] == 3) {
    h.d_ff = h.shape[0];
    h.d_model = h.shape[1];
  }
  h.payload_offset = prefix;
  h.payload_len = len - prefix;
  *o = h;
  return true;
}

// ---- GGUF -----------------------------------------------------------------

constexpr uint32_t kGgmlQ4_0 = 2, kGgmlQ8_0 = 8;

struct TensorInfo {
  std::vector<uint64_t> dims;
  uint32_t type = 0;
  uint64_t offset = 0;  // from the start of the tensor data section
};

}  // namespace

struct mer_gguf {
  int fd = -1;
  uint64_t file_len = 0;
  uint32_t version = 0;
  uint64_t data_start = 0;
  std::map<std::string, uint64_t> ints;  // integer metadata
  std::string arch;
  std::map<std::string, TensorInfo> tensors;
};

namespace {

struct Reader {
  const uint8_t *p;
  size_t n, pos = 0;
  bool ok = true;
  const uint8_t *take(size_t k) {
    if (!ok || k > n - pos) {
      ok = false;
      return nullptr;
    }
    const uint8_t *r = p + pos;
    pos += k;
    return r;
  }
  uint32_t u32() { const uint8_t *b = take(4); return b ? rd32(b) : 0; }
  uint64_t u64() { const uint8_t *b = take(8); return b ? rd64(b) : 0; }
  uint64_t count(uint32_t version) { return version == 1 ? u32() : u64(); }
  std::string str(uint32_t version) {
    const uint64_t len = count(version);
    if (len > (1u << 20)) { ok = false; return {}; }
    const uint8_t *b = take((size_t)len);
    return b ? std::string((const char *)b, (size_t)len) : std::string();
  }
};

// Value of GGUF metadata type `ty`; integers are returned through *iv.
bool read_value(Reader &r, uint32_t version, uint32_t ty, bool *is_int, uint64_t *iv, std::string *sv, int depth = 0) {
  *is_int = false;
  static const int kSize[] = {1, 1, 2, 2, 4, 4, 4, 1, 0, 0, 8, 8, 8};
  if (ty == 8) {  // string
    *sv = r.str(version);
    return r.ok;
  }
  if (ty == 9) {  // array: element type, count, elements
    if (depth > 2) return false;
    const uint32_t et = r.u32();
    const uint64_t cnt = r.count(version);
    for (uint64_t i = 0; i < cnt && r.ok; ++i) {
      bool ii;
      uint64_t x;
      std::string s;
      if (!read_value(r, version, et, &ii, &x, &s, depth + 1)) return false;
    }
    return r.ok;
  }
  if (ty > 12) return false;
  const uint8_t *b = r.take((size_t)kSize[ty]);
  if (!b) return false;
  if (ty == 6 || ty == 12) return true;  // float32 / float64: not consulted
  uint64_t v = 0;
  for (int i = 0; i < kSize[ty]; ++i) v |= (uint64_t)b[i] << (8 * i);
  *is_int = true;
  *iv = v;
  return true;
}

int parse_gguf(mer_gguf *g) {
  // read the header region in growing chunks until it parses
  std::vector<uint8_t> buf;
  size_t want = 1u << 20;
  for (;;) {
    const size_t n = (size_t)std::min<uint64_t>(want, g->file_len);
    buf.resize(n);
    if (pread(g->fd, buf.data(), n, 0) != (ssize_t)n) return report_error(MER_ERR_IO, "GGUF header read failed");
    Reader r{buf.data(), n};
    const uint8_t *magic = r.take(4);
    if (!magic || memcmp(magic, "GGUF", 4) != 0) return report_error(MER_ERR_INVALID_LAYOUT, "not a GGUF file (bad magic)");
    g->version = r.u32();
    if (g->version == 0 || g->version > 3) return report_error(MER_ERR_INVALID_LAYOUT, "unsupported GGUF version");
    const uint64_t n_tensors = r.count(g->version), n_kv = r.count(g->version);
    g->ints.clear();
    g->tensors.clear();
    uint64_t alignment = 32;
    for (uint64_t i = 0; i < n_kv && r.ok; ++i) {
      const std::string key = r.str(g->version);
      const uint32_t ty = r.u32();
      bool is_int;
      uint64_t iv = 0;
      std::string sv;
      if (!r.ok || !read_value(r, g->version, ty, &is_int, &iv, &sv)) {
        r.ok = false;
        break;
      }
      if (is_int) g->ints[key] = iv;
      if (key == "general.architecture") g->arch = sv;
      if (key == "general.alignment" && is_int) alignment = iv ? iv : 1;
    }
    for (uint64_t i = 0; i < n_tensors && r.ok; ++i) {
      const std::string name = r.str(g->version);
      const uint32_t nd = r.u32();
      if (nd > 8) {
        r.ok = false;
        break;
      }
      TensorInfo t;
      for (uint32_t d = 0; d < nd; ++d) t.dims.push_back(g->version == 1 ? r.u32() : r.u64());
      t.type = r.u32();
      t.offset = r.u64();
      if (r.ok) g->tensors[name] = t;
    }
    if (r.ok) {
      g->data_start = (r.pos + alignment - 1) / alignment * alignment;
      if (g->data_start > g->file_len) return report_error(MER_ERR_INVALID_LAYOUT, "GGUF tensor data starts past the end");
      return MER_OK;
    }
    if (n >= g->file_len || want > (1ull << 32))
      return report_error(MER_ERR_INVALID_LAYOUT, "truncated or malformed GGUF header");
    want *= 4;
  }
}

// metadata_lookup (gguf_loader.rs:136-150): "llama.<suffix>", then
// "<arch>.<suffix>", then the smallest key ending in ".<suffix>".
bool meta_int(const mer_gguf *g, const char *suffix, uint64_t *out) {
  const std::string s = suffix, dotted = "." + s;
  auto it = g->ints.find("llama." + s);
  if (it == g->ints.end() && !g->arch.empty()) it = g->ints.find(g->arch + "." + s);
  if (it == g->ints.end()) {
    for (auto j = g->ints.begin(); j != g->ints.end(); ++j)
      if (j->first.size() >= dotted.size() && j->first.compare(j->first.size() - dotted.size(), dotted.size(), dotted) == 0) {
        it = j;
        break;  // std::map iterates keys in order: the first match is the smallest
      }
  }
  if (it == g->ints.end()) return false;
  *out = it->second;
  return true;
}

int dtype_of(uint32_t ggml) {
  if (ggml == kGgmlQ4_0) return MER_DTYPE_Q4_0;
  if (ggml == kGgmlQ8_0) return MER_DTYPE_Q8_0;
  return -1;
}

struct LayerGeom {
  mer_gguf_moe_info info;
  const TensorInfo *t[3];  // stacked gate, up, down (layout 0)
};

int layer_geometry(mer_gguf *g, size_t layer, LayerGeom *lg) {
  LayerGeom r{};
  const std::string p = "blk." + std::to_string(layer) + ".";
  static const char *kProj[3] = {"gate", "up", "down"};
  auto find = [&](const std::string &name) -> const TensorInfo * {
    auto it = g->tensors.find(name);
    return it == g->tensors.end() ? nullptr : &it->second;
  };
  uint64_t dm = 0, dff = 0, ne = 0;
  const TensorInfo *g0 = find(p + "ffn_gate_exps.weight");
  if (g0) {
    r.info.layout = 0;
    for (int i = 0; i < 3; ++i) {
      r.t[i] = find(p + "ffn_" + kProj[i] + "_exps.weight");
      if (!r.t[i] || r.t[i]->dims.size() != 3)
        return report_error(MER_ERR_INVALID_LAYOUT, "stacked expert tensors must be 3-D gate, up and down");
    }
    // GGML dims, innermost first: gate/up [d_model, d_ff, E], down [d_ff, d_model, E]
    dm = r.t[0]->dims[0];
    dff = r.t[0]->dims[1];
    ne = r.t[0]->dims[2];
    if (r.t[1]->dims != r.t[0]->dims || r.t[2]->dims[0] != dff || r.t[2]->dims[1] != dm || r.t[2]->dims[2] != ne)
      return report_error(MER_ERR_INVALID_LAYOUT, "gate, up and down expert tensor shapes disagree");
    if (r.t[1]->type != r.t[0]->type || r.t[2]->type != r.t[0]->type)
      return report_error(MER_ERR_UNSUPPORTED_DTYPE, "gate, up and down expert tensors differ in dtype (mixed layouts are not on this path)");
  } else {
    const TensorInfo *g1 = find(p + "ffn_gate.0.weight");
    if (!g1) return report_error(MER_ERR_INVALID_LAYOUT, "layer has no expert weight tensors");
    r.info.layout = 1;
    if (g1->dims.size() != 2) return report_error(MER_ERR_INVALID_LAYOUT, "per-expert tensors must be 2-D");
    dm = g1->dims[0];
    dff = g1->dims[1];
    while (find(p + "ffn_gate." + std::to_string(ne) + ".weight")) ++ne;
  }
  // metadata geometry, when present, must agree (gguf_loader.rs:152-200)
  uint64_t v;
  if (meta_int(g, "embedding_length", &v) && v != dm)
    return report_error(MER_ERR_INVALID_LAYOUT, "embedding_length disagrees with the expert tensor shapes");
  if ((meta_int(g, "expert_feed_forward_length", &v) || meta_int(g, "feed_forward_length", &v)) && v != dff)
    return report_error(MER_ERR_INVALID_LAYOUT, "feed_forward_length disagrees with the expert tensor shapes");
  if (meta_int(g, "expert_count", &v) && v != ne)
    return report_error(MER_ERR_INVALID_LAYOUT, "expert_count disagrees with the expert tensor shapes");
  if (dm == 0 || dff == 0 || ne == 0) return report_error(MER_ERR_INVALID_LAYOUT, "empty expert geometry");
  const uint32_t type = r.info.layout == 0 ? r.t[0]->type : find(p + "ffn_gate.0.weight")->type;
  const int dtype = dtype_of(type);
  if (dtype < 0) return report_error(MER_ERR_UNSUPPORTED_DTYPE, "expert tensors are not Q4_0 or Q8_0");
  if ((dm * dff) % 32 != 0)
    return report_error(MER_ERR_INVALID_LAYOUT, "expert slices are not block-aligned (d_model * d_ff % 32 != 0)");
  r.info.dtype = dtype;
  r.info.d_model = dm;
  r.info.d_ff = dff;
  r.info.n_experts = ne;
  r.info.expert_bytes = mer_expert_weight_bytes(dtype, dm, dff);
  *lg = r;
  return MER_OK;
}

int read_range(const mer_gguf *g, uint64_t off, uint64_t len, uint8_t *dst) {
  if (off > g->file_len || len > g->file_len - off) return report_error(MER_ERR_INVALID_LAYOUT, "tensor data past the end of the GGUF file");
  while (len > 0) {
    const size_t chunk = (size_t)std::min<uint64_t>(len, 1u << 30);
    const ssize_t n = pread(g->fd, dst, chunk, (off_t)off);
    if (n <= 0) return report_error(MER_ERR_IO, "GGUF tensor data read failed");
    dst += n;
    off += (uint64_t)n;
    len -= (uint64_t)n;
  }
  return MER_OK;
}

}  // namespace

extern "C" {

int mer_uth_probe(const void *bytes, size_t len, size_t block_align, mer_uth_info *out) {
  if (!out || (!bytes && len)) return report_error(MER_ERR_INVALID_LAYOUT, "null argument");
  const uint8_t *b = (const uint8_t *)bytes;
  mer_uth_info h{};
  if (probe_uth2(b, len, block_align, &h) || probe_uth1(b, len, block_align, &h)) {
    *out = h;
    return MER_OK;
  }
  *out = mer_uth_info{};
  out->dtype = -1;
  out->payload_len = len;  // headerless: the whole blob is the payload
  return MER_OK;
}

int mer_uth_write_expert_header(int dtype, size_t d_model, size_t d_ff, size_t block_align, void *dst, size_t dst_len,
                                size_t *written) {
  // TensorHeader::for_swiglu_expert + write_padded (tensor_header.rs:398-470)
  if (dtype < 0 || dtype > kUthMaxDtype) return report_error(MER_ERR_UNSUPPORTED_DTYPE, "unknown UTH dtype id");
  if (d_model > UINT32_MAX || d_ff > UINT32_MAX) return report_error(MER_ERR_SHAPE_EXCEEDS_WORKSPACE, "dimension exceeds u32");
  const size_t total = padded_prefix(kUth1Bytes, kUthPageAligned, block_align);
  if (written) *written = total;
  if (!dst) return MER_OK;  // size query
  if (dst_len < total) return report_error(MER_ERR_BUFFER_TOO_SMALL, "header buffer too small");
  uint8_t *b = (uint8_t *)dst;
  memset(b, 0, total);
  memcpy(b, "UTH1", 4);
  wr16(b + 4, 1);
  b[6] = (uint8_t)dtype;
  b[7] = 3;
  wr32(b + 8, (uint32_t)d_ff);
  wr32(b + 12, (uint32_t)d_model);
  wr32(b + 16, 3);
  wr32(b + 28, dtype == 2 /* Int8: three f32 per-tensor scales at payload offset 0 */ ? 3u : 0u);
  wr32(b + 32, 16);
  wr32(b + 36, 16);
  wr32(b + 40, 64);
  wr32(b + 44, kUthPageAligned);
  return MER_OK;
}

int mer_gguf_open(const char *path, mer_gguf **out) {
  if (!path || !out) return report_error(MER_ERR_INVALID_LAYOUT, "null argument");
  *out = nullptr;
  const int fd = open(path, O_RDONLY | O_CLOEXEC);
  if (fd < 0) {
    char msg[512];
    snprintf(msg, sizeof msg, "cannot open %s: %s", path, strerror(errno));
    return report_error(MER_ERR_IO, msg);
  }
  struct stat st;
  if (fstat(fd, &st) != 0) {
    close(fd);
    return report_error(MER_ERR_IO, "cannot stat the GGUF file");
  }
  mer_gguf *g = new mer_gguf;
  g->fd = fd;
  g->file_len = (uint64_t)st.st_size;
  const int rc = parse_gguf(g);
  if (rc) {
    close(fd);
    delete g;
    return rc;
  }
  *out = g;
  return MER_OK;
}

int mer_gguf_close(mer_gguf *g) {
  if (g) {
    if (g->fd >= 0) close(g->fd);
    delete g;
  }
  return MER_OK;
}

int mer_gguf_moe_layer(mer_gguf *g, size_t layer, mer_gguf_moe_info *out) {
  if (!g || !out) return report_error(MER_ERR_INVALID_LAYOUT, "null argument");
  LayerGeom lg;
  const int rc = layer_geometry(g, layer, &lg);
  if (rc) return rc;
  *out = lg.info;
  return MER_OK;
}

int mer_gguf_read_expert(mer_gguf *g, size_t layer, size_t expert, void *dst, size_t dst_len) {
  if (!g || !dst) return report_error(MER_ERR_INVALID_LAYOUT, "null argument");
  LayerGeom lg;
  int rc = layer_geometry(g, layer, &lg);
  if (rc) return rc;
  const mer_gguf_moe_info &in = lg.info;
  if (expert >= in.n_experts) return report_error(MER_ERR_INVALID_LAYOUT, "expert index beyond the layer's expert count");
  if (dst_len < in.expert_bytes) return report_error(MER_ERR_BUFFER_TOO_SMALL, "destination smaller than one expert blob");
  const uint64_t proj = in.expert_bytes / 3;
  uint8_t *d = (uint8_t *)dst;
  static const char *kProj[3] = {"gate", "up", "down"};
  for (int i = 0; i < 3; ++i) {
    uint64_t off;
    if (in.layout == 0) {
      off = g->data_start + lg.t[i]->offset + (uint64_t)expert * proj;
    } else {
      auto it = g->tensors.find("blk." + std::to_string(layer) + ".ffn_" + kProj[i] + "." + std::to_string(expert) +
                                ".weight");
      if (it == g->tensors.end() || it->second.type != (in.dtype == MER_DTYPE_Q4_0 ? kGgmlQ4_0 : kGgmlQ8_0))
        return report_error(MER_ERR_INVALID_LAYOUT, "per-expert tensor missing or of another dtype");
      // gate / up [d_model, d_ff], down [d_ff, d_model] (GGML order)
      const std::vector<uint64_t> want = i < 2 ? std::vector<uint64_t>{in.d_model, in.d_ff}
                                               : std::vector<uint64_t>{in.d_ff, in.d_model};
      if (it->second.dims != want) return report_error(MER_ERR_INVALID_LAYOUT, "per-expert tensor shape disagrees with the layer's");
      off = g->data_start + it->second.offset;
    }
    if ((rc = read_range(g, off, proj, d + i * proj))) return rc;
  }
  return MER_OK;
}

}  // extern "C"
