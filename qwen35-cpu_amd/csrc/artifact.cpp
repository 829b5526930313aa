// Q35H128 v1 artifact reader/writer and the seeded random-init model
// generator. The byte format is the reference's (src/weights/q4_h128_artifact.cpp):
//   96-byte header: "Q35H128\0", u32 version 1, u32 0x01020304, u32 96, u32 64,
//     u64 tensor_count, u64 directory_offset (96), u64 directory_bytes,
//     u64 data_offset, u64 sign_seed, u32 layers, u32 hidden, u32 intermediate,
//     u32 vocab, zero padding;
//   directory entries: u32 name_size, u32 rank, u32 encoding, u32 transform_size,
//     u32 scale_group, u32 0, u64 sign_seed, u64 elements, u64 data_offset,
//     u64 data_size, u64 FNV-1a-64 checksum, name bytes, rank x u64 shape;
//   payloads 64-byte aligned.
// Weight packing follows the reference math: H128 rotation with the
// randomized signs, absmax/7 binary16 scale, round half away from zero
// (q4_h128.cpp:195-252), then the DOT4 row-8 interleave (q4_dot4.cpp:5-18).
#include "q35_hip_api.h"

#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <fstream>
#include <string>
#include <thread>
#include <vector>

#include "runtime.h"

namespace {

constexpr char kMagic[8] = {'Q', '3', '5', 'H', '1', '2', '8', '\0'};
constexpr uint32_t kHeaderSize = 96, kAlignment = 64;

uint64_t fnv1a(const void *data, size_t n) {
  const auto *b = static_cast<const uint8_t *>(data);
  uint64_t h = 14695981039346656037ull;
  for (size_t i = 0; i < n; ++i) {
    h ^= b[i];
    h *= 1099511628211ull;
  }
  return h;
}

uint64_t mix64(uint64_t v) {
  v += 0x9e3779b97f4a7c15ull;
  v = (v ^ (v >> 30)) * 0xbf58476d1ce4e5b9ull;
  v = (v ^ (v >> 27)) * 0x94d049bb133111ebull;
  return v ^ (v >> 31);
}

uint64_t name_hash(const std::string &s) { return fnv1a(s.data(), s.size()); }

// Counter-based normal generator: one independent stream per (tensor, row).
struct Normal {
  uint64_t state;
  bool has_spare = false;
  float spare = 0.0F;
  explicit Normal(uint64_t seed) : state(seed) {}
  double uniform() {
    state = mix64(state);
    return (static_cast<double>(state >> 11) + 0.5) * (1.0 / 9007199254740992.0);
  }
  float next() {
    if (has_spare) {
      has_spare = false;
      return spare;
    }
    const double u1 = uniform(), u2 = uniform();
    const double r = std::sqrt(-2.0 * std::log(u1)), t = 6.283185307179586 * u2;
    spare = static_cast<float>(r * std::sin(t));
    has_spare = true;
    return static_cast<float>(r * std::cos(t));
  }
};

uint16_t f2h(float value) {
  // q8_0.cpp:18-55
  uint32_t bits;
  std::memcpy(&bits, &value, 4);
  const uint32_t sign = (bits >> 16) & 0x8000u, mag = bits & 0x7fffffffu;
  if (mag >= 0x7f800000u) {
    if (mag == 0x7f800000u) return static_cast<uint16_t>(sign | 0x7c00u);
    const uint16_t payload = static_cast<uint16_t>((mag >> 13) & 0x03ffu);
    return static_cast<uint16_t>(sign | 0x7c00u | payload | (payload == 0));
  }
  if (mag > 0x477fefffu) return static_cast<uint16_t>(sign | 0x7c00u);
  if (mag < 0x38800000u) {
    if (mag < 0x33000000u) return static_cast<uint16_t>(sign);
    const uint32_t e = mag >> 23, mant = (mag & 0x007fffffu) | 0x00800000u, shift = 126u - e;
    uint32_t hm = mant >> shift;
    const uint32_t rem = mant & ((1u << shift) - 1u), half = 1u << (shift - 1u);
    if (rem > half || (rem == half && (hm & 1u))) ++hm;
    return static_cast<uint16_t>(sign | hm);
  }
  const uint32_t rounded = mag + 0x00000fffu + ((mag >> 13) & 1u);
  return static_cast<uint16_t>(sign | ((rounded - 0x38000000u) >> 13));
}

float h2f(uint16_t h) {
  const uint32_t sign = static_cast<uint32_t>(h & 0x8000u) << 16;
  uint32_t e = (h >> 10) & 0x1fu, m = h & 0x3ffu, bits;
  if (e == 0) {
    if (m == 0) {
      bits = sign;
    } else {
      uint32_t ne = 113u;
      while ((m & 0x400u) == 0) { m <<= 1; --ne; }
      bits = sign | (ne << 23) | ((m & 0x3ffu) << 13);
    }
  } else if (e == 0x1fu) {
    bits = sign | 0x7f800000u | (m << 13);
  } else {
    bits = sign | ((e + 112u) << 23) | (m << 13);
  }
  float f;
  std::memcpy(&f, &bits, 4);
  return f;
}

uint64_t sign_word(uint64_t block, uint64_t word, uint64_t seed) {
  return mix64(seed + block * 0x9e3779b97f4a7c15ull + word * 0xd1b54a32d192ed03ull);
}

// One 32-value Q4_0 block (18 bytes): q4_h128_quantize_transformed, q4_h128.cpp:195-222
void quantize_q4(const float *v, uint8_t *out18) {
  float amax = 0.0F;
  for (int i = 0; i < 32; ++i) amax = std::max(amax, std::fabs(v[i]));
  const uint16_t d = f2h(amax / 7.0F);
  const float stored = h2f(d);
  const float inv = stored == 0.0F ? 0.0F : 1.0F / stored;
  std::memcpy(out18, &d, 2);
  for (int i = 0; i < 16; ++i) {
    const int lo = static_cast<int>(std::clamp(std::round(v[i] * inv), -7.0F, 7.0F));
    const int hi = static_cast<int>(std::clamp(std::round(v[i + 16] * inv), -7.0F, 7.0F));
    out18[2 + i] = static_cast<uint8_t>((lo + 8) | ((hi + 8) << 4));
  }
}

// Scaled H128 transform of one 128-block (q4_h128.cpp:63-75)
void h128_block(float *x, size_t block, uint64_t seed) {
  for (int w = 0; w < 2; ++w) {
    const uint64_t s = sign_word(block, w, seed);
    for (int b = 0; b < 64; ++b)
      if ((s >> b) & 1u) x[w * 64 + b] = -x[w * 64 + b];
  }
  for (int stride = 1; stride < 128; stride *= 2)
    for (int base = 0; base < 128; base += 2 * stride)
      for (int l = 0; l < stride; ++l) {
        const float a = x[base + l], b = x[base + stride + l];
        x[base + l] = a + b;
        x[base + stride + l] = a - b;
      }
  for (int i = 0; i < 128; ++i) x[i] *= 0.08838834764831844055F;
}

// Random [rows, cols] matrix -> DOT4 packed Q4_0BlockX8 bytes.
std::vector<uint8_t> random_dot4(const std::string &name, uint64_t seed, uint64_t rows, uint64_t cols,
                                 float stdev, bool h128, uint64_t sign_seed) {
  const uint64_t blocks = cols / 32;
  std::vector<uint8_t> out(rows / 8 * blocks * 144);
  const uint64_t base = seed ^ name_hash(name);
  const unsigned threads = std::max(1u, std::min(16u, std::thread::hardware_concurrency()));
  auto work = [&](uint64_t t0, uint64_t t1) {
    std::vector<float> row(cols);
    std::vector<uint8_t> canon(8 * blocks * 18);
    for (uint64_t rt = t0; rt < t1; ++rt) {
      for (int r = 0; r < 8; ++r) {
        Normal g(mix64(base + (rt * 8 + r) * 0x632be59bd9b4e019ull));
        for (uint64_t c = 0; c < cols; ++c) row[c] = g.next() * stdev;
        if (h128)
          for (uint64_t b = 0; b < cols / 128; ++b) h128_block(row.data() + b * 128, b, sign_seed);
        for (uint64_t b = 0; b < blocks; ++b) quantize_q4(row.data() + b * 32, &canon[(r * blocks + b) * 18]);
      }
      // q4_dot4_pack_rows_8: qs[32t+4r+j] = u[r][8t+j] | u[r][8t+4+j] << 4
      for (uint64_t b = 0; b < blocks; ++b) {
        uint8_t *dst = &out[(rt * blocks + b) * 144];
        for (int r = 0; r < 8; ++r) {
          const uint8_t *src = &canon[(r * blocks + b) * 18];
          std::memcpy(dst + 2 * r, src, 2);
          auto nib = [&](int k) { return (src[2 + k % 16] >> (4 * (k / 16))) & 15; };
          for (int t = 0; t < 4; ++t)
            for (int j = 0; j < 4; ++j)
              dst[16 + 32 * t + 4 * r + j] = static_cast<uint8_t>(nib(8 * t + j) | (nib(8 * t + 4 + j) << 4));
        }
      }
    }
  };
  std::vector<std::thread> pool;
  const uint64_t tiles = rows / 8;
  for (unsigned i = 0; i < threads; ++i) {
    const uint64_t a = tiles * i / threads, b = tiles * (i + 1) / threads;
    if (a < b) pool.emplace_back(work, a, b);
  }
  for (auto &t : pool) t.join();
  return out;
}

// Random [rows, cols] identity-basis matrix -> Q4G16Tile bytes (q4_g16.h:5-6):
// per row, block and 16-column half an absmax/7 binary16 scale, codes
// round(x / d) + 8 clamped to 0..15, in the DOT4 nibble order.
std::vector<uint8_t> random_g16(const std::string &name, uint64_t seed, uint64_t rows, uint64_t cols, float stdev) {
  const uint64_t blocks = cols / 32;
  std::vector<uint8_t> out(rows / 8 * blocks * 160, 0);
  const uint64_t base = seed ^ name_hash(name);
  std::vector<float> row(cols);
  for (uint64_t r = 0; r < rows; ++r) {
    Normal g(mix64(base + r * 0x632be59bd9b4e019ull));
    for (uint64_t c = 0; c < cols; ++c) row[c] = g.next() * stdev;
    for (uint64_t b = 0; b < blocks; ++b) {
      uint8_t *tile = &out[((r / 8) * blocks + b) * 160];
      for (int half = 0; half < 2; ++half) {
        const float *x = row.data() + b * 32 + 16 * half;
        float amax = 0.0F;
        for (int i = 0; i < 16; ++i) amax = std::max(amax, std::fabs(x[i]));
        const uint16_t d = f2h(amax / 7.0F);
        std::memcpy(tile + 2 * (8 * half + r % 8), &d, 2);
        const float stored = h2f(d), inv = stored > 0.0F ? 1.0F / stored : 0.0F;
        for (int i = 0; i < 16; ++i) {
          const int k = 16 * half + i;
          const int q = static_cast<int>(std::clamp(std::round(x[i] * inv), -8.0F, 7.0F)) + 8;
          tile[32 + 32 * (k / 8) + 4 * (r % 8) + k % 4] |= static_cast<uint8_t>(q << (k % 8 < 4 ? 0 : 4));
        }
      }
    }
  }
  return out;
}

// Random [rows, cols] matrix -> row-major Q8_0 blocks (binary16 scale + 32
// codes; q8_0_quantize, q8_0.cpp:86-110).
std::vector<uint8_t> random_q8(const std::string &name, uint64_t seed, uint64_t rows, uint64_t cols, float stdev) {
  const uint64_t blocks = cols / 32;
  std::vector<uint8_t> out(rows * blocks * 34);
  const uint64_t base = seed ^ name_hash(name);
  std::vector<float> row(cols);
  for (uint64_t r = 0; r < rows; ++r) {
    Normal g(mix64(base + r * 0x632be59bd9b4e019ull));
    for (uint64_t c = 0; c < cols; ++c) row[c] = g.next() * stdev;
    for (uint64_t b = 0; b < blocks; ++b) {
      const float *x = row.data() + b * 32;
      float amax = 0.0F;
      for (int i = 0; i < 32; ++i) amax = std::max(amax, std::fabs(x[i]));
      const float scale = amax / 127.0F, inv = scale == 0.0F ? 0.0F : 1.0F / scale;
      uint8_t *dst = &out[(r * blocks + b) * 34];
      const uint16_t d = f2h(scale);
      std::memcpy(dst, &d, 2);
      for (int i = 0; i < 32; ++i)
        dst[2 + i] = static_cast<uint8_t>(static_cast<int8_t>(std::clamp(std::round(x[i] * inv), -127.0F, 127.0F)));
    }
  }
  return out;
}

struct Entry {
  std::string name;
  std::vector<uint64_t> shape;
  uint32_t encoding = 0, transform = 0, group = 0;
  uint64_t seed = 0, elements = 0, offset = 0, size = 0, checksum = 0;
};

uint64_t align_up(uint64_t v, uint64_t a) { return (v + a - 1) / a * a; }

// Tensor plan of the packed artifact (q4_h128_convert_main.cpp:52-170 names,
// fused rows as loaded by weights.inl:1697-1771).
std::vector<Entry> plan(const q35_model_dims &d, const uint8_t *is_linear, uint32_t flags) {
  std::vector<Entry> e;
  const uint64_t H = d.hidden, I = d.intermediate, hd = d.head_dim;
  const uint64_t q_dim = static_cast<uint64_t>(d.lin_k_heads) * d.lin_k_dim;
  const uint64_t v_dim = static_cast<uint64_t>(d.lin_v_heads) * d.lin_v_dim;
  const uint64_t ch = 2 * q_dim + v_dim;
  auto q4 = [&](const std::string &n, uint64_t r, uint64_t c, bool h128) {
    Entry x;
    x.name = n;
    x.shape = {r, c};
    x.encoding = h128 ? Q35_ENC_Q4_H128_DOT4 : Q35_ENC_Q4_0_DOT4;
    x.transform = h128 ? 128 : 0;
    x.group = 32;
    x.seed = h128 ? d.sign_seed : 0;
    x.size = r / 8 * (c / 32) * 144;
    e.push_back(x);
  };
  auto f32 = [&](const std::string &n, std::vector<uint64_t> shape) {
    Entry x;
    x.name = n;
    x.shape = shape;
    x.encoding = Q35_ENC_F32;
    uint64_t k = 1;
    for (auto s : shape) k *= s;
    x.size = k * 4;
    e.push_back(x);
  };
  if (flags & Q35_ARTIFACT_HEAD_G16) {
    // q4_g16_cpu_dot4: identity basis, 16-column scale groups
    Entry x;
    x.name = "model.language_model.embed_tokens.weight";
    x.shape = {static_cast<uint64_t>(d.vocab), H};
    x.encoding = Q35_ENC_Q4_G16_DOT4;
    x.group = 16;
    x.size = static_cast<uint64_t>(d.vocab) / 8 * (H / 32) * 160;
    e.push_back(x);
  } else {
    q4("model.language_model.embed_tokens.weight", d.vocab, H, false);
  }
  f32("model.language_model.norm.weight", {H});
  for (int i = 0; i < d.n_layers; ++i) {
    const std::string p = "model.language_model.layers." + std::to_string(i) + ".";
    f32(p + "input_layernorm.weight", {H});
    f32(p + "post_attention_layernorm.weight", {H});
    q4(p + "mlp.gate_up_proj.weight", 2 * I, H, true);
    q4(p + "mlp.down_proj.weight", H, I, true);
    if (is_linear[i]) {
      if (flags & Q35_ARTIFACT_Q8_GATES) {
        // [qkv | z] as Q4 and the b, a rows as Q8_0 (weights.inl:1700-1747)
        q4(p + "linear_attn.in_proj_all.weight", ch + v_dim, H, true);
        Entry x;
        x.name = p + "linear_attn.in_proj_ba.weight";
        x.shape = {2 * static_cast<uint64_t>(d.lin_v_heads), H};
        x.encoding = Q35_ENC_Q8_0;
        x.group = 32;
        x.size = x.shape[0] * (H / 32) * 34;
        e.push_back(x);
      } else {
        q4(p + "linear_attn.in_proj_all.weight", ch + v_dim + 2 * static_cast<uint64_t>(d.lin_v_heads), H, true);
      }
      f32(p + "linear_attn.conv1d.weight", {ch, 1, static_cast<uint64_t>(d.lin_kernel)});
      q4(p + "linear_attn.out_proj.weight", H, v_dim, true);
      f32(p + "linear_attn.norm.weight", {static_cast<uint64_t>(d.lin_v_dim)});
      f32(p + "linear_attn.A_log", {static_cast<uint64_t>(d.lin_v_heads)});
      f32(p + "linear_attn.dt_bias", {static_cast<uint64_t>(d.lin_v_heads)});
    } else {
      q4(p + "self_attn.qkv_proj.weight", 2 * d.n_heads * hd + 2 * d.n_kv_heads * hd, H, true);
      q4(p + "self_attn.o_proj.weight", H, d.n_heads * hd, true);
      f32(p + "self_attn.q_norm.weight", {hd});
      f32(p + "self_attn.k_norm.weight", {hd});
    }
  }
  for (auto &x : e) {
    x.elements = 1;
    for (auto s : x.shape) x.elements *= s;
  }
  return e;
}

std::vector<uint8_t> f32_payload(const Entry &x, uint64_t seed) {
  std::vector<float> v(x.elements, 0.0F);
  const std::string &n = x.name;
  auto ends_with = [&](const char *s) {
    const size_t l = std::strlen(s);
    return n.size() >= l && n.compare(n.size() - l, l, s) == 0;
  };
  Normal g(mix64(seed ^ name_hash(n)));
  if (ends_with("linear_attn.norm.weight")) {
    std::fill(v.begin(), v.end(), 1.0F);  // gated RMSNorm, offset 0
  } else if (ends_with("linear_attn.A_log")) {
    for (auto &a : v) a = static_cast<float>(std::log(1.0 + 15.0 * g.uniform()));
  } else if (ends_with("linear_attn.dt_bias")) {
    for (auto &a : v) a = 0.5F * g.next();
  } else if (ends_with("linear_attn.conv1d.weight")) {
    for (auto &a : v) a = 0.3F * g.next();
  }  // every (1 + w) norm weight stays 0
  std::vector<uint8_t> b(v.size() * 4);
  std::memcpy(b.data(), v.data(), b.size());
  return b;
}

void write_u32(std::vector<uint8_t> &o, uint32_t v) { o.insert(o.end(), reinterpret_cast<uint8_t *>(&v), reinterpret_cast<uint8_t *>(&v) + 4); }
void write_u64(std::vector<uint8_t> &o, uint64_t v) { o.insert(o.end(), reinterpret_cast<uint8_t *>(&v), reinterpret_cast<uint8_t *>(&v) + 8); }

}  // namespace

// The FP32 rows the generator quantizes for tensor `name` (before the H128
// rotation), so tests can push the same rows through the reference packer.
extern "C" int q35_random_weight_rows(const char *name, uint64_t seed, uint64_t row0, uint64_t rows,
                                      uint64_t cols, float stdev, float *out) {
  if (name == nullptr || out == nullptr) return Q35_ERR_INVALID;
  const uint64_t base = seed ^ name_hash(name);
  for (uint64_t r = 0; r < rows; ++r) {
    Normal g(mix64(base + (row0 + r) * 0x632be59bd9b4e019ull));
    for (uint64_t c = 0; c < cols; ++c) out[r * cols + c] = g.next() * stdev;
  }
  return Q35_OK;
}

extern "C" int q35_write_random_artifact(const char *path, const q35_model_dims *d,
                                         const uint8_t *is_linear, uint64_t seed, float stdev) {
  return q35_write_random_artifact_ex(path, d, is_linear, seed, stdev, 0);
}

extern "C" int q35_write_random_artifact_ex(const char *path, const q35_model_dims *d, const uint8_t *is_linear,
                                            uint64_t seed, float stdev, uint32_t flags) {
  if (path == nullptr || d == nullptr || is_linear == nullptr) return Q35_ERR_INVALID;
  std::vector<Entry> e = plan(*d, is_linear, flags);
  uint64_t dir_bytes = 0;
  for (auto &x : e) dir_bytes += 64 + x.name.size() + 8 * x.shape.size();
  const uint64_t data_offset = align_up(kHeaderSize + dir_bytes, kAlignment);
  uint64_t cursor = data_offset;
  for (auto &x : e) {
    cursor = align_up(cursor, kAlignment);
    x.offset = cursor;
    cursor += x.size;
  }
  std::FILE *f = std::fopen(path, "wb+");
  if (f == nullptr) return Q35_ERR_IO;
  bool ok = true;
  for (auto &x : e) {
    std::vector<uint8_t> payload;
    if (x.encoding == Q35_ENC_F32)
      payload = f32_payload(x, seed);
    else if (x.encoding == Q35_ENC_Q4_G16_DOT4)
      payload = random_g16(x.name, seed, x.shape[0], x.shape[1], stdev);
    else if (x.encoding == Q35_ENC_Q8_0)
      payload = random_q8(x.name, seed, x.shape[0], x.shape[1], stdev);
    else
      payload = random_dot4(x.name, seed, x.shape[0], x.shape[1], stdev, x.encoding == Q35_ENC_Q4_H128_DOT4,
                            d->sign_seed);
    if (payload.size() != x.size) { ok = false; break; }
    x.checksum = fnv1a(payload.data(), payload.size());
    ok = ok && std::fseek(f, static_cast<long>(x.offset), SEEK_SET) == 0 &&
         std::fwrite(payload.data(), 1, payload.size(), f) == payload.size();
    if (!ok) break;
  }
  if (ok) {
    std::vector<uint8_t> h;
    h.insert(h.end(), kMagic, kMagic + 8);
    write_u32(h, 1);
    write_u32(h, 0x01020304u);
    write_u32(h, kHeaderSize);
    write_u32(h, kAlignment);
    write_u64(h, e.size());
    write_u64(h, kHeaderSize);
    write_u64(h, dir_bytes);
    write_u64(h, data_offset);
    write_u64(h, d->sign_seed);
    write_u32(h, static_cast<uint32_t>(d->n_layers));
    write_u32(h, static_cast<uint32_t>(d->hidden));
    write_u32(h, static_cast<uint32_t>(d->intermediate));
    write_u32(h, static_cast<uint32_t>(d->vocab));
    h.resize(kHeaderSize, 0);
    for (auto &x : e) {
      write_u32(h, static_cast<uint32_t>(x.name.size()));
      write_u32(h, static_cast<uint32_t>(x.shape.size()));
      write_u32(h, x.encoding);
      write_u32(h, x.transform);
      write_u32(h, x.group);
      write_u32(h, 0);
      write_u64(h, x.seed);
      write_u64(h, x.elements);
      write_u64(h, x.offset);
      write_u64(h, x.size);
      write_u64(h, x.checksum);
      h.insert(h.end(), x.name.begin(), x.name.end());
      for (auto s : x.shape) write_u64(h, s);
    }
    ok = std::fseek(f, 0, SEEK_SET) == 0 && std::fwrite(h.data(), 1, h.size(), f) == h.size();
  }
  ok = (std::fclose(f) == 0) && ok;
  return ok ? Q35_OK : Q35_ERR_IO;
}

extern "C" int q35_model_load_artifact(q35_context *ctx, const char *path, const q35_model_dims *dims,
                                       const uint8_t *is_linear, q35_model **out) {
  if (ctx == nullptr || path == nullptr || dims == nullptr || out == nullptr) return Q35_ERR_INVALID;
  *out = nullptr;
  std::ifstream f(path, std::ios::binary);
  if (!f) return q35::set_error(ctx, Q35_ERR_IO, std::string("cannot open ") + path);
  f.seekg(0, std::ios::end);
  const uint64_t file_size = static_cast<uint64_t>(f.tellg());
  f.seekg(0, std::ios::beg);
  uint8_t hdr[kHeaderSize];
  if (file_size < kHeaderSize || !f.read(reinterpret_cast<char *>(hdr), kHeaderSize))
    return q35::set_error(ctx, Q35_ERR_IO, "truncated artifact header");
  auto u32 = [&](const uint8_t *p) { uint32_t v; std::memcpy(&v, p, 4); return v; };
  auto u64 = [&](const uint8_t *p) { uint64_t v; std::memcpy(&v, p, 8); return v; };
  if (std::memcmp(hdr, kMagic, 8) != 0 || u32(hdr + 8) != 1 || u32(hdr + 12) != 0x01020304u ||
      u32(hdr + 16) != kHeaderSize || u32(hdr + 20) != kAlignment || u64(hdr + 32) != kHeaderSize)
    return q35::set_error(ctx, Q35_ERR_IO, "not a Q35H128 v1 artifact");
  const uint64_t count = u64(hdr + 24), dir_bytes = u64(hdr + 40), seed = u64(hdr + 56);
  if (u32(hdr + 64) != static_cast<uint32_t>(dims->n_layers) || u32(hdr + 68) != static_cast<uint32_t>(dims->hidden) ||
      u32(hdr + 72) != static_cast<uint32_t>(dims->intermediate) || u32(hdr + 76) != static_cast<uint32_t>(dims->vocab) ||
      seed == 0 || (dims->sign_seed != 0 && seed != dims->sign_seed))
    return q35::set_error(ctx, Q35_ERR_IO, "artifact fingerprint does not match the model dims");
  if (count == 0 || count > 100000 || kHeaderSize + dir_bytes > file_size)
    return q35::set_error(ctx, Q35_ERR_IO, "bad artifact directory");
  std::vector<uint8_t> dir(dir_bytes);
  if (!f.read(reinterpret_cast<char *>(dir.data()), static_cast<std::streamsize>(dir_bytes)))
    return q35::set_error(ctx, Q35_ERR_IO, "truncated directory");
  q35_model_dims md = *dims;
  md.sign_seed = seed;  // 0 in dims: the artifact's own H128 sign seed
  q35_model *m = nullptr;
  int st = q35_model_create(ctx, &md, is_linear, &m);
  if (st != Q35_OK) return st;
  size_t o = 0;
  std::vector<uint8_t> payload;
  for (uint64_t i = 0; i < count && st == Q35_OK; ++i) {
    if (o + 64 > dir.size()) { st = q35::set_error(ctx, Q35_ERR_IO, "bad directory entry"); break; }
    const uint32_t name_size = u32(&dir[o]), rank = u32(&dir[o + 4]), enc = u32(&dir[o + 8]);
    const uint64_t offset = u64(&dir[o + 40]), size = u64(&dir[o + 48]), checksum = u64(&dir[o + 56]);
    o += 64;
    if (name_size == 0 || name_size > 4096 || rank == 0 || rank > 8 ||
        o + name_size + 8ull * rank > dir.size()) {
      st = q35::set_error(ctx, Q35_ERR_IO, "bad directory entry");
      break;
    }
    const std::string name(reinterpret_cast<const char *>(&dir[o]), name_size);
    o += name_size;
    std::vector<uint64_t> shape(rank);
    for (uint32_t r = 0; r < rank; ++r, o += 8) shape[r] = u64(&dir[o]);
    if (offset % kAlignment || offset + size > file_size) {
      st = q35::set_error(ctx, Q35_ERR_IO, "bad payload range for " + name);
      break;
    }
    payload.resize(size);
    f.seekg(static_cast<std::streamoff>(offset), std::ios::beg);
    if (!f.read(reinterpret_cast<char *>(payload.data()), static_cast<std::streamsize>(size)) ||
        fnv1a(payload.data(), payload.size()) != checksum) {
      st = q35::set_error(ctx, Q35_ERR_IO, "checksum mismatch for " + name);
      break;
    }
    // tensors the decode path does not use (e.g. MTP sidecars) are skipped
    if (!m->required.count(name)) continue;
    st = q35_model_upload_tensor(m, name.c_str(), static_cast<int>(enc), shape.data(), rank, payload.data(),
                                 payload.size());
  }
  if (st == Q35_OK) st = q35_model_finalize(m);
  if (st != Q35_OK) {
    q35_model_destroy(m);
    return st;
  }
  *out = m;
  return Q35_OK;
}
