// Model upload, request slots, KV page pool and the batched decode step
// (the MI355X body of CpuEngine::Impl::forward_batch, cpu_engine.inl:201-325).
#include "runtime.h"

#include "q35_hip_api.h"

#include <algorithm>
#include <cmath>
#include <cstring>
#include <new>
#include <string>
#include <vector>

using namespace q35;

namespace {

size_t align256(size_t n) { return (n + 255) & ~static_cast<size_t>(255); }

// IEEE binary16 -> float (subnormals, infinities and NaN included)
float half_bits_to_float_host(uint16_t h) {
  const uint32_t sign = static_cast<uint32_t>(h & 0x8000u) << 16;
  const int e = (h >> 10) & 0x1f;
  const uint32_t mant = h & 0x3ffu;
  float v;
  if (e == 0)
    v = std::ldexp(static_cast<float>(mant), -24);
  else if (e == 31)
    v = mant != 0 ? std::nanf("") : INFINITY;
  else
    v = std::ldexp(static_cast<float>(mant | 0x400u), e - 25);
  uint32_t bits;
  std::memcpy(&bits, &v, 4);
  bits |= sign;
  std::memcpy(&v, &bits, 4);
  return v;
}

std::string layer_prefix(int i) {
  return "model.language_model.layers." + std::to_string(i) + ".";
}

int model_alloc(q35_model *m, size_t bytes, void **out) {
  Q35_HIP_TRY(m->ctx, hipMalloc(out, bytes ? bytes : 1));
  m->allocations.push_back(*out);
  return Q35_OK;
}

int rt_alloc(q35_runtime *rt, size_t bytes, void **out) {
  Q35_HIP_TRY(rt->ctx, hipMalloc(out, bytes ? bytes : 1));
  rt->allocations.push_back(*out);
  return Q35_OK;
}

}  // namespace

// ===================================================================== model
extern "C" int q35_model_dims_preset(int which, q35_model_dims *d, uint8_t *is_linear,
                                     size_t capacity) {
  if (d == nullptr) return Q35_ERR_INVALID;
  // text_architecture, src/compiler/profile_loader.cpp:439-462; RuntimeDims
  // defaults (weights.inl:336-357, profile_loader.cpp:366-378)
  q35_model_dims x{};
  x.vocab = 248320;
  x.head_dim = 256;
  x.rope_theta = 10000000.0F;
  x.rms_eps = 1.0e-6F;
  x.lin_kernel = 4;
  x.lin_k_heads = 16;
  x.lin_k_dim = 128;
  x.lin_v_dim = 128;
  x.sign_seed = 0x5148333548313238ull;  // q4_h128.h:25-26
  if (which == 0) {
    x.n_layers = 24; x.hidden = 1024; x.intermediate = 3584;
    x.n_heads = 8; x.n_kv_heads = 2; x.lin_v_heads = 16;
  } else if (which == 1) {
    x.n_layers = 24; x.hidden = 2048; x.intermediate = 6144;
    x.n_heads = 8; x.n_kv_heads = 2; x.lin_v_heads = 16;
  } else if (which == 2) {
    x.n_layers = 32; x.hidden = 2560; x.intermediate = 9216;
    x.n_heads = 16; x.n_kv_heads = 4; x.lin_v_heads = 32;
  } else {
    return Q35_ERR_INVALID;
  }
  // partial_rotary_factor 0.25 (weights.inl:1580-1583)
  x.rope_dim = static_cast<int32_t>(static_cast<float>(x.head_dim) * 0.25F);
  if (x.rope_dim % 2) x.rope_dim -= 1;
  *d = x;
  if (is_linear != nullptr) {
    if (capacity < static_cast<size_t>(x.n_layers)) return Q35_ERR_INVALID;
    for (int i = 0; i < x.n_layers; ++i) is_linear[i] = ((i + 1) % 4 != 0) ? 1 : 0;
  }
  return Q35_OK;
}

extern "C" int q35_model_create(q35_context *ctx, const q35_model_dims *dims,
                                const uint8_t *layer_is_linear, q35_model **out) {
  if (ctx == nullptr || dims == nullptr || layer_is_linear == nullptr || out == nullptr)
    return Q35_ERR_INVALID;
  *out = nullptr;
  const q35_model_dims &d = *dims;
  if (d.n_layers <= 0 || d.hidden <= 0 || d.hidden % 128 || d.intermediate % 128 ||
      d.vocab <= 0 || d.vocab % 8 || d.n_heads <= 0 || d.n_kv_heads <= 0 ||
      d.n_heads % d.n_kv_heads || d.head_dim != 256 || d.lin_k_dim != 128 || d.lin_v_dim != 128 ||
      d.lin_v_heads % d.lin_k_heads || d.lin_kernel != 4 || d.rope_dim <= 0 || d.rope_dim > d.head_dim ||
      (d.lin_v_heads * d.lin_v_dim) % 128 || (d.n_heads * d.head_dim) % 128)
    return set_error(ctx, Q35_ERR_UNSUPPORTED, "model shape outside the kernels' support");
  auto *m = new (std::nothrow) q35_model();
  if (m == nullptr) return Q35_ERR_OOM;
  m->ctx = ctx;
  m->d = d;
  m->is_linear.assign(layer_is_linear, layer_is_linear + d.n_layers);
  m->layers.resize(d.n_layers);
  m->linear_index.assign(d.n_layers, -1);
  m->full_index.assign(d.n_layers, -1);
  m->required = {"model.language_model.embed_tokens.weight", "model.language_model.norm.weight"};
  for (int i = 0; i < d.n_layers; ++i) {
    const std::string p = layer_prefix(i);
    m->layers[i].linear = m->is_linear[i] != 0;
    for (const char *n : {"input_layernorm.weight", "post_attention_layernorm.weight",
                          "mlp.gate_up_proj.weight", "mlp.down_proj.weight"})
      m->required.insert(p + n);
    if (m->layers[i].linear) {
      m->linear_index[i] = m->n_linear++;
      for (const char *n : {"linear_attn.in_proj_all.weight", "linear_attn.conv1d.weight",
                            "linear_attn.out_proj.weight", "linear_attn.norm.weight",
                            "linear_attn.A_log", "linear_attn.dt_bias"})
        m->required.insert(p + n);
    } else {
      m->full_index[i] = m->n_full++;
      for (const char *n : {"self_attn.qkv_proj.weight", "self_attn.o_proj.weight",
                            "self_attn.q_norm.weight", "self_attn.k_norm.weight"})
        m->required.insert(p + n);
    }
  }
  *out = m;
  return Q35_OK;
}

extern "C" void q35_model_destroy(q35_model *m) {
  if (m == nullptr) return;
  (void)hipSetDevice(m->ctx->device);
  (void)hipStreamSynchronize(m->ctx->stream);
  for (void *p : m->allocations) (void)hipFree(p);
  delete m;
}

namespace {

int expect_shape(q35_model *m, const std::string &name, const uint64_t *shape, size_t rank,
                 std::initializer_list<uint64_t> want) {
  bool ok = rank == want.size();
  size_t i = 0;
  for (uint64_t w : want) {
    if (!ok) break;
    ok = shape[i++] == w;
  }
  return ok ? Q35_OK : set_error(m->ctx, Q35_ERR_INVALID, "wrong shape for " + name);
}

// Uploads `bytes` to a fresh device buffer; returns its address in *dst.
int upload(q35_model *m, const void *host, size_t bytes, const void **dst) {
  void *p = nullptr;
  int st = model_alloc(m, bytes, &p);
  if (st != Q35_OK) return st;
  Q35_HIP_TRY(m->ctx, hipMemcpy(p, host, bytes, hipMemcpyHostToDevice));
  *dst = p;
  return Q35_OK;
}

}  // namespace

extern "C" int q35_model_upload_tensor(q35_model *m, const char *name_c, int encoding,
                                       const uint64_t *shape, size_t rank, const void *bytes,
                                       size_t count) {
  if (m == nullptr || name_c == nullptr || shape == nullptr || bytes == nullptr) return Q35_ERR_INVALID;
  const std::string name(name_c);
  const q35_model_dims &d = m->d;
  const uint64_t H = d.hidden, I = d.intermediate;
  const uint64_t q_dim = static_cast<uint64_t>(d.lin_k_heads) * d.lin_k_dim;
  const uint64_t v_dim = static_cast<uint64_t>(d.lin_v_heads) * d.lin_v_dim;
  const uint64_t ch = 2 * q_dim + v_dim;
  const uint64_t hd = d.head_dim;
  auto q4 = [&](std::initializer_list<uint64_t> want, int enc, const q35_q4_0_block_x8 **dst,
                size_t *weight_bytes) -> int {
    int st = expect_shape(m, name, shape, rank, want);
    if (st != Q35_OK) return st;
    if (encoding != enc) return set_error(m->ctx, Q35_ERR_INVALID, "wrong encoding for " + name);
    const uint64_t rows = shape[0], cols = shape[1];
    if (rows % 8 || cols % 32 || count != rows / 8 * (cols / 32) * 144)
      return set_error(m->ctx, Q35_ERR_INVALID, "wrong DOT4 payload size for " + name);
    *weight_bytes += count;
    return upload(m, bytes, count, reinterpret_cast<const void **>(dst));
  };
  auto f32 = [&](std::initializer_list<uint64_t> want, const float **dst) -> int {
    int st = expect_shape(m, name, shape, rank, want);
    if (st != Q35_OK) return st;
    uint64_t n = 1;
    for (uint64_t w : want) n *= w;
    if (encoding != Q35_ENC_F32 || count != n * 4)
      return set_error(m->ctx, Q35_ERR_INVALID, "wrong F32 payload for " + name);
    return upload(m, bytes, count, reinterpret_cast<const void **>(dst));
  };
  int st = Q35_ERR_INVALID;
  if (name == "model.language_model.embed_tokens.weight" && encoding == Q35_ENC_Q4_G16_DOT4) {
    // Q4G16Tile head (weights.inl:724-734): 160 bytes per 8-row x 32-column
    // tile, every binary16 scale finite
    st = expect_shape(m, name, shape, rank, {static_cast<uint64_t>(d.vocab), H});
    if (st == Q35_OK && (d.vocab % 8 != 0 || H % 32 != 0 || count != static_cast<size_t>(d.vocab) / 8 * (H / 32) * 160))
      st = set_error(m->ctx, Q35_ERR_INVALID, "wrong G16 payload size for " + name);
    if (st == Q35_OK) {
      const uint8_t *b = static_cast<const uint8_t *>(bytes);
      for (size_t t = 0; t < count / 160 && st == Q35_OK; ++t)
        for (int i = 0; i < 16; ++i) {
          uint16_t s;
          std::memcpy(&s, b + t * 160 + 2 * i, 2);
          if ((s & 0x7c00u) == 0x7c00u) {
            st = set_error(m->ctx, Q35_ERR_INVALID, "non-finite G16 scale in " + name);
            break;
          }
        }
    }
    if (st == Q35_OK) {
      m->weight_bytes += count;
      st = upload(m, bytes, count, reinterpret_cast<const void **>(&m->embed));
      m->embed_g16 = st == Q35_OK;
    }
  } else if (name == "model.language_model.embed_tokens.weight") {
    st = q4({static_cast<uint64_t>(d.vocab), H}, Q35_ENC_Q4_0_DOT4, &m->embed, &m->weight_bytes);
  } else if (name == "model.language_model.norm.weight") {
    st = f32({H}, &m->final_norm);
  } else if (name.rfind("model.language_model.layers.", 0) == 0) {
    const size_t p0 = std::strlen("model.language_model.layers.");
    const size_t dot = name.find('.', p0);
    if (dot == std::string::npos) return set_error(m->ctx, Q35_ERR_INVALID, "bad tensor name " + name);
    const int li = std::atoi(name.substr(p0, dot - p0).c_str());
    if (li < 0 || li >= d.n_layers) return set_error(m->ctx, Q35_ERR_INVALID, "bad layer in " + name);
    const std::string leaf = name.substr(dot + 1);
    LayerDev &L = m->layers[li];
    if (leaf == "input_layernorm.weight") st = f32({H}, &L.input_norm);
    else if (leaf == "post_attention_layernorm.weight") st = f32({H}, &L.post_norm);
    else if (leaf == "mlp.gate_up_proj.weight") st = q4({2 * I, H}, Q35_ENC_Q4_H128_DOT4, &L.gate_up, &m->weight_bytes);
    else if (leaf == "mlp.down_proj.weight") st = q4({H, I}, Q35_ENC_Q4_H128_DOT4, &L.down, &m->weight_bytes);
    else if (L.linear && leaf == "linear_attn.in_proj_all.weight") {
      // [qkv | z | b | a], or [qkv | z] when the gate rows are a separate
      // Q8 tensor (weights.inl:1700-1747)
      const bool split_gates = rank == 2 && shape[0] == ch + v_dim;
      st = q4({split_gates ? ch + v_dim : ch + v_dim + 2 * static_cast<uint64_t>(d.lin_v_heads), H},
              Q35_ENC_Q4_H128_DOT4, &L.in_proj, &m->weight_bytes);
      if (st == Q35_OK) {
        L.in_rows = static_cast<int>(shape[0]);
        if (split_gates) m->required.insert(layer_prefix(li) + "linear_attn.in_proj_ba.weight");
      }
    } else if (L.linear && leaf == "linear_attn.in_proj_ba.weight") {
      // Q8_0 gate rows [b | a] over the identity-basis input: F32 scales as
      // q8_0_scales_to_f32 keeps them, finite and non-negative (weights.inl:735-746)
      const uint64_t rows = 2 * static_cast<uint64_t>(d.lin_v_heads), nb = H / 32;
      st = expect_shape(m, name, shape, rank, {rows, H});
      if (st == Q35_OK && (encoding != Q35_ENC_Q8_0 || H % 32 != 0 || rows > static_cast<uint64_t>(kMaxGateRows) ||
                           count != rows * nb * 34))
        st = set_error(m->ctx, Q35_ERR_INVALID, "wrong Q8_0 payload for " + name);
      // the input-norm kernel stages every (gate row, 32-column block) dot in LDS
      if (st == Q35_OK && rows * nb > static_cast<uint64_t>(kMaxGateItems))
        st = set_error(m->ctx, Q35_ERR_UNSUPPORTED,
                       name + ": gate rows x hidden/32 exceeds the " + std::to_string(kMaxGateItems) +
                           " (row, block) items the input-norm kernel stages");
      std::vector<int8_t> codes(rows * H);
      std::vector<float> scales(rows * nb);
      const uint8_t *b = static_cast<const uint8_t *>(bytes);
      for (uint64_t i = 0; st == Q35_OK && i < rows * nb; ++i) {
        uint16_t h;
        std::memcpy(&h, b + i * 34, 2);
        scales[i] = half_bits_to_float_host(h);
        if (!std::isfinite(scales[i]) || scales[i] < 0.0F)
          st = set_error(m->ctx, Q35_ERR_INVALID, "invalid Q8 weight scale in " + name);
        std::memcpy(&codes[i * 32], b + i * 34 + 2, 32);
      }
      if (st == Q35_OK) st = upload(m, codes.data(), codes.size(), reinterpret_cast<const void **>(&L.gate_codes));
      if (st == Q35_OK) st = upload(m, scales.data(), scales.size() * 4, reinterpret_cast<const void **>(&L.gate_scales));
      if (st == Q35_OK) {
        L.gate_rows = static_cast<int>(rows);
        m->weight_bytes += count;
      }
    } else if (L.linear && leaf == "linear_attn.out_proj.weight") {
      st = q4({H, v_dim}, Q35_ENC_Q4_H128_DOT4, &L.out_proj, &m->weight_bytes);
      L.out_cols = static_cast<int>(v_dim);
    } else if (L.linear && leaf == "linear_attn.conv1d.weight") {
      st = expect_shape(m, name, shape, rank, {ch, 1, static_cast<uint64_t>(d.lin_kernel)});
      if (st == Q35_OK && (encoding != Q35_ENC_F32 || count != ch * d.lin_kernel * 4))
        st = set_error(m->ctx, Q35_ERR_INVALID, "wrong F32 payload for " + name);
      if (st == Q35_OK) {
        // pack_conv1d_kernel_major (weights.inl:532-544): [channel][kernel] -> [kernel][channel]
        const float *src = static_cast<const float *>(bytes);
        std::vector<float> km(ch * d.lin_kernel);
        for (int k = 0; k < d.lin_kernel; ++k)
          for (uint64_t c = 0; c < ch; ++c) km[k * ch + c] = src[c * d.lin_kernel + k];
        st = upload(m, km.data(), km.size() * 4, reinterpret_cast<const void **>(&L.conv_w));
      }
    } else if (L.linear && leaf == "linear_attn.norm.weight") st = f32({static_cast<uint64_t>(d.lin_v_dim)}, &L.lin_norm);
    else if (L.linear && leaf == "linear_attn.dt_bias") st = f32({static_cast<uint64_t>(d.lin_v_heads)}, &L.dt_bias);
    else if (L.linear && leaf == "linear_attn.A_log") {
      st = expect_shape(m, name, shape, rank, {static_cast<uint64_t>(d.lin_v_heads)});
      if (st == Q35_OK && (encoding != Q35_ENC_F32 || count != static_cast<size_t>(d.lin_v_heads) * 4))
        st = set_error(m->ctx, Q35_ERR_INVALID, "wrong F32 payload for " + name);
      if (st == Q35_OK) {
        // ssm_a = -exp(A_log) in FP32 (weights.inl:1750-1754)
        const float *src = static_cast<const float *>(bytes);
        std::vector<float> a(d.lin_v_heads);
        for (int h = 0; h < d.lin_v_heads; ++h) a[h] = -std::exp(src[h]);
        st = upload(m, a.data(), a.size() * 4, reinterpret_cast<const void **>(&L.ssm_a));
      }
    } else if (!L.linear && leaf == "self_attn.qkv_proj.weight") {
      st = q4({2 * d.n_heads * hd + 2 * d.n_kv_heads * hd, H}, Q35_ENC_Q4_H128_DOT4, &L.in_proj,
              &m->weight_bytes);
      L.in_rows = static_cast<int>(shape[0]);
    } else if (!L.linear && leaf == "self_attn.o_proj.weight") {
      st = q4({H, d.n_heads * hd}, Q35_ENC_Q4_H128_DOT4, &L.out_proj, &m->weight_bytes);
      L.out_cols = static_cast<int>(d.n_heads * hd);
    } else if (!L.linear && leaf == "self_attn.q_norm.weight") st = f32({hd}, &L.q_norm);
    else if (!L.linear && leaf == "self_attn.k_norm.weight") st = f32({hd}, &L.k_norm);
    else return set_error(m->ctx, Q35_ERR_INVALID, "unexpected tensor " + name);
  } else {
    return set_error(m->ctx, Q35_ERR_INVALID, "unexpected tensor " + name);
  }
  if (st == Q35_OK) m->uploaded.insert(name);
  return st;
}

extern "C" int q35_model_finalize(q35_model *m) {
  if (m == nullptr) return Q35_ERR_INVALID;
  for (const auto &n : m->required)
    if (!m->uploaded.count(n)) return set_error(m->ctx, Q35_ERR_STATE, "missing tensor " + n);
  const int full_in = 2 * m->d.lin_k_heads * m->d.lin_k_dim + 2 * m->d.lin_v_heads * m->d.lin_v_dim;
  for (const auto &L : m->layers)
    if (L.linear && (L.gate_rows > 0) != (L.in_rows == full_in))
      return set_error(m->ctx, Q35_ERR_STATE, "in_proj_all rows do not match the Q8 gate rows");
  m->finalized = true;
  return Q35_OK;
}

// =================================================================== runtime
namespace {

struct MetaLayout {
  // per row
  size_t slots, positions, tokens, seq_lens, count_input, row_seg;
  // per segment: first row, rows, page-table row; segments longest first
  size_t seg_row0, seg_count, page_table, seg_order;
  // per head row (a segment that wants a token): its row, slot, penalty and
  // sampling settings
  size_t head_rows, head_slots, head_penalties, inv_temperature, top_k;
  // attention query tiles, the rows of one-row segments and those of the
  // other segments
  size_t tile_row0, tile_rows, attn_rows, chunk_rows;
  size_t total;
};

MetaLayout meta_layout(int max_rows, int max_segments, int max_pages) {
  MetaLayout L{};
  size_t o = 0;
  auto take = [&](size_t bytes) { const size_t at = o; o = align256(o + bytes); return at; };
  const size_t R = static_cast<size_t>(max_rows), M = static_cast<size_t>(max_segments);
  L.slots = take(R * 4);
  L.positions = take(R * 4);
  L.tokens = take(R * 4);
  L.seq_lens = take(R * 4);
  L.count_input = take(R);
  L.row_seg = take(R * 4);
  L.seg_row0 = take(M * 4);
  L.seg_count = take(M * 4);
  L.page_table = take(M * static_cast<size_t>(max_pages) * 4);
  L.seg_order = take(M * 4);
  L.head_rows = take(M * 4);
  L.head_slots = take(M * 4);
  L.head_penalties = take(M * 4);
  L.inv_temperature = take(M * 4);
  L.top_k = take(M * 4);
  L.tile_row0 = take(R * 4);
  L.tile_rows = take(R * 4);
  L.attn_rows = take(R * 4);
  L.chunk_rows = take(R * 4);
  L.total = o;
  return L;
}

MetaLayout meta_layout(const q35_runtime *rt) { return meta_layout(rt->max_rows, rt->max_segments, rt->max_pages_per_row); }

}  // namespace

extern "C" int q35_runtime_create(q35_model *m, const q35_runtime_config *cfg, q35_runtime **out) {
  if (m == nullptr || cfg == nullptr || out == nullptr) return Q35_ERR_INVALID;
  *out = nullptr;
  if (!m->finalized) return set_error(m->ctx, Q35_ERR_STATE, "model not finalized");
  const q35_model_dims &d = m->d;
  if (cfg->max_slots <= 0 || cfg->max_batch <= 0 || cfg->max_batch > kMaxTokens ||
      cfg->max_context <= 0 || cfg->page_tokens < 1 || (cfg->page_tokens & (cfg->page_tokens - 1)) ||
      cfg->max_step_rows < 0 || cfg->max_step_rows > kMaxStepRows)
    return set_error(m->ctx, Q35_ERR_INVALID, "invalid runtime config");
  auto *rt = new (std::nothrow) q35_runtime();
  if (rt == nullptr) return Q35_ERR_OOM;
  rt->model = m;
  rt->ctx = m->ctx;
  rt->cfg = *cfg;
  rt->max_pages_per_row = (cfg->max_context + cfg->page_tokens - 1) / cfg->page_tokens;
  rt->max_splits = (cfg->max_context + rt->split_tokens - 1) / rt->split_tokens;
  if (rt->cfg.total_pages <= 0) rt->cfg.total_pages = cfg->max_slots * rt->max_pages_per_row;
  rt->max_rows = std::max(cfg->max_batch, cfg->max_step_rows);
  rt->max_segments = cfg->max_batch + kMaxPrefillSegments;
  Context *ctx = m->ctx;
  // R rows of a packed step, M segments (and head rows)
  const int R = rt->max_rows, M = rt->max_segments;
  const size_t H = d.hidden, I = d.intermediate;
  const size_t v_dim = static_cast<size_t>(d.lin_v_heads) * d.lin_v_dim;
  const size_t q_dim = static_cast<size_t>(d.lin_k_heads) * d.lin_k_dim;
  const size_t ch = 2 * q_dim + v_dim;
  const size_t kvw = static_cast<size_t>(d.n_kv_heads) * d.head_dim;
  size_t in_max = 0;
  for (const auto &L : m->layers) in_max = std::max(in_max, static_cast<size_t>(L.in_rows));
  rt->proj_width = std::max(in_max, 2 * I);
  rt->core_width = std::max({v_dim, static_cast<size_t>(d.n_heads) * d.head_dim, I, H});
  int st = Q35_OK;
  auto alloc = [&](size_t bytes, void **p) {
    if (st == Q35_OK) st = rt_alloc(rt, bytes, p);
  };
  // slot state
  // two copies of every slot's recurrent state: the step at position p reads
  // copy p & 1 and writes the other one (see DeltaArgs::state_copy_stride)
  rt->rec_copy_stride = static_cast<long long>(m->n_linear) * d.lin_v_heads * d.lin_v_dim * d.lin_k_dim;
  rt->rec_slot_stride = 2 * rt->rec_copy_stride;
  // conv ring of lin_kernel slots per layer, slot = position % lin_kernel
  rt->conv_slot_stride = static_cast<long long>(m->n_linear) * d.lin_kernel * ch;
  alloc(static_cast<size_t>(cfg->max_slots) * rt->rec_slot_stride * 4, reinterpret_cast<void **>(&rt->recurrent));
  alloc(static_cast<size_t>(cfg->max_slots) * rt->conv_slot_stride * 4, reinterpret_cast<void **>(&rt->conv));
  alloc(static_cast<size_t>(cfg->max_slots) * d.vocab * 4, reinterpret_cast<void **>(&rt->counts));
  // KV pool
  rt->layer_pool_elems = static_cast<size_t>(rt->cfg.total_pages) * cfg->page_tokens * kvw;
  alloc(std::max<size_t>(1, m->n_full) * rt->layer_pool_elems * 2, reinterpret_cast<void **>(&rt->k_pool));
  alloc(std::max<size_t>(1, m->n_full) * rt->layer_pool_elems * 2, reinterpret_cast<void **>(&rt->v_pool));
  // RoPE tables, computed like CpuEngine::Impl::initialize (cpu_engine.inl:343-355)
  const size_t half = d.rope_dim / 2;
  alloc(static_cast<size_t>(cfg->max_context) * half * 4, reinterpret_cast<void **>(&rt->rope_cos));
  alloc(static_cast<size_t>(cfg->max_context) * half * 4, reinterpret_cast<void **>(&rt->rope_sin));
  // work buffers
  alloc(static_cast<size_t>(R) * H * 4, reinterpret_cast<void **>(&rt->x[0]));
  alloc(static_cast<size_t>(R) * H * 4, reinterpret_cast<void **>(&rt->x[1]));
  // group sums of squares of the residual rows (fused decode projections: 16 rows)
  alloc(static_cast<size_t>(16) * (H / 16) * 4, reinterpret_cast<void **>(&rt->sq_groups));
  // GEMM outputs: [split][rows][width] for the largest split plan of any
  // projection at any row count a step can have (split launches), and
  // [rows][width] for the dense GEMM
  size_t proj_floats = static_cast<size_t>(R) * rt->proj_width;
  for (const auto &L : m->layers) {
    proj_floats = std::max(proj_floats, gemm_partial_floats(L.in_rows, d.hidden / 32, R, ctx->cu_count));
    proj_floats = std::max(proj_floats, gemm_partial_floats(d.hidden, L.out_cols / 32, R, ctx->cu_count));
    proj_floats = std::max(proj_floats, gemm_partial_floats(2 * d.intermediate, d.hidden / 32, R, ctx->cu_count));
    proj_floats = std::max(proj_floats, gemm_partial_floats(d.hidden, d.intermediate / 32, R, ctx->cu_count));
  }
  alloc(proj_floats * 4, reinterpret_cast<void **>(&rt->proj));
  // chunked steps of split GEMMs: the in projection's split partials summed
  // once, [rows][width]
  alloc(static_cast<size_t>(R) * rt->proj_width * 4, reinterpret_cast<void **>(&rt->rows_final));
  alloc(static_cast<size_t>(R) * kMaxGateRows * 4, reinterpret_cast<void **>(&rt->q8_gates));
  if (d.lin_v_heads > 0)
    alloc(delta_chunk_scan_floats(R, d.lin_v_heads) * 4, reinterpret_cast<void **>(&rt->delta_scan));
  // sampling: per-head-row candidate lists and the slices' survivors
  alloc(sample_scratch_bytes(M), reinterpret_cast<void **>(&rt->sample_scratch));
  alloc(static_cast<size_t>(M) * kMaxCandidates * sizeof(q35_candidate), reinterpret_cast<void **>(&rt->candidates));
  alloc(static_cast<size_t>(R) * d.n_heads * d.head_dim * 4, reinterpret_cast<void **>(&rt->q_rot));
  alloc(static_cast<size_t>(R) * d.n_heads * d.head_dim * 4, reinterpret_cast<void **>(&rt->gates));
  // attention partials: every chunk of the decode kernel's rows (one-row
  // segments, at most M per step), and one merged partial per prompt row
  const size_t parts = static_cast<size_t>(M) * d.n_heads * rt->max_splits;
  alloc(parts * d.head_dim * 4, reinterpret_cast<void **>(&rt->part_o));
  alloc(parts * 2 * 4, reinterpret_cast<void **>(&rt->part_ml));
  const size_t prompt_parts = static_cast<size_t>(R) * d.n_heads;
  alloc(prompt_parts * d.head_dim * 4, reinterpret_cast<void **>(&rt->prompt_o));
  alloc(prompt_parts * 2 * 4, reinterpret_cast<void **>(&rt->prompt_ml));
  alloc(static_cast<size_t>(M) * H * 4, reinterpret_cast<void **>(&rt->hidden_out));
  const size_t kmax = std::max({H, I, rt->core_width});
  const size_t tiles = (static_cast<size_t>(R) + 15) / 16;
  alloc(tiles * 64 * (kmax / 32) * 8, reinterpret_cast<void **>(&rt->codes));
  alloc(tiles * 16 * (kmax / 32) * sizeof(float), reinterpret_cast<void **>(&rt->scales));
  rt->cand_rows = gemm_argmax_cand_capacity(d.vocab, ctx->cu_count);
  alloc(static_cast<size_t>(rt->cand_rows) * kMaxTokens * 8, reinterpret_cast<void **>(&rt->cand));
  const MetaLayout ml = meta_layout(rt);
  rt->meta_bytes = ml.total;
  alloc(ml.total, reinterpret_cast<void **>(&rt->meta_dev));
  if (st == Q35_OK && hipHostMalloc(reinterpret_cast<void **>(&rt->meta_host), ml.total) != hipSuccess)
    st = set_error(ctx, Q35_ERR_OOM, "pinned metadata");
  // the greedy tokens are stored by the argmax kernel straight into pinned
  // host memory (no copy node at the end of the step)
  if (st == Q35_OK && hipHostMalloc(reinterpret_cast<void **>(&rt->tokens_out_host), static_cast<size_t>(M) * 4) != hipSuccess)
    st = set_error(ctx, Q35_ERR_OOM, "pinned output");
  if (st == Q35_OK &&
      hipHostGetDevicePointer(reinterpret_cast<void **>(&rt->tokens_out_dev), rt->tokens_out_host, 0) != hipSuccess)
    st = set_error(ctx, Q35_ERR_HIP, "device address of the pinned output");
  if (st == Q35_OK) {
    std::vector<float> inv(half), cs(static_cast<size_t>(cfg->max_context) * half), sn(cs.size());
    for (size_t i = 0; i < half; ++i)
      inv[i] = std::pow(d.rope_theta, -static_cast<float>(2 * i) / static_cast<float>(d.rope_dim));
    for (size_t p = 0; p < static_cast<size_t>(cfg->max_context); ++p)
      for (size_t i = 0; i < half; ++i) {
        const float angle = static_cast<float>(p) * inv[i];
        cs[p * half + i] = std::cos(angle);
        sn[p * half + i] = std::sin(angle);
      }
    if (hipMemcpy(rt->rope_cos, cs.data(), cs.size() * 4, hipMemcpyHostToDevice) != hipSuccess ||
        hipMemcpy(rt->rope_sin, sn.data(), sn.size() * 4, hipMemcpyHostToDevice) != hipSuccess ||
        hipMemset(rt->k_pool, 0, std::max<size_t>(1, m->n_full) * rt->layer_pool_elems * 2) != hipSuccess ||
        hipMemset(rt->v_pool, 0, std::max<size_t>(1, m->n_full) * rt->layer_pool_elems * 2) != hipSuccess)
      st = set_error(ctx, Q35_ERR_HIP, "runtime initialisation copies");
  }
  if (st != Q35_OK) {
    q35_runtime_destroy(rt);
    return st;
  }
  rt->slot_used.assign(cfg->max_slots, 0);
  rt->page_ref.assign(rt->cfg.total_pages, 0);
  rt->free_pages.reserve(rt->cfg.total_pages);
  for (int p = rt->cfg.total_pages - 1; p >= 0; --p) rt->free_pages.push_back(p);
  *out = rt;
  return Q35_OK;
}

extern "C" void q35_runtime_destroy(q35_runtime *rt) {
  if (rt == nullptr) return;
  (void)hipSetDevice(rt->ctx->device);
  (void)hipStreamSynchronize(rt->ctx->stream);
  for (auto &kv : rt->graphs) (void)hipGraphExecDestroy(kv.second);
  for (auto &ev : rt->prof_events) (void)hipEventDestroy(ev.first), (void)hipEventDestroy(ev.second);
  for (hipEvent_t ev : rt->step_events)
    if (ev != nullptr) (void)hipEventDestroy(ev);
  for (void *p : rt->allocations) (void)hipFree(p);
  for (auto &kv : rt->trace) (void)hipFree(kv.second.first);
  if (rt->meta_host) (void)hipHostFree(rt->meta_host);
  if (rt->tokens_out_host) (void)hipHostFree(rt->tokens_out_host);
  delete rt;
}

extern "C" int q35_slot_alloc(q35_runtime *rt, const int32_t *prompt, size_t n, int32_t *out_slot) {
  if (rt == nullptr || out_slot == nullptr || (n && prompt == nullptr)) return Q35_ERR_INVALID;
  const q35_model_dims &d = rt->model->d;
  int slot = -1;
  for (int s = 0; s < rt->cfg.max_slots; ++s)
    if (!rt->slot_used[s]) { slot = s; break; }
  if (slot < 0) return set_error(rt->ctx, Q35_ERR_STATE, "no free request slot");
  for (size_t i = 0; i < n; ++i)
    if (prompt[i] < 0 || prompt[i] >= d.vocab) return set_error(rt->ctx, Q35_ERR_INVALID, "prompt token out of range");
  Context *ctx = rt->ctx;
  Q35_HIP_TRY(ctx, hipMemsetAsync(rt->recurrent + slot * rt->rec_slot_stride, 0, rt->rec_slot_stride * 4, ctx->stream));
  Q35_HIP_TRY(ctx, hipMemsetAsync(rt->conv + slot * rt->conv_slot_stride, 0, rt->conv_slot_stride * 4, ctx->stream));
  // prompt token counts (cpu_engine.inl:376-378)
  std::vector<int32_t> counts(d.vocab, 0);
  for (size_t i = 0; i < n; ++i) ++counts[prompt[i]];
  Q35_HIP_TRY(ctx, hipMemcpyAsync(rt->counts + static_cast<size_t>(slot) * d.vocab, counts.data(),
                                  counts.size() * 4, hipMemcpyHostToDevice, ctx->stream));
  Q35_HIP_TRY(ctx, hipStreamSynchronize(ctx->stream));
  rt->slot_used[slot] = 1;
  *out_slot = slot;
  return Q35_OK;
}

extern "C" int q35_slot_free(q35_runtime *rt, int32_t slot) {
  if (rt == nullptr || slot < 0 || slot >= rt->cfg.max_slots || !rt->slot_used[slot]) return Q35_ERR_STATE;
  rt->slot_used[slot] = 0;
  return Q35_OK;
}

extern "C" int q35_page_alloc(q35_runtime *rt, int32_t *out) {
  if (rt == nullptr || out == nullptr) return Q35_ERR_INVALID;
  if (rt->free_pages.empty()) return set_error(rt->ctx, Q35_ERR_OOM, "KV page pool exhausted");
  const int p = rt->free_pages.back();
  rt->free_pages.pop_back();
  rt->page_ref[p] = 1;
  *out = p;
  return Q35_OK;
}
extern "C" int q35_page_retain(q35_runtime *rt, int32_t p) {
  if (rt == nullptr || p < 0 || p >= rt->cfg.total_pages || rt->page_ref[p] <= 0) return Q35_ERR_STATE;
  ++rt->page_ref[p];
  return Q35_OK;
}
extern "C" int q35_page_release(q35_runtime *rt, int32_t p) {
  if (rt == nullptr || p < 0 || p >= rt->cfg.total_pages || rt->page_ref[p] <= 0) return Q35_ERR_STATE;
  if (--rt->page_ref[p] == 0) rt->free_pages.push_back(p);
  return Q35_OK;
}
extern "C" int q35_page_refcount(q35_runtime *rt, int32_t p) {
  if (rt == nullptr || p < 0 || p >= rt->cfg.total_pages) return -1;
  return rt->page_ref[p];
}
extern "C" int q35_runtime_free_pages(q35_runtime *rt) {
  return rt ? static_cast<int>(rt->free_pages.size()) : -1;
}
// Copy-on-write: the first `tokens` rows of src into dst, every full layer
// (KvPagesF16::append on a shared tail page, kv_pages.h:52-60).
extern "C" int q35_page_copy(q35_runtime *rt, int32_t src, int32_t dst, int32_t tokens) {
  if (rt == nullptr || src < 0 || dst < 0 || src >= rt->cfg.total_pages || dst >= rt->cfg.total_pages ||
      tokens < 0 || tokens > rt->cfg.page_tokens)
    return Q35_ERR_INVALID;
  const size_t kvw = static_cast<size_t>(rt->model->d.n_kv_heads) * rt->model->d.head_dim;
  const size_t page_elems = static_cast<size_t>(rt->cfg.page_tokens) * kvw;
  const size_t bytes = static_cast<size_t>(tokens) * kvw * 2;
  for (int l = 0; l < rt->model->n_full; ++l) {
    const size_t base = l * rt->layer_pool_elems;
    Q35_HIP_TRY(rt->ctx, hipMemcpyAsync(rt->k_pool + base + dst * page_elems, rt->k_pool + base + src * page_elems,
                                        bytes, hipMemcpyDeviceToDevice, rt->ctx->stream));
    Q35_HIP_TRY(rt->ctx, hipMemcpyAsync(rt->v_pool + base + dst * page_elems, rt->v_pool + base + src * page_elems,
                                        bytes, hipMemcpyDeviceToDevice, rt->ctx->stream));
  }
  return Q35_OK;
}

namespace q35 {

double gemm_algorithmic_bytes(int rows, int nb, int tokens, bool stores, bool residual) {
  const double weights = static_cast<double>(rows / 8) * nb * sizeof(q35_q4_0_block_x8);
  const double acts = static_cast<double>(tokens) * (nb * 32.0 + sizeof(float));
  const double outs = static_cast<double>(tokens) * rows * 4.0 * ((stores ? 1 : 0) + (residual ? 1 : 0));
  return weights + acts + outs;
}

namespace {

// The logical launch being enqueued under profiling: its class and bytes go to
// the first kernel it dispatches, every kernel gets its own event pair.
struct ProfScope {
  q35_runtime *rt;
  int cls;
  double bytes;
  bool first;
};
thread_local ProfScope *t_prof = nullptr;

// After the step's stream synchronisation: fold the bracketed kernels into the
// per-class totals (durations of every kernel, one launch per logical launch).
int profile_collect(q35_runtime *rt) {
  for (size_t i = 0; i < rt->prof_pending.size(); ++i) {
    float ms = 0;
    Q35_HIP_TRY(rt->ctx, hipEventElapsedTime(&ms, rt->prof_events[i].first, rt->prof_events[i].second));
    const auto &p = rt->prof_pending[i];
    rt->prof_ms[p.cls] += ms;
    rt->prof_bytes[p.cls] += p.bytes;
    rt->prof_launches[p.cls] += p.counted ? 1 : 0;
  }
  rt->prof_pending.clear();
  return Q35_OK;
}

}  // namespace

bool launch_events(hipEvent_t *start, hipEvent_t *stop) {
  ProfScope *p = t_prof;
  if (p == nullptr) return false;
  q35_runtime *rt = p->rt;
  const size_t i = rt->prof_pending.size();
  if (i == rt->prof_events.size()) {
    hipEvent_t a = nullptr, b = nullptr;
    if (hipEventCreate(&a) != hipSuccess) return false;
    if (hipEventCreate(&b) != hipSuccess) {
      (void)hipEventDestroy(a);
      return false;
    }
    rt->prof_events.emplace_back(a, b);
  }
  rt->prof_pending.push_back({p->cls, p->first ? p->bytes : 0.0, p->first});
  p->first = false;
  *start = rt->prof_events[i].first;
  *stop = rt->prof_events[i].second;
  return true;
}

// Enqueues one decode step for `batch` rows whose metadata is already in
// rt->meta_host; the host copy is part of the enqueued work so the whole
// sequence can be captured as a graph.
// The greedy head over `tokens` rows of A16 activations in rt->codes/scales:
// penalty counts of slot count_rows[t], penalty penalties[t] (device arrays).
static GemmArgs greedy_head_args(q35_runtime *rt, int tokens, const int32_t *count_rows, const float *penalties) {
  const q35_model_dims &d = rt->model->d;
  GemmArgs g;
  g.w = rt->model->embed;
  g.g16 = rt->model->embed_g16;
  g.rows = d.vocab;
  g.nb = d.hidden / 32;
  g.codes = rt->codes;
  g.scales = rt->scales;
  g.tokens = tokens;
  g.cand = rt->cand;
  g.cand_stride = kMaxTokens;
  g.counts = rt->counts;
  g.count_rows = count_rows;
  g.counts_stride = d.vocab;
  g.penalties = penalties;
  g.cu_count = rt->ctx->cu_count;
  return g;
}

// Stage trace: the device copy of (layer, point), grown to `bytes`.
static hipError_t trace_slot(q35_runtime *rt, int layer, int point, size_t bytes, void **out) {
  auto &e = rt->trace[std::make_pair(layer, point)];
  if (e.first == nullptr || e.second < bytes) {
    if (e.first != nullptr) (void)hipFree(e.first);
    e.first = nullptr;
    const hipError_t err = hipMalloc(&e.first, bytes ? bytes : 1);
    if (err != hipSuccess) return err;
  }
  e.second = bytes;
  *out = e.first;
  return hipSuccess;
}

static hipError_t trace_copy(q35_runtime *rt, int layer, int point, const void *src, size_t bytes, hipStream_t s) {
  void *dst = nullptr;
  hipError_t e = trace_slot(rt, layer, point, bytes, &dst);
  if (e == hipSuccess) e = hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, s);
  return e;
}

int runtime_enqueue_step(q35_runtime *rt, const StepShape &sh, bool want_logits) {
  q35_model *m = rt->model;
  Context *ctx = rt->ctx;
  const q35_model_dims &d = m->d;
  hipStream_t s = ctx->stream;
  const int batch = sh.rows;
  // segments of several positions: the DeltaNet chunk scan and the tiled
  // attention (a decode-only step runs the per-row kernels)
  const bool chunked = !sh.single;
  const MetaLayout ml = meta_layout(rt);
  auto *mdev = rt->meta_dev;
  const auto *slots = reinterpret_cast<const int32_t *>(mdev + ml.slots);
  const auto *positions = reinterpret_cast<const int32_t *>(mdev + ml.positions);
  const auto *tokens = reinterpret_cast<const int32_t *>(mdev + ml.tokens);
  const auto *seq_lens = reinterpret_cast<const int32_t *>(mdev + ml.seq_lens);
  const auto *count_input = reinterpret_cast<const uint8_t *>(mdev + ml.count_input);
  const auto *row_seg = reinterpret_cast<const int32_t *>(mdev + ml.row_seg);
  const auto *seg_row0 = reinterpret_cast<const int32_t *>(mdev + ml.seg_row0);
  const auto *seg_count = reinterpret_cast<const int32_t *>(mdev + ml.seg_count);
  const auto *seg_order = reinterpret_cast<const int32_t *>(mdev + ml.seg_order);
  const auto *page_table = reinterpret_cast<const int32_t *>(mdev + ml.page_table);
  const auto *head_rows = reinterpret_cast<const int32_t *>(mdev + ml.head_rows);
  const auto *head_slots = reinterpret_cast<const int32_t *>(mdev + ml.head_slots);
  const auto *head_penalties = reinterpret_cast<const float *>(mdev + ml.head_penalties);
  const auto *tile_row0 = reinterpret_cast<const int32_t *>(mdev + ml.tile_row0);
  const auto *attn_rows = reinterpret_cast<const int32_t *>(mdev + ml.attn_rows);
  const auto *chunk_rows = reinterpret_cast<const int32_t *>(mdev + ml.chunk_rows);
  const auto *tile_rows = reinterpret_cast<const int32_t *>(mdev + ml.tile_rows);
  const int H = d.hidden, I = d.intermediate;
  const int v_dim = d.lin_v_heads * d.lin_v_dim;
  const int q_dim = d.lin_k_heads * d.lin_k_dim;
  const int ch = 2 * q_dim + v_dim;
  const size_t kvw = static_cast<size_t>(d.n_kv_heads) * d.head_dim;
  const size_t page_elems = static_cast<size_t>(rt->cfg.page_tokens) * kvw;
  (void)page_elems;
  hipError_t e;
#define Q35_STEP(expr, what)                               \
  do {                                                     \
    e = (expr);                                            \
    if (e != hipSuccess) return hip_error(ctx, e, what);   \
  } while (0)
  // A logical launch (one or more kernels); with profiling on each kernel
  // records its own start and end events and the launch is counted under
  // `cls` with `bytes` algorithmic HBM bytes.
#define Q35_KERNEL(cls, bytes, expr, what)                                     \
  do {                                                                         \
    ProfScope q35_scope_{rt, (cls), (bytes), true};                            \
    if (rt->profiling) t_prof = &q35_scope_;                                   \
    e = (expr);                                                                \
    t_prof = nullptr;                                                          \
    if (e != hipSuccess) return hip_error(ctx, e, what);                       \
  } while (0)
  const double B = batch;
  const auto *host_seq = reinterpret_cast<const int32_t *>(rt->meta_host + ml.seq_lens);
  double kv_tokens = 0;
  for (int b = 0; b < batch; ++b) kv_tokens += host_seq[b];
  // activation prep: FP32 rows in (x_cols wide), A16 codes + scales out

  Q35_STEP(hipMemcpyAsync(rt->meta_dev, rt->meta_host, rt->meta_bytes, hipMemcpyHostToDevice, s), "metadata copy");
  // a G16 head tile is 160 bytes per 8 x 32 (20 per row block) against 144 (18)
  const double g16_extra = m->embed_g16 ? static_cast<double>(d.vocab / 8) * (H / 32) * 16.0 : 0.0;
  // the embedding gather runs inside the first layer's input norm (its rows
  // land in x[0]); a model without layers gathers them on their own
  const bool embed_in_norm = d.n_layers > 0;
  const double embed_bytes = B * (H / 32 * (m->embed_g16 ? 20.0 : 18.0) + H * 4.0 + 8.0);
  if (!embed_in_norm)
    Q35_KERNEL(Q35_KERNEL_EMBED, embed_bytes,
               launch_embed(m->embed, H / 32, tokens, batch, rt->x[0], H, rt->counts, d.vocab, slots, count_input, s,
                            m->embed_g16),
               "embedding");

  // Residual stream: x[cur] holds it; a residual update writes x[cur ^ 1]
  // (the prep kernels read whole rows, so the update cannot run in place).
  int cur = 0;
  // GEMM outputs land in rt->proj as [split][batch][rows]; `pending` describes
  // the last one for its consumer.
  SplitRows pending;
  // Consumers that sum at most kConsumerSplits partials (DeltaNet, the
  // attention prep, the SiLU prep) get GEMMs split at most that many ways.
  constexpr int kConsumerSplits = 8;
  auto gemm = [&](const q35_q4_0_block_x8 *w, int rows, int K, int max_split = 32) -> hipError_t {
    if (gemm_dense_fits(rows, batch, ctx->cu_count)) {
      // the dense GEMM: finished rows with the split launch's bits
      GemmArgs g;
      g.w = w;
      g.rows = rows;
      g.nb = K / 32;
      g.codes = rt->codes;
      g.scales = rt->scales;
      g.tokens = batch;
      g.out = rt->proj;
      g.stride = rows;
      g.cu_count = ctx->cu_count;
      g.max_split = max_split;
      pending.p = rt->proj;
      pending.splits = 1;
      pending.split_stride = 0;
      pending.width = rows;
      return launch_gemm_dense(g, s);
    }
    const GemmPlan p = gemm_plan(rows, K / 32, false, false, ctx->cu_count, 0, 0, max_split);
    GemmArgs g;
    g.w = w;
    g.rows = rows;
    g.nb = K / 32;
    g.codes = rt->codes;
    g.scales = rt->scales;
    g.tokens = batch;
    g.out = rt->proj;
    g.stride = rows;
    g.partials = rt->proj;
    g.cu_count = ctx->cu_count;
    g.max_split = max_split;
    pending.p = rt->proj;
    pending.splits = p.split;
    pending.split_stride = static_cast<long long>(batch) * rows;
    pending.width = rows;
    return launch_gemm(g, s);
  };
  // Residual update with the pending split rows (if `add`) + RMSNorm + prep.
  bool groups_ready = false;  // rt->sq_groups holds the sums of squares of x[cur] (set by gemm_resid)
  auto rms_prep = [&](const float *w, bool add, bool h128, float *normed, const LayerDev *gate_layer = nullptr,
                      bool embed_rows = false) -> hipError_t {
    RmsPrepArgs a;
    if (embed_rows) {  // the rows are the tokens' embeddings, kept in x[cur]
      a.embed = m->embed;
      a.embed_g16 = m->embed_g16;
      a.token_ids = tokens;
      a.counts = rt->counts;
      a.counts_stride = d.vocab;
      a.slots = slots;
      a.count_input = count_input;
      a.x_out = rt->x[cur];
    }
    if (gate_layer != nullptr && gate_layer->gate_rows > 0) {
      a.gate_codes = gate_layer->gate_codes;
      a.gate_scales = gate_layer->gate_scales;
      a.gate_rows = gate_layer->gate_rows;
      a.gates = rt->q8_gates;
    }
    a.x_in = rt->x[cur];
    if (add) {
      a.add = pending;
      a.x_out = rt->x[cur ^ 1];
    }
    a.weight = w;
    a.eps = d.rms_eps;
    a.tokens = batch;
    a.K = H;
    a.h128 = h128;
    a.seed = d.sign_seed;
    a.codes = rt->codes;
    a.scales = rt->scales;
    a.normed_out = normed;
    const hipError_t e = launch_rms_prep(a, s);
    if (add) {
      cur ^= 1;
      groups_ready = false;
    }
    return e;
  };
  // Algorithmic bytes count each projection output row once (a split
  // GEMM's partial rows are traffic, not algorithm: the measured HBM bytes
  // show them). rms_prep: residual row in (+ the projection row and the new
  // residual out), codes and scales out.
  auto rms_bytes = [&](bool add) {
    return B * (H * 4.0 + (add ? H * 4.0 + H * 4.0 : 0.0) + H + H / 32.0 * 4.0) + H * 4.0;
  };
  // Steps of one token tile fold the residual + RMSNorm preparations into
  // the projections (fused.hip): the in / qkv and gate_up projections
  // normalize and prepare complete residual rows in their prologue, and the
  // out / o and down projections finish their rows with the residual added.
  // Same bits as the split launches and rms_prep (q35_runtime_set_fused).
  const bool fuse = rt->fuse_decode && batch <= 16;
  constexpr bool fuse_down = false;
  auto gemm_norm = [&](const q35_q4_0_block_x8 *w, int rows, const float *norm_w, int max_split,
                       float *normed) -> hipError_t {
    NormGemmArgs a;
    a.g.w = w;
    a.g.rows = rows;
    a.g.nb = H / 32;
    a.g.tokens = batch;
    a.g.out = rt->proj;
    a.g.stride = rows;
    a.g.partials = rt->proj;
    a.g.cu_count = ctx->cu_count;
    a.max_split = max_split;
    a.x = rt->x[cur];
    a.sq_groups = rt->sq_groups;
    a.weight = norm_w;
    a.eps = d.rms_eps;
    a.seed = d.sign_seed;
    a.normed_out = normed;
    if (normed != nullptr) {  // the stage trace copies the prepared activations
      a.codes_out = rt->codes;
      a.scales_out = rt->scales;
    }
    return launch_gemm_norm(a, &pending, s);
  };
  auto gemm_resid = [&](const q35_q4_0_block_x8 *w, int K, float *proj_out) -> hipError_t {
    ResidGemmArgs a;
    a.g.w = w;
    a.g.rows = H;
    a.g.nb = K / 32;
    a.g.codes = rt->codes;
    a.g.scales = rt->scales;
    a.g.tokens = batch;
    a.g.cu_count = ctx->cu_count;
    a.residual = rt->x[cur];
    a.x_out = rt->x[cur ^ 1];
    a.proj_out = proj_out;
    a.sq_groups = rt->sq_groups;
    const hipError_t e = launch_gemm_resid(a, s);
    cur ^= 1;
    groups_ready = true;
    return e;
  };
  // weights, residual rows, group sums and the norm weight in (no A16
  // activations read), one output row out
  auto norm_bytes = [&](int rows) {
    return gemm_algorithmic_bytes(rows, H / 32, batch, true, false) + B * H * 4.0 + H * 4.0 + B * (H / 16) * 4.0 -
           B * (H + 4.0);
  };
  // weights, A16 activations in, one output row out
  auto gemm_bytes = [&](int rows, int K) { return gemm_algorithmic_bytes(rows, K / 32, batch, true, false); };

  // Stage trace (test hook, decode steps only): copies of the stage inputs
  // and outputs; the split GEMM outputs are summed in split order into the
  // copy, exactly as their consumer sums them.
  const bool tracing = rt->tracing && sh.single && sh.heads_identity;
  const auto *host_slots = reinterpret_cast<const int32_t *>(rt->meta_host + ml.slots);
  const auto *host_pos = reinterpret_cast<const int32_t *>(rt->meta_host + ml.positions);
  const size_t code_tiles = (batch + 15) / 16;
  auto trace_codes = [&](int layer, int point_codes, int K) -> hipError_t {
    hipError_t te = trace_copy(rt, layer, point_codes, rt->codes, code_tiles * (K / 32) * 64 * 8, s);
    if (te == hipSuccess) te = trace_copy(rt, layer, point_codes + 1, rt->scales, code_tiles * (K / 32) * 16 * 4, s);
    return te;
  };
  auto trace_rows = [&](int layer, int point, int width) -> hipError_t {
    void *dst = nullptr;
    hipError_t te = trace_slot(rt, layer, point, static_cast<size_t>(batch) * width * 4, &dst);
    if (te == hipSuccess) te = launch_split_reduce(pending, batch, static_cast<float *>(dst), width, nullptr, s);
    return te;
  };
  auto trace_fp32 = [&](int layer, int point, int width) -> float * {
    void *dst = nullptr;
    return trace_slot(rt, layer, point, static_cast<size_t>(batch) * width * 4, &dst) == hipSuccess
               ? static_cast<float *>(dst) : nullptr;
  };
  // per-row copies of a linear layer's recurrent state (copy `which` of the
  // position: 0 = read, 1 = written) and conv ring
  auto trace_state = [&](int l, int li, int point, int which) -> hipError_t {
    const size_t head_floats = static_cast<size_t>(d.lin_v_heads) * d.lin_v_dim * d.lin_k_dim;
    void *dst = nullptr;
    hipError_t te = trace_slot(rt, l, point, batch * head_floats * 4, &dst);
    for (int b = 0; te == hipSuccess && b < batch; ++b) {
      const int copy = (host_pos[b] & 1) ^ which;
      const float *src = rt->recurrent + host_slots[b] * rt->rec_slot_stride + copy * rt->rec_copy_stride +
                         static_cast<size_t>(li) * head_floats;
      te = hipMemcpyAsync(static_cast<float *>(dst) + b * head_floats, src, head_floats * 4, hipMemcpyDeviceToDevice, s);
    }
    return te;
  };
  auto trace_conv = [&](int l, int li, int point) -> hipError_t {
    const size_t ring = static_cast<size_t>(d.lin_kernel) * ch;
    void *dst = nullptr;
    hipError_t te = trace_slot(rt, l, point, batch * ring * 4, &dst);
    for (int b = 0; te == hipSuccess && b < batch; ++b) {
      const float *src = rt->conv + host_slots[b] * rt->conv_slot_stride + static_cast<size_t>(li) * ring;
      te = hipMemcpyAsync(static_cast<float *>(dst) + b * ring, src, ring * 4, hipMemcpyDeviceToDevice, s);
    }
    return te;
  };

  bool add_pending = false;  // the previous layer's down projection is still split
  for (int l = 0; l < d.n_layers; ++l) {
    const LayerDev &L = m->layers[l];
    float *normed_in = tracing ? trace_fp32(l, Q35_TRACE_NORMED_IN, H) : nullptr;
    const bool fuse_in = fuse && groups_ready && !add_pending && L.gate_rows == 0 &&
                         gemm_norm_fits(L.in_rows, H / 32, batch, ctx->cu_count, kConsumerSplits);
    if (fuse_in) {
      Q35_KERNEL(Q35_KERNEL_GEMM, norm_bytes(L.in_rows),
                 gemm_norm(L.in_proj, L.in_rows, L.input_norm, kConsumerSplits, normed_in), "norm + in projection");
    } else {
      const bool embed_rows = embed_in_norm && l == 0;
      Q35_KERNEL(Q35_KERNEL_PREP, rms_bytes(add_pending) + (embed_rows ? embed_bytes : 0.0),
                 rms_prep(L.input_norm, add_pending, true, normed_in, L.linear ? &L : nullptr, embed_rows),
                 "input norm prep");
    }
    if (tracing) {
      Q35_STEP(trace_copy(rt, l, Q35_TRACE_X_IN, rt->x[cur], static_cast<size_t>(batch) * H * 4, s), "trace");
      Q35_STEP(trace_codes(l, Q35_TRACE_CODES_IN, H), "trace");
      if (L.gate_rows > 0)
        Q35_STEP(trace_copy(rt, l, Q35_TRACE_GATES, rt->q8_gates, static_cast<size_t>(batch) * L.gate_rows * 4, s),
                 "trace");
    }
    if (!fuse_in)
      Q35_KERNEL(Q35_KERNEL_GEMM, gemm_bytes(L.in_rows, H),
                 gemm(L.in_proj, L.in_rows, H, kConsumerSplits), "in projection");
    if (tracing) Q35_STEP(trace_rows(l, Q35_TRACE_PROJ_IN, L.in_rows), "trace");
    if (L.linear) {
      const int li = m->linear_index[l];
      DeltaArgs a;
      a.fused = true;
      a.state_base = rt->recurrent + static_cast<size_t>(li) * d.lin_v_heads * d.lin_v_dim * d.lin_k_dim;
      a.slots = slots;
      a.state_slot_stride = rt->rec_slot_stride;
      a.state_copy_stride = rt->rec_copy_stride;
      a.batch = batch;
      a.k_heads = d.lin_k_heads;
      a.v_heads = d.lin_v_heads;
      a.kd = d.lin_k_dim;
      a.vd = d.lin_v_dim;
      a.out = nullptr;
      a.proj = pending;
      a.gates = L.gate_rows > 0 ? rt->q8_gates : nullptr;
      if (chunked && pending.splits > 1) {
        // the chunk scan reads every token's inputs in order: sum the split
        // partials once over the whole GPU, so each token is one load per channel
        Q35_KERNEL(Q35_KERNEL_PREP, B * L.in_rows * 2 * 4.0,
                   launch_split_reduce(pending, batch, rt->rows_final, L.in_rows, nullptr, s), "prefill row sum");
        a.proj.p = rt->rows_final;
        a.proj.width = L.in_rows;
        a.proj.splits = 1;
        a.proj.split_stride = 0;
      }
      a.conv_base = rt->conv + static_cast<size_t>(li) * d.lin_kernel * ch;
      a.conv_slot_stride = rt->conv_slot_stride;
      a.positions = positions;
      a.conv_w = L.conv_w;
      a.kernel = d.lin_kernel;
      a.dt_bias = L.dt_bias;
      a.ssm_a = L.ssm_a;
      a.norm_w = L.lin_norm;
      a.eps = d.rms_eps;
      a.codes = rt->codes;
      a.scales = rt->scales;
      a.seed = d.sign_seed;
      a.scan = rt->delta_scan;
      if (chunked) {
        a.row_seg = row_seg;
        a.seg_row0 = seg_row0;
        a.seg_count = seg_count;
        a.segments = sh.segments;
        a.seg_order = seg_order;
        a.chunk_rows = chunk_rows;
        a.chunk_row_count = sh.rows - sh.attn_rows;
        a.scan_segments = sh.segments - sh.attn_rows;  // seg_order puts them first
        a.row_list = attn_rows;
        a.row_count = sh.attn_rows;
      }
      // recurrent state read + written, projection row in, conv ring (K-1
      // rows read, one written), prepared out-projection activations
      const double delta_bytes =
          B * (2.0 * d.lin_v_heads * d.lin_v_dim * d.lin_k_dim * 4.0 + L.in_rows * 4.0 +
               static_cast<double>(d.lin_kernel) * ch * 4.0 + v_dim + v_dim / 32.0 * 4.0);
      if (tracing) {
        Q35_STEP(trace_state(l, li, Q35_TRACE_STATE_BEFORE, 0), "trace");
        Q35_STEP(trace_conv(l, li, Q35_TRACE_CONV_BEFORE), "trace");
        a.out = trace_fp32(l, Q35_TRACE_CORE, v_dim);
      }
      Q35_KERNEL(Q35_KERNEL_DELTA, delta_bytes, (chunked ? launch_delta_chunk(a, s) : launch_delta(a, s)), "DeltaNet");
      if (tracing) {
        Q35_STEP(trace_state(l, li, Q35_TRACE_STATE_AFTER, 1), "trace");
        Q35_STEP(trace_conv(l, li, Q35_TRACE_CONV_AFTER), "trace");
        Q35_STEP(trace_codes(l, Q35_TRACE_CODES_CORE, v_dim), "trace");
      }
    } else {
      const int fi = m->full_index[l];
      AttnPrepArgs p;
      p.proj = pending;
      p.batch = batch;
      p.heads = d.n_heads;
      p.kv_heads = d.n_kv_heads;
      p.head_dim = d.head_dim;
      p.rope_dim = d.rope_dim;
      p.q_norm = L.q_norm;
      p.k_norm = L.k_norm;
      p.eps = d.rms_eps;
      p.rope_cos = rt->rope_cos;
      p.rope_sin = rt->rope_sin;
      p.positions = positions;
      p.page_table = page_table;
      p.row_seg = row_seg;
      p.max_pages = rt->max_pages_per_row;
      p.page_tokens = rt->cfg.page_tokens;
      p.k_pool = rt->k_pool + static_cast<size_t>(fi) * rt->layer_pool_elems;
      p.v_pool = rt->v_pool + static_cast<size_t>(fi) * rt->layer_pool_elems;
      p.q_out = rt->q_rot;
      p.gate_out = rt->gates;
      // projection row in; rotated q, gate, and the new K/V rows (FP16) out
      Q35_KERNEL(Q35_KERNEL_ATTN_PREP,
                 B * (L.in_rows * 4.0 + 2.0 * d.n_heads * d.head_dim * 4.0 + 2.0 * kvw * 2.0),
                 launch_attn_prep(p, s), "attention prep");
      if (tracing) {
        const size_t qb = static_cast<size_t>(batch) * d.n_heads * d.head_dim * 4;
        Q35_STEP(trace_copy(rt, l, Q35_TRACE_Q_ROT, rt->q_rot, qb, s), "trace");
        Q35_STEP(trace_copy(rt, l, Q35_TRACE_ATTN_GATE, rt->gates, qb, s), "trace");
        Q35_STEP(trace_copy(rt, l, Q35_TRACE_K_POOL, p.k_pool, rt->layer_pool_elems * 2, s), "trace");
        Q35_STEP(trace_copy(rt, l, Q35_TRACE_V_POOL, p.v_pool, rt->layer_pool_elems * 2, s), "trace");
      }
      AttnArgs a;
      a.q = rt->q_rot;
      a.k_pool = p.k_pool;
      a.v_pool = p.v_pool;
      a.page_table = page_table;
      a.max_pages = rt->max_pages_per_row;
      a.page_tokens = rt->cfg.page_tokens;
      a.seq_lens = seq_lens;
      a.batch = batch;
      a.heads = d.n_heads;
      a.kv_heads = d.n_kv_heads;
      a.head_dim = d.head_dim;
      a.scale = 1.0F / std::sqrt(static_cast<float>(d.head_dim));
      a.split_tokens = rt->split_tokens;
      a.max_splits = rt->max_splits;
      a.grid_splits = sh.grid_splits;
      a.part_o = rt->part_o;
      a.part_ml = rt->part_ml;
      a.prompt_o = rt->prompt_o;
      a.prompt_ml = rt->prompt_ml;
      a.row_seg = row_seg;
      if (chunked) {
        a.tile_row0 = tile_row0;
        a.tile_rows = tile_rows;
        a.tiles = sh.tiles;
        a.row_list = attn_rows;
        a.row_count = sh.attn_rows;
        a.prompt_rows = chunk_rows;
        a.prompt_row_count = sh.rows - sh.attn_rows;
      }
      // every cached K and V row of each request once, q in, one output row
      // out (chunk partials are traffic, as the split GEMMs')
      Q35_KERNEL(Q35_KERNEL_ATTENTION, kv_tokens * kvw * 2.0 * 2.0 + 2.0 * B * d.n_heads * d.head_dim * 4.0,
                 launch_attention(a, s), "attention");
      // the attention row and the gates in, o projection A16 activations out
      Q35_KERNEL(Q35_KERNEL_PREP,
                 B * d.n_heads * d.head_dim * (4.0 + 4.0 + 1.0) + B * d.n_heads * d.head_dim / 32.0 * 4.0,
                 launch_attention_merge(a, rt->gates, tracing ? trace_fp32(l, Q35_TRACE_CORE, d.n_heads * d.head_dim)
                                                              : nullptr,
                                        rt->codes, rt->scales, d.sign_seed, s),
                 "attention merge");
      if (tracing) Q35_STEP(trace_codes(l, Q35_TRACE_CODES_CORE, d.n_heads * d.head_dim), "trace");
    }
    const bool fuse_out = fuse && gemm_resid_fits(H, L.out_cols / 32, batch, ctx->cu_count);
    if (fuse_out) {
      Q35_KERNEL(Q35_KERNEL_GEMM, gemm_algorithmic_bytes(H, L.out_cols / 32, batch, true, true),
                 gemm_resid(L.out_proj, L.out_cols, tracing ? trace_fp32(l, Q35_TRACE_PROJ_OUT, H) : nullptr),
                 "out projection + residual");
    } else {
      Q35_KERNEL(Q35_KERNEL_GEMM, gemm_bytes(H, L.out_cols), gemm(L.out_proj, H, L.out_cols), "out projection");
      if (tracing) Q35_STEP(trace_rows(l, Q35_TRACE_PROJ_OUT, H), "trace");
    }
    float *normed_post = tracing ? trace_fp32(l, Q35_TRACE_NORMED_POST, H) : nullptr;
    const bool fuse_post = fuse_out && gemm_norm_fits(2 * I, H / 32, batch, ctx->cu_count, kConsumerSplits);
    if (fuse_post) {
      Q35_KERNEL(Q35_KERNEL_GEMM, norm_bytes(2 * I),
                 gemm_norm(L.gate_up, 2 * I, L.post_norm, kConsumerSplits, normed_post), "post norm + gate_up projection");
    } else {
      Q35_KERNEL(Q35_KERNEL_PREP, rms_bytes(!fuse_out), rms_prep(L.post_norm, !fuse_out, true, normed_post),
                 "post norm prep");
    }
    if (tracing) {
      Q35_STEP(trace_copy(rt, l, Q35_TRACE_X_MID, rt->x[cur], static_cast<size_t>(batch) * H * 4, s), "trace");
      Q35_STEP(trace_codes(l, Q35_TRACE_CODES_POST, H), "trace");
    }
    if (!fuse_post)
      Q35_KERNEL(Q35_KERNEL_GEMM, gemm_bytes(2 * I, H), gemm(L.gate_up, 2 * I, H, kConsumerSplits),
                 "gate_up projection");
    if (tracing) Q35_STEP(trace_rows(l, Q35_TRACE_GATE_UP, 2 * I), "trace");
    PrepArgs sp;
    sp.source = kPrepSiluMul;
    sp.gate_up = pending;
    sp.tokens = batch;
    sp.K = I;
    sp.h128 = true;
    sp.seed = d.sign_seed;
    sp.codes = rt->codes;
    sp.scales = rt->scales;
    if (tracing) sp.y_out = trace_fp32(l, Q35_TRACE_SILU, I);
    Q35_KERNEL(Q35_KERNEL_PREP, B * (2.0 * I * 4.0 + I + I / 32.0 * 4.0), launch_prep(sp, s),
               "silu prep");
    if (tracing) Q35_STEP(trace_codes(l, Q35_TRACE_CODES_DOWN, I), "trace");
    // the down projection stays split: owning all of its K splits, a
    // 16-row workgroup re-reads every activation code (K x 16 bytes), and the
    // next input norm then runs as rms_prep + the split in projection
    if (fuse && fuse_down && gemm_resid_fits(H, I / 32, batch, ctx->cu_count)) {
      Q35_KERNEL(Q35_KERNEL_GEMM, gemm_algorithmic_bytes(H, I / 32, batch, true, true),
                 gemm_resid(L.down, I, tracing ? trace_fp32(l, Q35_TRACE_DOWN, H) : nullptr),
                 "down projection + residual");
      add_pending = false;
    } else {
      Q35_KERNEL(Q35_KERNEL_GEMM, gemm_bytes(H, I), gemm(L.down, H, I), "down projection");
      if (tracing) Q35_STEP(trace_rows(l, Q35_TRACE_DOWN, H), "trace");
      add_pending = true;
    }
  }
  // Final norm and head on the head rows: every row of a decode step, the
  // last position of each segment that wants a token otherwise (hidden_out
  // and the head outputs are then indexed by head row).
  const int heads = sh.heads;
  {
    RmsPrepArgs a;
    a.x_in = rt->x[cur];
    if (add_pending) {
      a.add = pending;
      a.x_out = rt->x[cur ^ 1];
    }
    a.weight = m->final_norm;
    a.eps = d.rms_eps;
    a.tokens = heads;
    a.K = H;
    a.h128 = false;
    a.seed = d.sign_seed;
    a.codes = rt->codes;
    a.scales = rt->scales;
    a.normed_out = rt->hidden_out;
    a.rows = sh.heads_identity ? nullptr : head_rows;
    const double HR = heads;
    const double add_rows = add_pending ? H * 4.0 + H * 4.0 : 0.0;
    Q35_KERNEL(Q35_KERNEL_PREP, HR * (H * 4.0 + add_rows + H + H / 32.0 * 4.0) + H * 4.0 + HR * H * 4.0,
               launch_rms_prep(a, s), "final norm prep");
    if (add_pending) cur ^= 1;
  }
  if (tracing) {
    const int fl = d.n_layers;
    Q35_STEP(trace_copy(rt, fl, Q35_TRACE_X_FINAL, rt->x[cur], static_cast<size_t>(batch) * H * 4, s), "trace");
    Q35_STEP(trace_copy(rt, fl, Q35_TRACE_HIDDEN, rt->hidden_out, static_cast<size_t>(batch) * H * 4, s), "trace");
    Q35_STEP(trace_codes(fl, Q35_TRACE_CODES_HEAD, H), "trace");
  }
  // the head in launches of at most kMaxTokens rows
  for (int h0 = 0; h0 < heads; h0 += kMaxTokens) {
    const int n = std::min(kMaxTokens, heads - h0);
    const double HB = n;
    const size_t tile0 = static_cast<size_t>(h0 / 16);
    if (want_logits) {
      GemmArgs g;
      g.w = m->embed;
      g.g16 = m->embed_g16;
      g.rows = d.vocab;
      g.nb = H / 32;
      g.codes = rt->codes + tile0 * (H / 32) * 64;
      g.scales = rt->scales + tile0 * (H / 32) * 16;
      g.tokens = n;
      g.out = rt->logits + static_cast<size_t>(h0) * d.vocab;
      g.stride = d.vocab;
      g.head = true;
      g.force_split = 1;  // rt->logits holds one [rows][vocab] copy: never split K here
      g.cu_count = ctx->cu_count;
      Q35_KERNEL(Q35_KERNEL_HEAD, gemm_algorithmic_bytes(d.vocab, H / 32, n, true, false) + g16_extra,
                 launch_gemm(g, s), "logits head");
    } else {
      GemmArgs g = greedy_head_args(rt, n, head_slots + h0, head_penalties + h0);
      g.codes = rt->codes + tile0 * (H / 32) * 64;
      g.scales = rt->scales + tile0 * (H / 32) * 16;
      const int ncand = gemm_argmax_cands(d.vocab, H / 32, n, ctx->cu_count, 0, m->embed_g16);
      Q35_KERNEL(Q35_KERNEL_HEAD,
                 gemm_algorithmic_bytes(d.vocab, H / 32, n, false, false) + g16_extra + ncand * HB * 8.0,
                 launch_gemm(g, s), "greedy head");
      Q35_KERNEL(Q35_KERNEL_ARGMAX, ncand * HB * 8.0 + HB * 4.0,
                 launch_argmax_finalize(rt->cand, ncand, kMaxTokens, n, rt->tokens_out_dev + h0, nullptr, s),
                 "argmax finalize");
    }
  }
#undef Q35_KERNEL
#undef Q35_STEP
  return Q35_OK;
}

}  // namespace q35

namespace {

// Validates the segments of a packed step on the host (no kernel ever sees
// an out-of-range index) and packs them into the pinned metadata block:
// rows segment by segment, a page-table row per segment, the head rows (the
// last position of each segment that wants a token) and the attention query
// tiles (runs of up to kAttnTileRows positions of one segment).
int pack_segments(q35_runtime *rt, const q35_segment *segs, int n, StepShape *shape) {
  Context *ctx = rt->ctx;
  const q35_model_dims &d = rt->model->d;
  if (segs == nullptr || n <= 0 || n > rt->max_segments)
    return set_error(ctx, Q35_ERR_INVALID, "segment count outside 1 .. max_batch + " +
                                               std::to_string(kMaxPrefillSegments));
  std::vector<uint8_t> seen(rt->cfg.max_slots, 0);
  long long rows = 0;
  for (int i = 0; i < n; ++i) {
    const q35_segment &g = segs[i];
    if (g.slot < 0 || g.slot >= rt->cfg.max_slots || !rt->slot_used[g.slot] || seen[g.slot])
      return set_error(ctx, Q35_ERR_INVALID, "step rows need distinct allocated slots");
    seen[g.slot] = 1;
    if (g.count <= 0 || g.tokens == nullptr || g.page_table == nullptr || g.max_pages <= 0)
      return set_error(ctx, Q35_ERR_INVALID, "invalid step segment");
    if (g.pos0 < 0 || static_cast<long long>(g.pos0) + g.count > rt->cfg.max_context)
      return set_error(ctx, Q35_ERR_INVALID, "position outside max_context");
    if (!(g.penalty >= 1.0F)) return set_error(ctx, Q35_ERR_INVALID, "penalty must be >= 1");
    for (int r = 0; r < g.count; ++r)
      if (g.tokens[r] < 0 || g.tokens[r] >= d.vocab) return set_error(ctx, Q35_ERR_INVALID, "token out of range");
    const int last = (g.pos0 + g.count - 1) / rt->cfg.page_tokens;
    if (last >= g.max_pages) return set_error(ctx, Q35_ERR_INVALID, "page table does not cover the position");
    for (int pg = 0; pg <= last; ++pg)
      if (g.page_table[pg] < 0 || g.page_table[pg] >= rt->cfg.total_pages || rt->page_ref[g.page_table[pg]] <= 0)
        return set_error(ctx, Q35_ERR_INVALID, "page table names a free or invalid page");
    rows += g.count;
  }
  if (rows > rt->max_rows)
    return set_error(ctx, Q35_ERR_INVALID, "step rows exceed max_step_rows (" + std::to_string(rt->max_rows) + ")");
  const MetaLayout ml = meta_layout(rt);
  unsigned char *h = rt->meta_host;
  std::memset(h, 0, rt->meta_bytes);
  auto *slots = reinterpret_cast<int32_t *>(h + ml.slots);
  auto *positions = reinterpret_cast<int32_t *>(h + ml.positions);
  auto *tokens = reinterpret_cast<int32_t *>(h + ml.tokens);
  auto *seq_lens = reinterpret_cast<int32_t *>(h + ml.seq_lens);
  auto *count_input = reinterpret_cast<uint8_t *>(h + ml.count_input);
  auto *row_seg = reinterpret_cast<int32_t *>(h + ml.row_seg);
  auto *seg_row0 = reinterpret_cast<int32_t *>(h + ml.seg_row0);
  auto *seg_count = reinterpret_cast<int32_t *>(h + ml.seg_count);
  auto *pt = reinterpret_cast<int32_t *>(h + ml.page_table);
  auto *head_rows = reinterpret_cast<int32_t *>(h + ml.head_rows);
  auto *head_slots = reinterpret_cast<int32_t *>(h + ml.head_slots);
  auto *head_pen = reinterpret_cast<float *>(h + ml.head_penalties);
  auto *tile_row0 = reinterpret_cast<int32_t *>(h + ml.tile_row0);
  auto *tile_rows = reinterpret_cast<int32_t *>(h + ml.tile_rows);
  auto *attn_rows = reinterpret_cast<int32_t *>(h + ml.attn_rows);
  auto *chunk_rows = reinterpret_cast<int32_t *>(h + ml.chunk_rows);
  StepShape sh;
  int r = 0, heads = 0, tiles = 0, singles = 0, multis = 0, longest = 1;
  for (int i = 0; i < n; ++i) {
    const q35_segment &g = segs[i];
    seg_row0[i] = r;
    seg_count[i] = g.count;
    const int used = std::min(g.max_pages, rt->max_pages_per_row);
    std::memcpy(pt + static_cast<size_t>(i) * rt->max_pages_per_row, g.page_table, static_cast<size_t>(used) * 4);
    if (g.count == 1) {
      attn_rows[singles++] = r;
    } else {
      for (int k = 0; k < g.count; ++k) chunk_rows[multis++] = r + k;
      for (int t0 = 0; t0 < g.count; t0 += kAttnTileRows) {
        tile_row0[tiles] = r + t0;
        tile_rows[tiles] = std::min(kAttnTileRows, g.count - t0);
        ++tiles;
      }
    }
    for (int k = 0; k < g.count; ++k, ++r) {
      slots[r] = g.slot;
      positions[r] = g.pos0 + k;
      tokens[r] = g.tokens[k];
      seq_lens[r] = g.pos0 + k + 1;  // causal: the prefix and the segment up to this position
      count_input[r] = g.count_input;
      row_seg[r] = i;
    }
    longest = std::max(longest, g.pos0 + g.count);
    if (g.want_token) {
      head_rows[heads] = r - 1;
      head_slots[heads] = g.slot;
      head_pen[heads] = g.penalty;
      sh.heads_identity = sh.heads_identity && heads == r - 1;
      ++heads;
    }
    sh.single = sh.single && g.count == 1;
  }
  if (heads == 0) return set_error(ctx, Q35_ERR_INVALID, "a step needs at least one segment that wants a token");
  // the scan's dispatch order: segments by row count, longest first (ties in
  // segment order)
  auto *seg_order = reinterpret_cast<int32_t *>(h + ml.seg_order);
  for (int i = 0; i < n; ++i) seg_order[i] = i;
  std::stable_sort(seg_order, seg_order + n, [&](int x, int y) { return seg_count[x] > seg_count[y]; });
  sh.rows = r;
  sh.segments = n;
  sh.heads = heads;
  sh.tiles = tiles;
  sh.attn_rows = singles;
  sh.heads_identity = sh.heads_identity && heads == r;
  // attention chunks of the longest context, rounded up to a power of two so
  // that few graph shapes cover a growing context
  const int need = (longest + rt->split_tokens - 1) / rt->split_tokens;
  int gs = 1;
  while (gs < need) gs <<= 1;
  sh.grid_splits = std::min(gs, rt->max_splits);
  *shape = sh;
  rt->shape = sh;
  return Q35_OK;
}

// A decode step descriptor as segments of one row that all want a token.
int pack_step(q35_runtime *rt, const q35_step_desc *desc, StepShape *shape) {
  const int B = desc->batch;
  if (B <= 0 || B > rt->cfg.max_batch || desc->slots == nullptr || desc->positions == nullptr ||
      desc->tokens == nullptr || desc->page_table == nullptr || desc->max_pages <= 0)
    return set_error(rt->ctx, Q35_ERR_INVALID, "invalid step descriptor");
  std::vector<q35_segment> segs(B);
  for (int b = 0; b < B; ++b) {
    q35_segment &g = segs[b];
    g.slot = desc->slots[b];
    g.pos0 = desc->positions[b];
    g.count = 1;
    g.tokens = desc->tokens + b;
    g.page_table = desc->page_table + static_cast<size_t>(b) * desc->max_pages;
    g.max_pages = desc->max_pages;
    g.penalty = desc->penalties ? desc->penalties[b] : 1.0F;
    g.count_input = desc->count_input ? desc->count_input[b] : 0;
    g.want_token = 1;
  }
  return pack_segments(rt, segs.data(), B, shape);
}

int ensure_logits(q35_runtime *rt) {
  if (rt->logits != nullptr) return Q35_OK;
  return rt_alloc(rt, static_cast<size_t>(rt->max_segments) * rt->model->d.vocab * 4,
                  reinterpret_cast<void **>(&rt->logits));
}

// Runs the packed step: replays (or captures) the graph of its shape, or
// launches eagerly (profiling and the stage trace time or copy single launches).
int launch_step_work(q35_runtime *rt, const StepShape &sh, bool want_logits) {
  Context *ctx = rt->ctx;
  int st = Q35_OK;
  if (rt->cfg.use_graphs && !rt->profiling && !rt->tracing) {
    const auto key = sh.key(want_logits);
    auto it = rt->graphs.find(key);
    if (it == rt->graphs.end()) {
      // a bounded cache: the decode shapes of a serving loop and a few chunk
      // shapes recur; anything else is re-captured when it comes back
      if (rt->graphs.size() >= 64) {
        Q35_HIP_TRY(ctx, hipStreamSynchronize(ctx->stream));
        for (auto &kv : rt->graphs) (void)hipGraphExecDestroy(kv.second);
        rt->graphs.clear();
      }
      Q35_HIP_TRY(ctx, hipStreamSynchronize(ctx->stream));
      Q35_HIP_TRY(ctx, hipStreamBeginCapture(ctx->stream, hipStreamCaptureModeThreadLocal));
      st = runtime_enqueue_step(rt, sh, want_logits);
      hipGraph_t graph = nullptr;
      const hipError_t ce = hipStreamEndCapture(ctx->stream, &graph);
      if (st != Q35_OK) {
        if (graph) (void)hipGraphDestroy(graph);
        return st;
      }
      if (ce != hipSuccess) return hip_error(ctx, ce, "end capture");
      hipGraphExec_t exec = nullptr;
      const hipError_t ie = hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0);
      (void)hipGraphDestroy(graph);
      if (ie != hipSuccess) return hip_error(ctx, ie, "graph instantiate");
      it = rt->graphs.emplace(key, exec).first;
    }
    if (rt->step_timing) Q35_HIP_TRY(ctx, hipEventRecord(rt->step_events[0], ctx->stream));
    Q35_HIP_TRY(ctx, hipGraphLaunch(it->second, ctx->stream));
  } else {
    if (rt->step_timing) Q35_HIP_TRY(ctx, hipEventRecord(rt->step_events[0], ctx->stream));
    st = runtime_enqueue_step(rt, sh, want_logits);
    if (st != Q35_OK) return st;
  }
  return Q35_OK;
}

// The step's launch, with step timing: an event pair on the stream around it
// (the graph replay, or the eager launches; a graph's capture, on the host,
// comes before the first event), waited on and added up at once.
int launch_step(q35_runtime *rt, const StepShape &sh, bool want_logits) {
  if (!rt->step_timing) return launch_step_work(rt, sh, want_logits);
  Context *ctx = rt->ctx;
  for (hipEvent_t &ev : rt->step_events)
    if (ev == nullptr) Q35_HIP_TRY(ctx, hipEventCreate(&ev));
  const int st = launch_step_work(rt, sh, want_logits);
  if (st != Q35_OK) return st;
  Q35_HIP_TRY(ctx, hipEventRecord(rt->step_events[1], ctx->stream));
  Q35_HIP_TRY(ctx, hipEventSynchronize(rt->step_events[1]));
  float ms = 0.0F;
  Q35_HIP_TRY(ctx, hipEventElapsedTime(&ms, rt->step_events[0], rt->step_events[1]));
  rt->step_gpu_ms += ms;
  ++rt->step_count;
  return Q35_OK;
}

}  // namespace

extern "C" int q35_runtime_step(q35_runtime *rt, const q35_step_desc *desc, int32_t *out_tokens,
                                float *out_logits) {
  if (rt == nullptr || desc == nullptr) return Q35_ERR_INVALID;
  Context *ctx = rt->ctx;
  const q35_model_dims &d = rt->model->d;
  const int B = desc->batch;
  StepShape sh;
  int st = pack_step(rt, desc, &sh);
  if (st != Q35_OK) return st;
  const bool want_logits = out_logits != nullptr;
  if (want_logits && (st = ensure_logits(rt)) != Q35_OK) return st;
  if ((st = launch_step(rt, sh, want_logits)) != Q35_OK) return st;
  if (want_logits)
    Q35_HIP_TRY(ctx, hipMemcpyAsync(out_logits, rt->logits, static_cast<size_t>(B) * d.vocab * 4,
                                    hipMemcpyDeviceToHost, ctx->stream));
  Q35_HIP_TRY(ctx, hipStreamSynchronize(ctx->stream));
  if (rt->profiling) {
    st = profile_collect(rt);
    if (st != Q35_OK) return st;
  }
  rt->last_batch = B;
  if (out_tokens != nullptr) {
    if (want_logits) {
      // greedy token from the raw logits with the penalty rule
      // (cpu_engine_greedy.inl:45-57 / sample_token_from_logits, layers.inl:519-545)
      std::vector<int32_t> cnt(d.vocab);
      for (int b = 0; b < B; ++b) {
        const float *lg = out_logits + static_cast<size_t>(b) * d.vocab;
        const float pen = desc->penalties ? desc->penalties[b] : 1.0F;
        if (pen > 1.0F)
          Q35_HIP_TRY(ctx, hipMemcpy(cnt.data(), rt->counts + static_cast<size_t>(desc->slots[b]) * d.vocab,
                                     d.vocab * 4, hipMemcpyDeviceToHost));
        float best = -INFINITY;
        int at = 0;
        for (int t = 0; t < d.vocab; ++t) {
          float v = lg[t];
          if (pen > 1.0F && cnt[t] > 0) v = v > 0 ? v / pen : v * pen;
          if (v > best) { best = v; at = t; }
        }
        out_tokens[b] = at;
      }
    } else {
      std::memcpy(out_tokens, rt->tokens_out_host, B * 4);
    }
  }
  return Q35_OK;
}

namespace {

// Per-head-row candidate settings into the metadata block (head rows
// 0..B-1; `sampling` indexed by head row).
int pack_sampling(q35_runtime *rt, int B, const q35_row_sampling *sampling) {
  if (sampling == nullptr) return set_error(rt->ctx, Q35_ERR_INVALID, "missing sampling rows");
  const MetaLayout ml = meta_layout(rt);
  auto *inv_t = reinterpret_cast<float *>(rt->meta_host + ml.inv_temperature);
  auto *top_k = reinterpret_cast<int32_t *>(rt->meta_host + ml.top_k);
  for (int b = 0; b < B; ++b) {
    const q35_row_sampling &r = sampling[b];
    if (r.top_k < 1 || r.top_k > kMaxCandidates || !std::isfinite(r.inv_temperature) || !(r.inv_temperature > 0.0F))
      return set_error(rt->ctx, Q35_ERR_INVALID, "candidate count must be 1..64 and the scale finite and positive");
    inv_t[b] = r.inv_temperature;
    top_k[b] = r.top_k;
  }
  return Q35_OK;
}

// Candidate selection over rows 0..rows-1 of rt->logits with the metadata
// block's slots, penalties and sampling settings, then the copies back.
int finish_candidates(q35_runtime *rt, int rows, q35_candidate *out, float *raw_logits) {
  Context *ctx = rt->ctx;
  const q35_model_dims &d = rt->model->d;
  const MetaLayout ml = meta_layout(rt);
  SampleArgs a;
  a.logits = rt->logits;
  a.logits_stride = d.vocab;
  a.rows = rows;
  a.vocab = d.vocab;
  a.counts = rt->counts;
  a.count_rows = reinterpret_cast<const int32_t *>(rt->meta_dev + ml.head_slots);
  a.penalties = reinterpret_cast<const float *>(rt->meta_dev + ml.head_penalties);
  a.inv_temperature = reinterpret_cast<const float *>(rt->meta_dev + ml.inv_temperature);
  a.top_k = reinterpret_cast<const int32_t *>(rt->meta_dev + ml.top_k);
  a.out = rt->candidates;
  Q35_HIP_TRY(ctx, launch_sample_candidates(a, rt->sample_scratch, ctx->stream));
  Q35_HIP_TRY(ctx, hipMemcpyAsync(out, rt->candidates, static_cast<size_t>(rows) * kMaxCandidates * sizeof(q35_candidate),
                                  hipMemcpyDeviceToHost, ctx->stream));
  if (raw_logits != nullptr)
    Q35_HIP_TRY(ctx, hipMemcpyAsync(raw_logits, rt->logits, static_cast<size_t>(rows) * d.vocab * 4,
                                    hipMemcpyDeviceToHost, ctx->stream));
  Q35_HIP_TRY(ctx, hipStreamSynchronize(ctx->stream));
  rt->last_batch = rows;
  return Q35_OK;
}

}  // namespace

extern "C" int q35_runtime_step_candidates(q35_runtime *rt, const q35_step_desc *desc,
                                           const q35_row_sampling *sampling, q35_candidate *out_candidates,
                                           float *raw_logits) {
  if (rt == nullptr || desc == nullptr || out_candidates == nullptr) return Q35_ERR_INVALID;
  StepShape sh;
  int st = pack_step(rt, desc, &sh);
  if (st == Q35_OK) st = pack_sampling(rt, desc->batch, sampling);
  if (st == Q35_OK) st = ensure_logits(rt);
  if (st == Q35_OK) st = launch_step(rt, sh, true);
  if (st != Q35_OK) return st;
  if (rt->profiling) {
    Q35_HIP_TRY(rt->ctx, hipStreamSynchronize(rt->ctx->stream));
    if ((st = profile_collect(rt)) != Q35_OK) return st;
  }
  return finish_candidates(rt, desc->batch, out_candidates, raw_logits);
}

extern "C" int q35_runtime_head_candidates(q35_runtime *rt, int32_t slot, const float *hidden, float penalty,
                                           const q35_row_sampling *sampling, q35_candidate *out_candidates,
                                           float *raw_logits) {
  if (rt == nullptr || hidden == nullptr || out_candidates == nullptr) return Q35_ERR_INVALID;
  if (slot < 0 || slot >= rt->cfg.max_slots || !rt->slot_used[slot])
    return set_error(rt->ctx, Q35_ERR_INVALID, "head needs an allocated slot");
  if (!(penalty >= 1.0F)) return set_error(rt->ctx, Q35_ERR_INVALID, "penalty must be >= 1");
  Context *ctx = rt->ctx;
  const q35_model_dims &d = rt->model->d;
  const MetaLayout ml = meta_layout(rt);
  std::memset(rt->meta_host, 0, rt->meta_bytes);
  int st = pack_sampling(rt, 1, sampling);
  if (st == Q35_OK) st = ensure_logits(rt);
  if (st != Q35_OK) return st;
  reinterpret_cast<int32_t *>(rt->meta_host + ml.head_slots)[0] = slot;
  reinterpret_cast<float *>(rt->meta_host + ml.head_penalties)[0] = penalty;
  hipStream_t s = ctx->stream;
  Q35_HIP_TRY(ctx, hipMemcpyAsync(rt->meta_dev, rt->meta_host, rt->meta_bytes, hipMemcpyHostToDevice, s));
  Q35_HIP_TRY(ctx, hipMemcpyAsync(rt->hidden_out, hidden, static_cast<size_t>(d.hidden) * 4, hipMemcpyHostToDevice, s));
  PrepArgs p;
  p.source = kPrepPlain;
  p.x = rt->hidden_out;
  p.x_stride = d.hidden;
  p.tokens = 1;
  p.K = d.hidden;
  p.h128 = false;
  p.seed = d.sign_seed;
  p.codes = rt->codes;
  p.scales = rt->scales;
  Q35_HIP_TRY(ctx, launch_prep(p, s));
  GemmArgs g;
  g.w = rt->model->embed;
  g.g16 = rt->model->embed_g16;
  g.rows = d.vocab;
  g.nb = d.hidden / 32;
  g.codes = rt->codes;
  g.scales = rt->scales;
  g.tokens = 1;
  g.out = rt->logits;
  g.stride = d.vocab;
  g.head = true;
  g.force_split = 1;
  g.cu_count = ctx->cu_count;
  Q35_HIP_TRY(ctx, launch_gemm(g, s));
  return finish_candidates(rt, 1, out_candidates, raw_logits);
}

extern "C" int q35_slot_counts(q35_runtime *rt, int32_t slot, int32_t *out, size_t count) {
  if (rt == nullptr || out == nullptr) return Q35_ERR_INVALID;
  if (slot < 0 || slot >= rt->cfg.max_slots || !rt->slot_used[slot] || count < static_cast<size_t>(rt->model->d.vocab))
    return set_error(rt->ctx, Q35_ERR_INVALID, "counts need an allocated slot and vocab entries");
  Q35_HIP_TRY(rt->ctx, hipMemcpy(out, rt->counts + static_cast<size_t>(slot) * rt->model->d.vocab,
                                 static_cast<size_t>(rt->model->d.vocab) * 4, hipMemcpyDeviceToHost));
  return Q35_OK;
}

extern "C" int q35_runtime_set_profiling(q35_runtime *rt, int enable) {
  if (rt == nullptr) return Q35_ERR_INVALID;
  rt->profiling = enable != 0;
  rt->prof_pending.clear();
  return Q35_OK;
}

extern "C" int q35_runtime_profile_reset(q35_runtime *rt) {
  if (rt == nullptr) return Q35_ERR_INVALID;
  for (int c = 0; c < Q35_KERNEL_CLASSES; ++c) rt->prof_ms[c] = rt->prof_bytes[c] = 0, rt->prof_launches[c] = 0;
  return Q35_OK;
}

extern "C" int q35_runtime_profile_read(q35_runtime *rt, int cls, double *total_ms, uint64_t *launches,
                                        double *bytes) {
  if (rt == nullptr || cls < 0 || cls >= Q35_KERNEL_CLASSES) return Q35_ERR_INVALID;
  if (total_ms) *total_ms = rt->prof_ms[cls];
  if (launches) *launches = rt->prof_launches[cls];
  if (bytes) *bytes = rt->prof_bytes[cls];
  return Q35_OK;
}

extern "C" int q35_runtime_set_step_timing(q35_runtime *rt, int enable) {
  if (rt == nullptr) return Q35_ERR_INVALID;
  rt->step_timing = enable != 0;
  rt->step_gpu_ms = 0.0;
  rt->step_count = 0;
  return Q35_OK;
}

extern "C" int q35_runtime_step_timing_read(q35_runtime *rt, double *gpu_ms, uint64_t *steps) {
  if (rt == nullptr) return Q35_ERR_INVALID;
  if (gpu_ms) *gpu_ms = rt->step_gpu_ms;
  if (steps) *steps = rt->step_count;
  return Q35_OK;
}

extern "C" int q35_runtime_set_fused(q35_runtime *rt, int enable) {
  if (rt == nullptr) return Q35_ERR_INVALID;
  if (rt->fuse_decode != (enable != 0)) {
    for (auto &kv : rt->graphs) (void)hipGraphExecDestroy(kv.second);
    rt->graphs.clear();
  }
  rt->fuse_decode = enable != 0;
  return Q35_OK;
}

extern "C" int q35_runtime_set_trace(q35_runtime *rt, int enable) {
  if (rt == nullptr) return Q35_ERR_INVALID;
  rt->tracing = enable != 0;
  return Q35_OK;
}

extern "C" int q35_runtime_trace_read(q35_runtime *rt, int layer, int point, void *out, size_t capacity,
                                      size_t *bytes) {
  if (rt == nullptr || point < 0 || point >= Q35_TRACE_POINTS) return Q35_ERR_INVALID;
  auto it = rt->trace.find(std::make_pair(layer, point));
  const size_t n = it == rt->trace.end() ? 0 : it->second.second;
  if (bytes != nullptr) *bytes = n;
  if (n == 0 || out == nullptr) return Q35_OK;
  Q35_HIP_TRY(rt->ctx, hipStreamSynchronize(rt->ctx->stream));
  Q35_HIP_TRY(rt->ctx, hipMemcpy(out, it->second.first, std::min(n, capacity), hipMemcpyDeviceToHost));
  return Q35_OK;
}

extern "C" int q35_runtime_prefill(q35_runtime *rt, int32_t slot, int32_t pos0, const int32_t *tokens,
                                   int32_t count, const int32_t *page_table, int32_t max_pages, float penalty,
                                   int32_t *out_token) {
  if (rt == nullptr) return Q35_ERR_INVALID;
  Context *ctx = rt->ctx;
  if (tokens == nullptr || page_table == nullptr || count <= 0 || count > rt->max_rows || max_pages <= 0)
    return set_error(ctx, Q35_ERR_INVALID, "invalid prefill chunk");
  // one segment: every position of the chunk on the request's slot and pages
  q35_segment g{};
  g.slot = slot;
  g.pos0 = pos0;
  g.count = count;
  g.tokens = tokens;
  g.page_table = page_table;
  g.max_pages = max_pages;
  g.penalty = penalty;
  g.count_input = 0;
  g.want_token = 1;
  StepShape sh;
  int st = pack_segments(rt, &g, 1, &sh);
  if (st != Q35_OK) return st;
  if ((st = launch_step(rt, sh, false)) != Q35_OK) return st;
  Q35_HIP_TRY(ctx, hipStreamSynchronize(ctx->stream));
  if (rt->profiling) {
    st = profile_collect(rt);
    if (st != Q35_OK) return st;
  }
  rt->last_batch = 1;  // the head ran on the chunk's last position only
  if (out_token != nullptr) *out_token = rt->tokens_out_host[0];
  return Q35_OK;
}

extern "C" int q35_runtime_step_segments(q35_runtime *rt, const q35_segment *segments, int32_t count,
                                         const q35_row_sampling *sampling, int32_t *out_tokens,
                                         q35_candidate *out_candidates, float *raw_logits) {
  if (rt == nullptr || out_tokens == nullptr) return Q35_ERR_INVALID;
  Context *ctx = rt->ctx;
  if (sampling != nullptr && out_candidates == nullptr)
    return set_error(ctx, Q35_ERR_INVALID, "sampling needs out_candidates");
  StepShape sh;
  int st = pack_segments(rt, segments, count, &sh);
  if (st != Q35_OK) return st;
  // head row h -> segment
  std::vector<int> head_seg;
  for (int i = 0; i < count; ++i)
    if (segments[i].want_token) head_seg.push_back(i);
  const bool want_logits = sampling != nullptr;
  if (want_logits) {
    std::vector<q35_row_sampling> rows(sh.heads);
    for (int h = 0; h < sh.heads; ++h) rows[h] = sampling[head_seg[h]];
    if ((st = pack_sampling(rt, sh.heads, rows.data())) != Q35_OK) return st;
    if ((st = ensure_logits(rt)) != Q35_OK) return st;
  }
  if ((st = launch_step(rt, sh, want_logits)) != Q35_OK) return st;
  if (rt->profiling) {
    Q35_HIP_TRY(ctx, hipStreamSynchronize(ctx->stream));
    if ((st = profile_collect(rt)) != Q35_OK) return st;
  }
  for (int i = 0; i < count; ++i) out_tokens[i] = -1;
  if (!want_logits) {
    Q35_HIP_TRY(ctx, hipStreamSynchronize(ctx->stream));
    rt->last_batch = sh.heads;
    for (int h = 0; h < sh.heads; ++h) out_tokens[head_seg[h]] = rt->tokens_out_host[h];
    return Q35_OK;
  }
  const int vocab = rt->model->d.vocab;
  std::vector<q35_candidate> cands(static_cast<size_t>(sh.heads) * kMaxCandidates);
  std::vector<float> raw(raw_logits != nullptr ? static_cast<size_t>(sh.heads) * vocab : 0);
  if ((st = finish_candidates(rt, sh.heads, cands.data(), raw_logits != nullptr ? raw.data() : nullptr)) != Q35_OK)
    return st;
  rt->last_batch = sh.heads;
  for (int i = 0; i < count; ++i)
    for (int k = 0; k < kMaxCandidates; ++k)
      out_candidates[static_cast<size_t>(i) * kMaxCandidates + k] = q35_candidate{-INFINITY, -1};
  for (int h = 0; h < sh.heads; ++h) {
    std::memcpy(out_candidates + static_cast<size_t>(head_seg[h]) * kMaxCandidates,
                cands.data() + static_cast<size_t>(h) * kMaxCandidates, kMaxCandidates * sizeof(q35_candidate));
    if (raw_logits != nullptr)
      std::memcpy(raw_logits + static_cast<size_t>(head_seg[h]) * vocab, raw.data() + static_cast<size_t>(h) * vocab,
                  static_cast<size_t>(vocab) * 4);
  }
  return Q35_OK;
}

extern "C" int q35_runtime_last_hidden(q35_runtime *rt, float *out, size_t count) {
  if (rt == nullptr || out == nullptr) return Q35_ERR_INVALID;
  const size_t n = std::min(count, static_cast<size_t>(rt->last_batch) * rt->model->d.hidden);
  Q35_HIP_TRY(rt->ctx, hipMemcpy(out, rt->hidden_out, n * 4, hipMemcpyDeviceToHost));
  return Q35_OK;
}

// ============================================================ prefix snapshots
// CpuPrefix (cpu_engine.h:32-45): captured by register_prefix
// (cpu_engine_prefix.inl:31-96), restored in initialize (cpu_engine.inl:386-407).
struct q35_state_snapshot {
  q35_runtime *rt = nullptr;
  int32_t tokens = 0;
  float *state = nullptr;     // one recurrent copy, then the conv ring
  std::vector<float> hidden;  // final normalized row of position tokens - 1
  size_t bytes = 0;
};

extern "C" int q35_state_snapshot_create(q35_runtime *rt, int32_t slot, int32_t tokens, const float *hidden,
                                         q35_state_snapshot **out) {
  if (rt == nullptr || out == nullptr) return Q35_ERR_INVALID;
  *out = nullptr;
  if (slot < 0 || slot >= rt->cfg.max_slots || !rt->slot_used[slot] || tokens <= 0 || tokens > rt->cfg.max_context)
    return set_error(rt->ctx, Q35_ERR_INVALID, "snapshot needs an allocated slot and a token count");
  auto *snap = new (std::nothrow) q35_state_snapshot();
  if (snap == nullptr) return Q35_ERR_OOM;
  const size_t rec = static_cast<size_t>(rt->rec_copy_stride), conv = static_cast<size_t>(rt->conv_slot_stride);
  snap->rt = rt;
  snap->tokens = tokens;
  snap->bytes = (rec + conv) * 4 + (hidden != nullptr ? rt->model->d.hidden * 4 : 0);
  if (hidden != nullptr) snap->hidden.assign(hidden, hidden + rt->model->d.hidden);
  Context *ctx = rt->ctx;
  const hipError_t e = hipMalloc(reinterpret_cast<void **>(&snap->state), (rec + conv) * 4);
  if (e != hipSuccess) {
    delete snap;
    return hip_error(ctx, e, "snapshot allocation");
  }
  // the state after `tokens` positions is copy (tokens & 1): position p reads
  // copy p & 1 and writes the other
  const float *src = rt->recurrent + slot * rt->rec_slot_stride + (tokens & 1) * rt->rec_copy_stride;
  hipError_t c = hipMemcpyAsync(snap->state, src, rec * 4, hipMemcpyDeviceToDevice, ctx->stream);
  if (c == hipSuccess)
    c = hipMemcpyAsync(snap->state + rec, rt->conv + slot * rt->conv_slot_stride, conv * 4, hipMemcpyDeviceToDevice,
                       ctx->stream);
  if (c == hipSuccess) c = hipStreamSynchronize(ctx->stream);
  if (c != hipSuccess) {
    (void)hipFree(snap->state);
    delete snap;
    return hip_error(ctx, c, "snapshot copy");
  }
  *out = snap;
  return Q35_OK;
}

extern "C" int q35_state_snapshot_restore(q35_runtime *rt, const q35_state_snapshot *snap, int32_t slot) {
  if (rt == nullptr || snap == nullptr || snap->rt != rt) return Q35_ERR_INVALID;
  if (slot < 0 || slot >= rt->cfg.max_slots || !rt->slot_used[slot])
    return set_error(rt->ctx, Q35_ERR_INVALID, "restore needs an allocated slot");
  Context *ctx = rt->ctx;
  const size_t rec = static_cast<size_t>(rt->rec_copy_stride), conv = static_cast<size_t>(rt->conv_slot_stride);
  float *dst = rt->recurrent + slot * rt->rec_slot_stride + (snap->tokens & 1) * rt->rec_copy_stride;
  Q35_HIP_TRY(ctx, hipMemcpyAsync(dst, snap->state, rec * 4, hipMemcpyDeviceToDevice, ctx->stream));
  Q35_HIP_TRY(ctx, hipMemcpyAsync(rt->conv + slot * rt->conv_slot_stride, snap->state + rec, conv * 4,
                                  hipMemcpyDeviceToDevice, ctx->stream));
  Q35_HIP_TRY(ctx, hipStreamSynchronize(ctx->stream));
  return Q35_OK;
}

extern "C" int32_t q35_state_snapshot_tokens(const q35_state_snapshot *snap) { return snap ? snap->tokens : 0; }
extern "C" size_t q35_state_snapshot_bytes(const q35_state_snapshot *snap) { return snap ? snap->bytes : 0; }

extern "C" void q35_state_snapshot_destroy(q35_state_snapshot *snap) {
  if (snap == nullptr) return;
  (void)hipSetDevice(snap->rt->ctx->device);
  (void)hipStreamSynchronize(snap->rt->ctx->stream);
  (void)hipFree(snap->state);
  delete snap;
}

extern "C" int q35_state_snapshot_hidden(const q35_state_snapshot *snap, float *out, size_t count) {
  if (snap == nullptr || out == nullptr || snap->hidden.empty() || count < snap->hidden.size()) return Q35_ERR_INVALID;
  std::memcpy(out, snap->hidden.data(), snap->hidden.size() * 4);
  return Q35_OK;
}

// Greedy head of one final normalized hidden row (greedy_q4_token,
// weights.inl:1217-1295): identity-basis q8 preparation of the row (the same
// codes the step's final norm writes for it), the Q4 head with the slot's
// penalty counts, argmax.
extern "C" int q35_runtime_head(q35_runtime *rt, int32_t slot, const float *hidden, float penalty,
                                int32_t *out_token) {
  if (rt == nullptr || hidden == nullptr || out_token == nullptr) return Q35_ERR_INVALID;
  if (slot < 0 || slot >= rt->cfg.max_slots || !rt->slot_used[slot])
    return set_error(rt->ctx, Q35_ERR_INVALID, "head needs an allocated slot");
  if (!(penalty >= 1.0F)) return set_error(rt->ctx, Q35_ERR_INVALID, "penalty must be >= 1");
  Context *ctx = rt->ctx;
  const q35_model_dims &d = rt->model->d;
  const MetaLayout ml = meta_layout(rt);
  std::memset(rt->meta_host, 0, rt->meta_bytes);
  reinterpret_cast<int32_t *>(rt->meta_host + ml.head_slots)[0] = slot;
  reinterpret_cast<float *>(rt->meta_host + ml.head_penalties)[0] = penalty;
  hipStream_t s = ctx->stream;
  Q35_HIP_TRY(ctx, hipMemcpyAsync(rt->meta_dev, rt->meta_host, rt->meta_bytes, hipMemcpyHostToDevice, s));
  Q35_HIP_TRY(ctx, hipMemcpyAsync(rt->hidden_out, hidden, static_cast<size_t>(d.hidden) * 4, hipMemcpyHostToDevice, s));
  PrepArgs p;
  p.source = kPrepPlain;
  p.x = rt->hidden_out;
  p.x_stride = d.hidden;
  p.tokens = 1;
  p.K = d.hidden;
  p.h128 = false;
  p.seed = d.sign_seed;
  p.codes = rt->codes;
  p.scales = rt->scales;
  Q35_HIP_TRY(ctx, launch_prep(p, s));
  const GemmArgs g = greedy_head_args(rt, 1, reinterpret_cast<const int32_t *>(rt->meta_dev + ml.head_slots),
                                      reinterpret_cast<const float *>(rt->meta_dev + ml.head_penalties));
  Q35_HIP_TRY(ctx, launch_gemm(g, s));
  const int ncand = gemm_argmax_cands(d.vocab, d.hidden / 32, 1, ctx->cu_count, 0, rt->model->embed_g16);
  Q35_HIP_TRY(ctx, launch_argmax_finalize(rt->cand, ncand, kMaxTokens, 1, rt->tokens_out_dev, nullptr, s));
  Q35_HIP_TRY(ctx, hipStreamSynchronize(s));
  rt->last_batch = 1;
  *out_token = rt->tokens_out_host[0];
  return Q35_OK;
}
