// extern "C" boundary of libmi355x_encoder.so (declared in include/mi355x_encoder.h).
//
// Every entry point validates its arguments, launches on the caller's stream and
// returns a status code; the message of the last failure is kept per thread.
// Nothing here allocates device memory or synchronises the host.
#include <hip/hip_runtime.h>

#include <cstdio>
#include <cstring>
#include <mutex>
#include <string>

#include "../../include/mi355x_encoder.h"
#include "common.h"
#include "kernels.h"

namespace {

thread_local std::string g_last_error;

int fail(int code, const std::string& msg) {
  g_last_error = msg;
  return code;
}

int fail_hip(hipError_t err, const std::string& where) {
  std::string msg = where + ": " + hipGetErrorString(err);
  if (err == hipErrorOutOfMemory || err == hipErrorMemoryAllocation) {
    return fail(ENC_ERR_OOM, msg + " (out of memory)");
  }
  return fail(ENC_ERR_HIP, msg);
}

int ok() {
  g_last_error.clear();
  return ENC_OK;
}

// Compute units of the current device, cached per device ordinal.
int device_cus() {
  static int cache[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (cache[dev] == 0) {
    int cus = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0)
      cus = 256;
    cache[dev] = cus;
  }
  return cache[dev];
}

inline int64_t align_up(int64_t v, int64_t a) { return (v + a - 1) / a * a; }

// Library-owned activation workspace of enc_encoder_forward_bf16_noalloc: one
// copy per GPU, loaded with the code object and held until the process ends.
// In host code `scratch` names a host-side stand-in; kernels get the device
// address kept in g_scratch_ptr, looked up once per device.
constexpr int64_t kScratchBytes = ENC_NOALLOC_SCRATCH_BYTES;
__device__ __align__(256) unsigned char scratch[kScratchBytes];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mutex;
void* g_scratch_ptr[kMaxDevices] = {nullptr};

// Device address of this device's scratch array (looked up on the first call
// per device, with that device current), or an error code.
int scratch_for_current_device(void** ptr) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return fail_hip(e, "noalloc: hipGetDevice");
  if (dev < 0 || dev >= kMaxDevices) return fail(ENC_ERR_UNSUPPORTED, "noalloc: device ordinal out of range");
  std::lock_guard<std::mutex> guard(g_scratch_mutex);
  if (g_scratch_ptr[dev] == nullptr) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return fail_hip(e, "noalloc: hipGetSymbolAddress(scratch)");
    if (p == nullptr) return fail(ENC_ERR_HIP, "noalloc: scratch has no device address");
    g_scratch_ptr[dev] = p;
  }
  *ptr = g_scratch_ptr[dev];
  return ENC_OK;
}

// Workspace carve-up for the encoder forward.
struct EncoderWorkspace {
  int64_t ln, q, k, vt, ctx, xa, xb, hidden, total;
};

EncoderWorkspace plan_workspace(int64_t B, int64_t S, int64_t D, int64_t H, int64_t F) {
  const int64_t T = B * S;
  const int64_t hd = D / H;
  const int64_t e = 2;  // bf16 bytes
  EncoderWorkspace w{};
  int64_t off = 0;
  auto take = [&](int64_t bytes) {
    const int64_t at = off;
    off = align_up(off + bytes, 256);
    return at;
  };
  w.ln = take(T * D * e);
  w.q = take(T * D * e);
  w.k = take(T * D * e);
  w.vt = take(B * H * hd * enc::vt_stride(S) * e);
  w.ctx = take(T * D * e);
  w.xa = take(T * D * e);
  w.xb = take(T * D * e);
  w.hidden = take(T * F * e);
  w.total = off;
  return w;
}

bool shape_ok(int64_t v) { return v > 0 && v < (int64_t(1) << 31); }

int check_encoder_shape(int64_t B, int64_t S, int64_t D, int64_t H, int64_t F, bool exact_attention) {
  if (!shape_ok(B) || !shape_ok(S) || !shape_ok(D) || !shape_ok(H) || !shape_ok(F))
    return fail(ENC_ERR_INVALID, "batch, seq_len, d_model, num_heads and ffn_dim must be positive");
  if (D % H != 0) return fail(ENC_ERR_INVALID, "d_model must be divisible by num_heads");
  const int64_t hd = D / H;
  if (exact_attention ? !(hd == 8 || hd == 32 || hd == 64 || hd == 128 || hd == 256) : hd != 64)
    return fail(ENC_ERR_UNSUPPORTED,
                std::string(exact_attention ? "attention kernel supports head_dim 8, 32, 64, 128 or 256"
                                            : "online attention kernel supports head_dim 64 only") +
                    " (got " + std::to_string(hd) + ")");
  if (!enc::layernorm_supported(D))
    return fail(ENC_ERR_UNSUPPORTED, "LayerNorm width must be a power of two in [32, 4096] (got " +
                                         std::to_string(D) + ")");
  if (exact_attention && !enc::attention_seq_supported(S, hd))
    return fail(ENC_ERR_UNSUPPORTED, "seq_len above 2048 must be a multiple of 4, and one head's keys under "
                                     "4 GiB (got " + std::to_string(S) + ")");
  if (D % 32 != 0 || F % 32 != 0)
    return fail(ENC_ERR_UNSUPPORTED, "d_model and ffn_dim must be multiples of 32");
  if (B * S >= (int64_t(1) << 31)) return fail(ENC_ERR_UNSUPPORTED, "batch * seq_len must be < 2^31");
  return ENC_OK;
}

}  // namespace

namespace {

// Argument checks shared by the two encoder entry points; on success *plan
// holds the workspace carve-up for the shape.
int check_encoder_call(const void* x, void* out, const void* const* weights, int64_t batch, int64_t seq_len,
                       int64_t d_model, int64_t num_heads, int64_t ffn_dim, int64_t num_layers, float eps,
                       const int32_t* kv_len, const uint8_t* key_mask, int32_t flags, EncoderWorkspace* plan) {
  if (flags & ~(ENC_FWD_ONLINE_ATTENTION | ENC_FWD_SKIP_FINAL_NORM | ENC_FWD_PACKED_WEIGHTS))
    return fail(ENC_ERR_INVALID, "encoder: unknown flags");
  const bool final_norm = (flags & ENC_FWD_SKIP_FINAL_NORM) == 0;
  if (!final_norm && num_layers < 1) return fail(ENC_ERR_INVALID, "encoder: skipping final_norm needs a layer");
  const bool exact = (flags & ENC_FWD_ONLINE_ATTENTION) == 0;
  int rc = check_encoder_shape(batch, seq_len, d_model, num_heads, ffn_dim, exact);
  if (rc != ENC_OK) return rc;
  if (num_layers < 0) return fail(ENC_ERR_INVALID, "encoder: num_layers must be >= 0");
  if (!x || !out || !weights) return fail(ENC_ERR_INVALID, "encoder: null pointer");
  if (kv_len && key_mask) return fail(ENC_ERR_INVALID, "encoder: pass kv_len or key_mask, not both");
  if (!(eps > 0.f)) return fail(ENC_ERR_INVALID, "encoder: eps must be positive");
  const int64_t num_ptrs = 12 * num_layers + 2 + ((flags & ENC_FWD_PACKED_WEIGHTS) ? 4 * num_layers : 0);
  for (int64_t i = 0; i < num_ptrs; ++i)
    if (!weights[i]) return fail(ENC_ERR_INVALID, "encoder: null weight pointer at index " + std::to_string(i));
  if (flags & ENC_FWD_PACKED_WEIGHTS) {
    // every packed matrix must have the shape's packed form
    const int64_t shapes[4][2] = {{3 * d_model, d_model}, {d_model, d_model}, {ffn_dim, d_model}, {d_model, ffn_dim}};
    for (const auto& nk : shapes)
      if (enc::gemm_prepack_rows(nk[0], nk[1]) == 0)
        return fail(ENC_ERR_UNSUPPORTED, "encoder: packed weights need out_features % 128 == 0 (got " +
                                             std::to_string(nk[0]) + " x " + std::to_string(nk[1]) + ")");
  }
  *plan = plan_workspace(batch, seq_len, d_model, num_heads, ffn_dim);
  return ENC_OK;
}

// The FFN half of a block: hidden = bf16(gelu(bf16(h . w_in^T + b_in))),
// out = bf16(residual + bf16(hidden . w_out^T + b_out)), rows with
// row_mask == 0 written as zeros (the block output's masked_fill).  Optional
// packed weight copies (null: the plain weights only).
hipError_t ffn_block(const enc::bf16_t* h, const enc::bf16_t* w_in, const enc::bf16_t* b_in,
                     const enc::bf16_t* w_out, const enc::bf16_t* b_out, const enc::bf16_t* residual,
                     enc::bf16_t* out, enc::bf16_t* hidden, int64_t rows, int64_t D, int64_t F,
                     const uint8_t* row_mask, const enc::bf16_t* w_in_packed, const enc::bf16_t* w_out_packed,
                     int cus, hipStream_t st, const char** stage) {
  enc::GemmEpilogueArgs fa;
  fa.bias = b_in;
  fa.out = hidden;
  if (w_in_packed) {
    fa.w_packed = w_in_packed;
    fa.w_packed_rows = enc::gemm_prepack_rows(F, D);
  }
  *stage = "ffn_in";
  hipError_t e = enc::gemm_bf16(h, w_in, rows, F, D, enc::kEpiBiasGelu, fa, cus, st);
  if (e != hipSuccess) return e;
  enc::GemmEpilogueArgs fo;
  fo.bias = b_out;
  fo.residual = residual;
  fo.row_mask = row_mask;
  fo.out = out;
  if (w_out_packed) {
    fo.w_packed = w_out_packed;
    fo.w_packed_rows = enc::gemm_prepack_rows(D, F);
  }
  *stage = "ffn_out";
  return enc::gemm_bf16(hidden, w_out, rows, D, F, enc::kEpiResidualZero, fo, cus, st);
}

// The launch sequence of the encoder forward over a workspace laid out as `w`.
int run_encoder_forward(const void* x, void* out, void* workspace, const EncoderWorkspace& w,
                        const void* const* weights, int64_t batch, int64_t seq_len, int64_t d_model,
                        int64_t num_heads, int64_t ffn_dim, int64_t num_layers, float eps, int32_t causal,
                        const int32_t* kv_len, const uint8_t* key_mask, const uint8_t* row_mask, int32_t flags,
                        void* stream) {
  const bool final_norm = (flags & ENC_FWD_SKIP_FINAL_NORM) == 0;
  const bool exact = (flags & ENC_FWD_ONLINE_ATTENTION) == 0;
  using enc::bf16_t;
  hipStream_t st = static_cast<hipStream_t>(stream);
  char* base = static_cast<char*>(workspace);
  bf16_t* ln = reinterpret_cast<bf16_t*>(base + w.ln);
  bf16_t* q = reinterpret_cast<bf16_t*>(base + w.q);
  bf16_t* k = reinterpret_cast<bf16_t*>(base + w.k);
  bf16_t* vt = reinterpret_cast<bf16_t*>(base + w.vt);
  bf16_t* ctx = reinterpret_cast<bf16_t*>(base + w.ctx);
  bf16_t* xa = reinterpret_cast<bf16_t*>(base + w.xa);
  bf16_t* xb = reinterpret_cast<bf16_t*>(base + w.xb);
  bf16_t* hidden = reinterpret_cast<bf16_t*>(base + w.hidden);

  const int64_t T = batch * seq_len;
  const int64_t D = d_model, F = ffn_dim, H = num_heads;
  const int cus = device_cus();
  const float scale = 1.0f / sqrtf(static_cast<float>(D / H));
  auto W = [&](int64_t layer, int idx) { return static_cast<const bf16_t*>(weights[layer * 12 + idx]); };
  // Tile-packed copies of the four projection weights (qkv, out, ffn_in,
  // ffn_out) follow the 12 * num_layers + 2 pointers when asked for.
  const bool packed = (flags & ENC_FWD_PACKED_WEIGHTS) != 0;
  auto P = [&](int64_t layer, int which) {
    return static_cast<const bf16_t*>(weights[12 * num_layers + 2 + 4 * layer + which]);
  };
  auto use_packed = [&](enc::GemmEpilogueArgs& a, int64_t layer, int which, int64_t n, int64_t k) {
    if (!packed) return;
    a.w_packed = P(layer, which);
    a.w_packed_rows = enc::gemm_prepack_rows(n, k);
  };

  // Narrow models with up to 8192 tokens run the block tail (out_proj ..
  // ffn_out, and the next layer's norm1) as one kernel, whose 16-byte loads
  // need 16-byte aligned weights (all but the QKV projection's).
  // (With more tokens the four launches win: the fused kernel's one workgroup
  // per CU cannot hide its per-slab latency; measured on MI355X.)
  bool tail_fused = enc::block_tail_supported(D, F) && T <= 8192 && !enc::gemm_has_split_tail(T, D, D, cus) &&
                    !enc::gemm_has_split_tail(T, F, D, cus) && !enc::gemm_has_split_tail(T, D, F, cus);
  for (int64_t layer = 0; tail_fused && layer < num_layers; ++layer)
    for (int idx = 0; idx < 12; ++idx)
      tail_fused = tail_fused && (idx == 2 || idx == 3 || reinterpret_cast<uintptr_t>(W(layer, idx)) % 16 == 0);

  const bf16_t* cur = static_cast<const bf16_t*>(x);
  hipError_t e = hipSuccess;
  bool ln_ready = false;  // the fused tail already wrote this layer's norm1
  for (int64_t layer = 0; layer < num_layers; ++layer) {
    bf16_t* x_attn = (cur == xa) ? xb : xa;  // residual stream after attention
    // norm1
    if (!ln_ready) {
      e = enc::layernorm_bf16(cur, W(layer, 0), W(layer, 1), ln, T, D, eps, nullptr, st);
      if (e != hipSuccess) return fail_hip(e, "encoder norm1");
    }
    ln_ready = false;
    // packed QKV, head-major
    enc::GemmEpilogueArgs qa;
    qa.bias = W(layer, 3);
    qa.q = q;
    qa.k = k;
    qa.v_t = vt;
    qa.seq_len = static_cast<int>(seq_len);
    qa.num_heads = static_cast<int>(H);
    qa.head_dim = static_cast<int>(D / H);
    qa.d_model = static_cast<int>(D);
    qa.ld_vt = static_cast<int>(enc::vt_stride(seq_len));
    use_packed(qa, layer, 0, 3 * D, D);
    e = enc::gemm_bf16(ln, W(layer, 2), T, 3 * D, D, enc::kEpiQkvHeadMajor, qa, cus, st);
    if (e != hipSuccess) return fail_hip(e, "encoder qkv");
    // attention -> context [T, D]
    auto attention = exact ? enc::attention_fwd_bf16 : enc::flash_attention_fwd_bf16;
    e = attention(q, k, vt, ctx, static_cast<int>(batch), static_cast<int>(H), static_cast<int>(seq_len),
                  static_cast<int>(D / H), scale, causal != 0, kv_len, key_mask, st);
    if (e != hipSuccess) return fail_hip(e, "encoder attention");
    if (tail_fused) {
      // out_proj .. ffn_out in one launch (narrow models), same arithmetic
      enc::BlockTailArgs ta;
      ta.ctx = ctx;
      ta.x = cur;
      ta.wo = W(layer, 4);
      ta.bo = W(layer, 5);
      ta.g2 = W(layer, 6);
      ta.be2 = W(layer, 7);
      ta.w1 = W(layer, 8);
      ta.b1 = W(layer, 9);
      ta.w2 = W(layer, 10);
      ta.b2 = W(layer, 11);
      ta.out = (!final_norm && layer == num_layers - 1) ? static_cast<bf16_t*>(out) : x_attn;
      ta.row_mask = row_mask;
      if (layer + 1 < num_layers) {  // the next layer's norm1 comes with the tail
        ta.g1n = W(layer + 1, 0);
        ta.be1n = W(layer + 1, 1);
        ta.ln_out = ln;
        ln_ready = true;
      }
      e = enc::block_tail_bf16(ta, T, D, F, eps, cus, st);
      if (e != hipSuccess) return fail_hip(e, "encoder block tail");
      cur = ta.out;
      continue;
    }
    // out_proj + residual; padded rows keep the residual (attention output is 0 there)
    enc::GemmEpilogueArgs oa;
    oa.bias = W(layer, 5);
    oa.residual = cur;
    oa.row_mask = row_mask;
    oa.out = x_attn;
    use_packed(oa, layer, 1, D, D);
    e = enc::gemm_bf16(ctx, W(layer, 4), T, D, D, enc::kEpiResidualKeep, oa, cus, st);
    if (e != hipSuccess) return fail_hip(e, "encoder out_proj");
    // norm2
    e = enc::layernorm_bf16(x_attn, W(layer, 6), W(layer, 7), ln, T, D, eps, nullptr, st);
    if (e != hipSuccess) return fail_hip(e, "encoder norm2");
    // ffn_in + exact GELU, then ffn_out + residual; padded rows are zeroed
    // (block output masked_fill)
    bf16_t* x_next = (!final_norm && layer == num_layers - 1) ? static_cast<bf16_t*>(out) : (x_attn == xa) ? xb : xa;
    const char* stage = "";
    e = ffn_block(ln, W(layer, 8), W(layer, 9), W(layer, 10), W(layer, 11), x_attn, x_next, hidden, T, D, F, row_mask,
                  packed ? P(layer, 2) : nullptr, packed ? P(layer, 3) : nullptr, cus, st, &stage);
    if (e != hipSuccess) return fail_hip(e, std::string("encoder ") + stage);
    cur = x_next;
  }
  if (!final_norm) return ok();  // out holds the last block's output
  e = enc::layernorm_bf16(cur, static_cast<const bf16_t*>(weights[12 * num_layers]),
                          static_cast<const bf16_t*>(weights[12 * num_layers + 1]), static_cast<bf16_t*>(out), T, D,
                          eps, row_mask, st);
  if (e != hipSuccess) return fail_hip(e, "encoder final_norm");
  return ok();
}


}  // namespace

extern "C" {

int enc_version(void) { return (1 << 16) | 1; }

const char* enc_last_error(void) { return g_last_error.c_str(); }

int enc_linear_order_register(int32_t device, int64_t rows, int64_t out_features, int64_t in_features,
                              int32_t first_tile_row, int32_t tile_rows, int32_t tile_cols, const uint16_t* split) {
  if (device < 0) return fail(ENC_ERR_INVALID, "linear_order_register: device must be >= 0");
  if (enc::gemm_order_register(device, rows, out_features, in_features, first_tile_row, tile_rows, tile_cols,
                               split) != 0)
    return fail(ENC_ERR_INVALID,
                "linear_order_register: the table does not fit the shape (out_features % 256 == 0, "
                "tile_cols == out_features / 256, at most 1024 entries, tiles covering the last rows, "
                "split points multiples of 32 below in_features)");
  return ok();
}

int enc_linear_order_clear(void) {
  enc::gemm_order_clear();
  return ok();
}

int enc_debug_gelu_table(int32_t ready, int32_t entry, int32_t value, void* stream) {
  if (ready > 1 || entry > 65535 || value > 65535 || value < -1 || (entry < 0 && value != -1))
    return fail(ENC_ERR_INVALID, "debug_gelu_table: ready in {-1, 0, 1}, entry in [-1, 65535], value in [-1, 65535]");
  hipError_t e = enc::gemm_debug_gelu_table(ready, entry, value, static_cast<hipStream_t>(stream));
  if (e != hipSuccess) return fail_hip(e, "debug_gelu_table launch");
  return ok();
}

int enc_layernorm_bf16(const void* x, const void* gamma, const void* beta, void* y, int64_t rows,
                       int64_t width, float eps, const uint8_t* row_mask, void* stream) {
  if (rows < 0 || width <= 0) return fail(ENC_ERR_INVALID, "layernorm: rows must be >= 0 and width > 0");
  if (rows == 0) return ok();
  if (!x || !gamma || !beta || !y) return fail(ENC_ERR_INVALID, "layernorm: null tensor pointer");
  if (!enc::layernorm_supported(width))
    return fail(ENC_ERR_UNSUPPORTED, "layernorm: width must be a power of two in [32, 4096]");
  if (!(eps > 0.f)) return fail(ENC_ERR_INVALID, "layernorm: eps must be positive");
  hipError_t e = enc::layernorm_bf16(static_cast<const enc::bf16_t*>(x), static_cast<const enc::bf16_t*>(gamma),
                                     static_cast<const enc::bf16_t*>(beta), static_cast<enc::bf16_t*>(y), rows,
                                     width, eps, row_mask, static_cast<hipStream_t>(stream));
  if (e != hipSuccess) return fail_hip(e, "layernorm launch");
  return ok();
}

}  // extern "C"

namespace {

int linear_entry(const void* a, const void* weight, const void* packed_weight, const void* bias,
                 const void* residual, void* out, int64_t rows, int64_t out_features, int64_t in_features,
                 int32_t epilogue, const uint8_t* row_mask, void* stream) {
  if (epilogue < ENC_EPI_BIAS || epilogue > ENC_EPI_BIAS_RESIDUAL_ZERO)
    return fail(ENC_ERR_INVALID, "linear: unknown epilogue " + std::to_string(epilogue));
  if (rows < 0 || out_features <= 0 || in_features <= 0)
    return fail(ENC_ERR_INVALID, "linear: rows must be >= 0, features > 0");
  if (rows == 0) return ok();
  if (!a || !weight || !bias || !out) return fail(ENC_ERR_INVALID, "linear: null tensor pointer");
  const bool needs_res = epilogue == ENC_EPI_BIAS_RESIDUAL_KEEP || epilogue == ENC_EPI_BIAS_RESIDUAL_ZERO;
  if (needs_res && !residual) return fail(ENC_ERR_INVALID, "linear: residual epilogue needs a residual");
  if (!enc::gemm_supported(rows, out_features, in_features))
    return fail(ENC_ERR_UNSUPPORTED, "linear: in_features and out_features must be multiples of 32 (got " +
                                         std::to_string(in_features) + ", " + std::to_string(out_features) + ")");
  enc::GemmEpilogueArgs ep;
  ep.bias = static_cast<const enc::bf16_t*>(bias);
  ep.residual = static_cast<const enc::bf16_t*>(residual);
  ep.row_mask = row_mask;
  ep.out = static_cast<enc::bf16_t*>(out);
  if (packed_weight != nullptr) {
    ep.w_packed = static_cast<const enc::bf16_t*>(packed_weight);
    ep.w_packed_rows = enc::gemm_prepack_rows(out_features, in_features);
    if (ep.w_packed_rows == 0)
      return fail(ENC_ERR_UNSUPPORTED, "linear: a packed weight needs out_features % 128 == 0 (got " +
                                           std::to_string(out_features) + ")");
  }
  hipError_t e = enc::gemm_bf16(static_cast<const enc::bf16_t*>(a), static_cast<const enc::bf16_t*>(weight), rows,
                                out_features, in_features, epilogue, ep, device_cus(),
                                static_cast<hipStream_t>(stream));
  if (e != hipSuccess) return fail_hip(e, "linear launch");
  return ok();
}

}  // namespace

extern "C" {

int enc_linear_bf16(const void* a, const void* weight, const void* bias, const void* residual,
                    void* out, int64_t rows, int64_t out_features, int64_t in_features,
                    int32_t epilogue, const uint8_t* row_mask, void* stream) {
  return linear_entry(a, weight, nullptr, bias, residual, out, rows, out_features, in_features, epilogue, row_mask,
                      stream);
}

int enc_prepack_weight_bf16(const void* weight, void* packed, int64_t out_features, int64_t in_features,
                            void* stream) {
  if (out_features <= 0 || in_features <= 0) return fail(ENC_ERR_INVALID, "prepack: features must be > 0");
  if (!weight || !packed) return fail(ENC_ERR_INVALID, "prepack: null tensor pointer");
  if (weight == packed) return fail(ENC_ERR_INVALID, "prepack: packed must not alias weight");
  if (enc::gemm_prepack_rows(out_features, in_features) == 0)
    return fail(ENC_ERR_UNSUPPORTED, "prepack: out_features must be a multiple of 128 and in_features of 32 (got " +
                                         std::to_string(out_features) + " x " + std::to_string(in_features) + ")");
  if (out_features * in_features > (int64_t(1) << 31))
    return fail(ENC_ERR_UNSUPPORTED, "prepack: at most 2^31 elements");
  if (reinterpret_cast<uintptr_t>(weight) % 16 != 0 || reinterpret_cast<uintptr_t>(packed) % 16 != 0)
    return fail(ENC_ERR_INVALID, "prepack: weight and packed must be 16-byte aligned");
  hipError_t e = enc::gemm_prepack_weight(static_cast<const enc::bf16_t*>(weight), static_cast<enc::bf16_t*>(packed),
                                          out_features, in_features, static_cast<hipStream_t>(stream));
  if (e != hipSuccess) return fail_hip(e, "prepack launch");
  return ok();
}

int enc_linear_prepacked_bf16(const void* a, const void* weight, const void* packed_weight, const void* bias,
                              const void* residual, void* out, int64_t rows, int64_t out_features,
                              int64_t in_features, int32_t epilogue, const uint8_t* row_mask, void* stream) {
  if (!packed_weight) return fail(ENC_ERR_INVALID, "linear: null packed weight");
  return linear_entry(a, weight, packed_weight, bias, residual, out, rows, out_features, in_features, epilogue,
                      row_mask, stream);
}

int enc_ffn_fused_bf16(const void* h, const void* w_in, const void* b_in, const void* w_out, const void* b_out,
                       const void* residual, void* out, void* hidden, int64_t rows, int64_t d_model,
                       int64_t ffn_dim, const uint8_t* row_mask, void* stream) {
  if (rows < 0 || d_model <= 0 || ffn_dim <= 0) return fail(ENC_ERR_INVALID, "ffn: rows must be >= 0, widths > 0");
  if (rows == 0) return ok();
  if (!h || !w_in || !b_in || !w_out || !b_out || !residual || !out || !hidden)
    return fail(ENC_ERR_INVALID, "ffn: null tensor pointer");
  if (!enc::gemm_supported(rows, ffn_dim, d_model) || !enc::gemm_supported(rows, d_model, ffn_dim))
    return fail(ENC_ERR_UNSUPPORTED, "ffn: d_model and ffn_dim must be multiples of 32 (got " +
                                         std::to_string(d_model) + ", " + std::to_string(ffn_dim) + ")");
  // hidden is written by the first product and read by the second
  auto span_overlaps = [](const void* a, int64_t a_bytes, const void* b, int64_t b_bytes) {
    const char* pa = static_cast<const char*>(a);
    const char* pb = static_cast<const char*>(b);
    return pa < pb + b_bytes && pb < pa + a_bytes;
  };
  const int64_t hidden_bytes = rows * ffn_dim * 2, act_bytes = rows * d_model * 2;
  if (span_overlaps(hidden, hidden_bytes, h, act_bytes) || span_overlaps(hidden, hidden_bytes, out, act_bytes) ||
      span_overlaps(hidden, hidden_bytes, residual, act_bytes))
    return fail(ENC_ERR_INVALID, "ffn: hidden must not overlap h, residual or out");
  const char* stage = "";
  hipError_t e = ffn_block(static_cast<const enc::bf16_t*>(h), static_cast<const enc::bf16_t*>(w_in),
                           static_cast<const enc::bf16_t*>(b_in), static_cast<const enc::bf16_t*>(w_out),
                           static_cast<const enc::bf16_t*>(b_out), static_cast<const enc::bf16_t*>(residual),
                           static_cast<enc::bf16_t*>(out), static_cast<enc::bf16_t*>(hidden), rows, d_model, ffn_dim,
                           row_mask, nullptr, nullptr, device_cus(), static_cast<hipStream_t>(stream), &stage);
  if (e != hipSuccess) return fail_hip(e, std::string("ffn ") + stage);
  return ok();
}

int enc_qkv_proj_bf16(const void* x, const void* weight, const void* bias, void* q, void* k, void* v_t,
                      int64_t batch, int64_t seq_len, int64_t d_model, int64_t num_heads, void* stream) {
  if (batch < 0 || seq_len < 0 || d_model <= 0 || num_heads <= 0)
    return fail(ENC_ERR_INVALID, "qkv: bad shape");
  if (batch == 0 || seq_len == 0) return ok();
  if (!x || !weight || !bias || !q || !k || !v_t) return fail(ENC_ERR_INVALID, "qkv: null tensor pointer");
  if (d_model % num_heads != 0) return fail(ENC_ERR_INVALID, "qkv: d_model must be divisible by num_heads");
  const int64_t M = batch * seq_len;
  if (!enc::gemm_supported(M, 3 * d_model, d_model))
    return fail(ENC_ERR_UNSUPPORTED, "qkv: d_model must be a multiple of 32");
  enc::GemmEpilogueArgs ep;
  ep.bias = static_cast<const enc::bf16_t*>(bias);
  ep.q = static_cast<enc::bf16_t*>(q);
  ep.k = static_cast<enc::bf16_t*>(k);
  ep.v_t = static_cast<enc::bf16_t*>(v_t);
  ep.seq_len = static_cast<int>(seq_len);
  ep.num_heads = static_cast<int>(num_heads);
  ep.head_dim = static_cast<int>(d_model / num_heads);
  ep.d_model = static_cast<int>(d_model);
  ep.ld_vt = static_cast<int>(enc::vt_stride(seq_len));
  hipError_t e = enc::gemm_bf16(static_cast<const enc::bf16_t*>(x), static_cast<const enc::bf16_t*>(weight), M,
                                3 * d_model, d_model, enc::kEpiQkvHeadMajor, ep, device_cus(),
                                static_cast<hipStream_t>(stream));
  if (e != hipSuccess) return fail_hip(e, "qkv launch");
  return ok();
}

namespace {

int attention_entry(bool exact, const void* q, const void* k, const void* v_t, void* context, int64_t batch,
                    int64_t num_heads, int64_t seq_len, int64_t head_dim, float scale, int32_t causal,
                    const int32_t* kv_len, const uint8_t* key_mask, void* stream) {
  if (batch < 0 || num_heads <= 0 || seq_len < 0 || head_dim <= 0)
    return fail(ENC_ERR_INVALID, "attention: bad shape");
  if (batch == 0 || seq_len == 0) return ok();
  if (!q || !k || !v_t || !context) return fail(ENC_ERR_INVALID, "attention: null tensor pointer");
  if (exact ? !(head_dim == 8 || head_dim == 32 || head_dim == 64 || head_dim == 128 || head_dim == 256)
            : head_dim != 64)
    return fail(ENC_ERR_UNSUPPORTED, exact ? "attention: head_dim must be 8, 32, 64, 128 or 256"
                                           : "online attention: head_dim must be 64");
  if (kv_len && key_mask) return fail(ENC_ERR_INVALID, "attention: pass kv_len or key_mask, not both");
  if (!(scale > 0.f)) return fail(ENC_ERR_INVALID, "attention: scale must be positive");
  if (exact && !enc::attention_seq_supported(seq_len, head_dim))
    return fail(ENC_ERR_UNSUPPORTED,
                "attention: seq_len above 2048 must be a multiple of 4, and one head's keys under 4 GiB");
  if (seq_len >= (int64_t(1) << 30) || batch * num_heads * ((seq_len + 31) / 32) >= (int64_t(1) << 31))
    return fail(ENC_ERR_UNSUPPORTED, "attention: grid too large");
  auto fn = exact ? enc::attention_fwd_bf16 : enc::flash_attention_fwd_bf16;
  hipError_t e = fn(static_cast<const enc::bf16_t*>(q), static_cast<const enc::bf16_t*>(k),
                    static_cast<const enc::bf16_t*>(v_t), static_cast<enc::bf16_t*>(context),
                    static_cast<int>(batch), static_cast<int>(num_heads), static_cast<int>(seq_len),
                    static_cast<int>(head_dim), scale, causal != 0, kv_len, key_mask,
                    static_cast<hipStream_t>(stream));
  if (e != hipSuccess) return fail_hip(e, "attention launch");
  return ok();
}

}  // namespace

int enc_attention_fwd_bf16(const void* q, const void* k, const void* v_t, void* context, int64_t batch,
                           int64_t num_heads, int64_t seq_len, int64_t head_dim, float scale, int32_t causal,
                           const int32_t* kv_len, const uint8_t* key_mask, void* stream) {
  return attention_entry(true, q, k, v_t, context, batch, num_heads, seq_len, head_dim, scale, causal, kv_len,
                         key_mask, stream);
}

int enc_attention_online_fwd_bf16(const void* q, const void* k, const void* v_t, void* context, int64_t batch,
                                  int64_t num_heads, int64_t seq_len, int64_t head_dim, float scale,
                                  int32_t causal, const int32_t* kv_len, const uint8_t* key_mask, void* stream) {
  return attention_entry(false, q, k, v_t, context, batch, num_heads, seq_len, head_dim, scale, causal, kv_len,
                         key_mask, stream);
}

int enc_selfcheck_expf(uint32_t lo_bits, uint32_t hi_bits, uint32_t* mismatches, void* stream) {
  if (!mismatches) return fail(ENC_ERR_INVALID, "selfcheck_expf: null counter");
  if (hi_bits < lo_bits) return fail(ENC_ERR_INVALID, "selfcheck_expf: empty range");
  hipError_t e = enc::expf_selfcheck(lo_bits, hi_bits, mismatches, static_cast<hipStream_t>(stream));
  if (e != hipSuccess) return fail_hip(e, "selfcheck_expf launch");
  return ok();
}

int enc_mask_lengths(const uint8_t* mask, int64_t batch, int64_t seq_len, int32_t* kv_len, void* stream) {
  if (batch < 0 || seq_len < 0) return fail(ENC_ERR_INVALID, "mask_lengths: bad shape");
  if (batch == 0) return ok();
  if (!mask || !kv_len) return fail(ENC_ERR_INVALID, "mask_lengths: null pointer");
  hipError_t e = enc::mask_lengths(mask, batch, seq_len, kv_len, static_cast<hipStream_t>(stream));
  if (e != hipSuccess) return fail_hip(e, "mask_lengths launch");
  return ok();
}

int64_t enc_encoder_workspace_bytes(int64_t batch, int64_t seq_len, int64_t d_model, int64_t num_heads,
                                    int64_t ffn_dim) {
  if (!shape_ok(batch) || !shape_ok(seq_len) || !shape_ok(d_model) || !shape_ok(num_heads) || !shape_ok(ffn_dim) ||
      d_model % num_heads != 0)
    return -1;
  return plan_workspace(batch, seq_len, d_model, num_heads, ffn_dim).total;
}

int enc_encoder_forward_bf16(const void* x, void* out, void* workspace, int64_t workspace_bytes,
                             const void* const* weights, int64_t batch, int64_t seq_len, int64_t d_model,
                             int64_t num_heads, int64_t ffn_dim, int64_t num_layers, float eps, int32_t causal,
                             const int32_t* kv_len, const uint8_t* key_mask, const uint8_t* row_mask,
                             int32_t flags, void* stream) {
  EncoderWorkspace w{};
  int rc = check_encoder_call(x, out, weights, batch, seq_len, d_model, num_heads, ffn_dim, num_layers, eps, kv_len,
                              key_mask, flags, &w);
  if (rc != ENC_OK) return rc;
  if (!workspace) return fail(ENC_ERR_INVALID, "encoder: null workspace");
  if (workspace_bytes < w.total)
    return fail(ENC_ERR_INVALID, "encoder: workspace too small (" + std::to_string(workspace_bytes) + " < " +
                                     std::to_string(w.total) + ")");
  return run_encoder_forward(x, out, workspace, w, weights, batch, seq_len, d_model, num_heads, ffn_dim, num_layers,
                             eps, causal, kv_len, key_mask, row_mask, flags, stream);
}

int enc_encoder_forward_bf16_noalloc(const void* x, void* out, const void* const* weights, int64_t batch,
                                     int64_t seq_len, int64_t d_model, int64_t num_heads, int64_t ffn_dim,
                                     int64_t num_layers, float eps, int32_t causal, const int32_t* kv_len,
                                     const uint8_t* key_mask, const uint8_t* row_mask, int32_t flags,
                                     void* stream) {
  EncoderWorkspace w{};
  int rc = check_encoder_call(x, out, weights, batch, seq_len, d_model, num_heads, ffn_dim, num_layers, eps, kv_len,
                              key_mask, flags, &w);
  if (rc != ENC_OK) return rc;
  if (w.total > kScratchBytes)
    return fail(ENC_ERR_UNSUPPORTED, "encoder noalloc: this shape needs " + std::to_string(w.total) +
                                         " bytes of workspace, above the library's " +
                                         std::to_string(kScratchBytes) + "-byte scratch array");
  void* ws = nullptr;
  rc = scratch_for_current_device(&ws);
  if (rc != ENC_OK) return rc;
  // Every buffer of the workspace is written by a kernel of the forward before
  // any kernel reads it, so the array's contents from an earlier call need no
  // clearing.
  return run_encoder_forward(x, out, ws, w, weights, batch, seq_len, d_model, num_heads, ffn_dim, num_layers, eps,
                             causal, kv_len, key_mask, row_mask, flags, stream);
}

}  // extern "C"
