// Fused elementwise work of a Qwen3 decoder layer around the paged attention.
//
// The reference runs each of these as a chain of ATen kernels (one launch per op): RMSNorm
// (src/mini_infra/model/qwen3.py:55-78: fp32 square, mean, rsqrt, product, cast, weight product),
// the residual adds of Qwen3DecoderLayer.forward (:368-400), q/k RMSNorm + RoPE of
// Qwen3Attention._project_qkv (:182-217) with _rotate_half / _apply_rotary_embedding (:111-145),
// the decode K/V append of _apply_paged_kv_pool (:282-283), and the SwiGLU product of
// Qwen3MLP.forward (:347-355).  Here each group is one launch that keeps the reference's bf16
// rounding points:
//   * RMSNorm:  n = bf16(x * r), y = bf16(w * n), with r = 1 / sqrt(sum(x^2) / N + eps) from an
//     exact sum of squares (fp64) and one rounding to fp32 per step (mi_common.h, rms_inv);
//   * residual: h = bf16(a + b);
//   * RoPE:     y = bf16(bf16(x * cos) + bf16(rotate_half(x) * sin));
//   * SwiGLU:   y = bf16(bf16(silu(g)) * u), silu(g) = g / (1 + exp(-g)) in fp32.
// The one deviation from the ATen chain is that the sum of squares is exact instead of an fp32
// sum in ATen's order, so the result does not depend on how the sum is split over lanes.
//
// All tensors are bf16 with rows of contiguous elements; the kernels are memory-light (a decode
// step moves a few MB), so the point is launch count, not bandwidth.

#include <math.h>

#include "mi_common.h"

namespace mi {
namespace {

constexpr int kThreads = 256;  // 4 wavefronts
constexpr int kWave = 64;

__device__ __forceinline__ float bf16_to_f32(uint16_t b) { return __uint_as_float(static_cast<uint32_t>(b) << 16); }
__device__ __forceinline__ uint16_t f32_to_bf16(float f) { return static_cast<uint16_t>(f32_to_bf16_bits(f)); }

// ------------------------------------------------------------------ RMSNorm (+ residual add)
struct NormArgs {
  uint16_t* out;
  const uint16_t* x;
  const uint16_t* residual;  // may be null
  uint16_t* residual_out;    // written when residual != null
  const uint16_t* weight;
  int64_t rows;
  int32_t hidden;
  float eps;
};

// One wavefront per row; lane l owns 16-byte pieces l, l + 64, ... (kPieces of them).
template <int kPieces>
__global__ __launch_bounds__(kThreads) void rms_norm_kernel(const NormArgs a) {
  const int64_t row = static_cast<int64_t>(blockIdx.x) * (kThreads / kWave) + threadIdx.x / kWave;
  if (row >= a.rows) return;
  const int lane = threadIdx.x % kWave;
  const int pieces = a.hidden / 8;
  const int64_t base = row * a.hidden;
  u32x4 h[kPieces];
  double ss = 0.0;
#pragma unroll
  for (int p = 0; p < kPieces; ++p) {
    const int piece = lane + p * kWave;
    if (piece < pieces) {
      u32x4 v = *reinterpret_cast<const u32x4*>(a.x + base + piece * 8);
      if (a.residual) {
        const u32x4 r = *reinterpret_cast<const u32x4*>(a.residual + base + piece * 8);
#pragma unroll
        for (int j = 0; j < 4; ++j)
          v[j] = pack_bf16x2(bf16_lo(v[j]) + bf16_lo(r[j]), bf16_hi(v[j]) + bf16_hi(r[j]));
        *reinterpret_cast<u32x4*>(a.residual_out + base + piece * 8) = v;
      }
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const double lo = bf16_lo(v[j]), hi = bf16_hi(v[j]);
        ss += lo * lo;
        ss += hi * hi;
      }
      h[p] = v;
    }
  }
  const float r = rms_inv(wave_sum64_f64(ss), static_cast<double>(a.hidden), a.eps);
#pragma unroll
  for (int p = 0; p < kPieces; ++p) {
    const int piece = lane + p * kWave;
    if (piece < pieces) {
      const u32x4 w = *reinterpret_cast<const u32x4*>(a.weight + piece * 8);
      u32x4 o;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const float n_lo = round_bf16(bf16_lo(h[p][j]) * r), n_hi = round_bf16(bf16_hi(h[p][j]) * r);
        o[j] = pack_bf16x2(bf16_lo(w[j]) * n_lo, bf16_hi(w[j]) * n_hi);
      }
      *reinterpret_cast<u32x4*>(a.out + base + piece * 8) = o;
    }
  }
}

// ------------------------------------------------------------ q/k RMSNorm + RoPE (+ append)
struct QkArgs {
  uint16_t* q_out;        // [T, Hq, 128]
  uint16_t* k_out;        // [T, Hkv, 128] (rows form) or null
  uint16_t* v_out;        // [T, Hkv, 128] (rows form) or null
  const uint16_t* q;      // row stride q_stride
  const uint16_t* k;
  const uint16_t* v;
  int64_t q_stride, k_stride, v_stride;
  const uint16_t* q_weight;  // [128]
  const uint16_t* k_weight;  // [128]
  const uint16_t* cos;       // [T, 128]
  const uint16_t* sin;       // [T, 128]
  const int64_t* slot_mapping;  // K/V rows also (or only, without k_out) go to these pool slots; or null
  int64_t slot_stride;
  uint16_t* key_pool;        // [num_slots, Hkv, 128]
  uint16_t* value_pool;
  int64_t num_slots;
  int64_t tokens;
  int32_t q_heads, kv_heads;
  float eps;
};

// One wavefront per (token, head): heads [0, Hq) are query heads, [Hq, Hq + Hkv) key heads
// (which also move their value head).  Lane l owns elements l and l + 64, the two halves that
// rotate_half pairs, so the rotation is lane-local.
__global__ __launch_bounds__(kThreads) void qk_norm_rope_kernel(const QkArgs a) {
  const int heads = a.q_heads + a.kv_heads;
  const int64_t unit = static_cast<int64_t>(blockIdx.x) * (kThreads / kWave) + threadIdx.x / kWave;
  if (unit >= a.tokens * heads) return;
  const int64_t t = unit / heads;
  const int head = static_cast<int>(unit % heads);
  const int lane = threadIdx.x % kWave;
  const bool is_q = head < a.q_heads;
  const int h = is_q ? head : head - a.q_heads;
  int64_t slot = -1;
  if (!is_q && a.slot_mapping) {
    slot = a.slot_mapping[t * a.slot_stride];
    if (slot < 0 || slot >= a.num_slots) slot = -1;
  }
  const uint16_t* src = is_q ? a.q + t * a.q_stride + h * 128 : a.k + t * a.k_stride + h * 128;
  float o0, o1;
  norm_rope_head(src, is_q ? a.q_weight : a.k_weight, a.cos + t * 128, a.sin + t * 128, a.eps, lane, o0, o1);
  if (is_q) {
    uint16_t* dst = a.q_out + (t * a.q_heads + h) * 128;
    dst[lane] = f32_to_bf16(o0);
    dst[lane + 64] = f32_to_bf16(o1);
    return;
  }
  const uint16_t* vs = a.v + t * a.v_stride + h * 128;
  const uint16_t v0 = vs[lane], v1 = vs[lane + 64];
  if (a.k_out) {  // the token's rows
    uint16_t* kd = a.k_out + (t * a.kv_heads + h) * 128;
    uint16_t* vd = a.v_out + (t * a.kv_heads + h) * 128;
    kd[lane] = f32_to_bf16(o0);
    kd[lane + 64] = f32_to_bf16(o1);
    vd[lane] = v0;
    vd[lane + 64] = v1;
  }
  if (slot >= 0) {  // and / or its pool slot
    uint16_t* kd = a.key_pool + (slot * a.kv_heads + h) * 128;
    uint16_t* vd = a.value_pool + (slot * a.kv_heads + h) * 128;
    kd[lane] = f32_to_bf16(o0);
    kd[lane + 64] = f32_to_bf16(o1);
    vd[lane] = v0;
    vd[lane + 64] = v1;
  }
}

// Vector form, for 16-byte aligned rows: 16 lanes (one DPP row) per (token, head), lane j holding
// elements [8 j, 8 j + 8) (16-byte loads and stores), a wavefront four heads of one token.  The sum
// of squares is exact in fp64 in any order, so the 16-lane reduction gives the scalar form's bits;
// rotate_half pairs lane j with lane j ^ 8 (a rotation of the row by 8).  Every lane of a wavefront
// that starts runs the cross-lane steps.
__global__ __launch_bounds__(kThreads) void qk_norm_rope_vec_kernel(const QkArgs a) {
  const int heads = a.q_heads + a.kv_heads;
  const int quads = (heads + 3) / 4;
  const int64_t wave = static_cast<int64_t>(blockIdx.x) * (kThreads / kWave) + threadIdx.x / kWave;
  if (wave >= a.tokens * quads) return;  // uniform per wavefront
  const int lane = threadIdx.x % kWave;
  const int j = lane & 15;
  const int64_t t = wave / quads;
  const int head_raw = static_cast<int>(wave % quads) * 4 + (lane >> 4);
  const bool live = head_raw < heads;  // uniform per 16-lane group
  const int head = live ? head_raw : heads - 1;
  const bool is_q = head < a.q_heads;
  const int h = is_q ? head : head - a.q_heads;
  const uint16_t* src = (is_q ? a.q + t * a.q_stride : a.k + t * a.k_stride) + h * 128 + 8 * j;
  const u32x4 x = *reinterpret_cast<const u32x4*>(src);
  const u32x4 w = *reinterpret_cast<const u32x4*>((is_q ? a.q_weight : a.k_weight) + 8 * j);
  const u32x4 cs = *reinterpret_cast<const u32x4*>(a.cos + t * 128 + 8 * j);
  const u32x4 sn = *reinterpret_cast<const u32x4*>(a.sin + t * 128 + 8 * j);
  float xf[8];
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    xf[2 * e] = bf16_lo(x[e]);
    xf[2 * e + 1] = bf16_hi(x[e]);
  }
  double sq = 0.0;
#pragma unroll
  for (int e = 0; e < 8; ++e) sq += static_cast<double>(xf[e]) * xf[e];
  const float r = rms_inv(dpp_sum16_f64(sq), 128.0, a.eps);
  float y[8];
  u32x4 yb;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    y[2 * e] = round_bf16(bf16_lo(w[e]) * round_bf16(xf[2 * e] * r));
    y[2 * e + 1] = round_bf16(bf16_hi(w[e]) * round_bf16(xf[2 * e + 1] * r));
    yb[e] = pack_bf16x2(y[2 * e], y[2 * e + 1]);
  }
  u32x4 pb;  // the rotate_half partner's normalised values (elements 64 apart): DPP row_ror:8 = lane ^ 8
#pragma unroll
  for (int e = 0; e < 4; ++e)
    pb[e] = static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(yb[e]), 0x128, 0xf, 0xf, false));
  const float sign = j < 8 ? -1.0f : 1.0f;  // element e < 64: y cos - y[e + 64] sin; else y cos + y[e - 64] sin
  u32x4 o;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const float o0 = round_bf16(round_bf16(y[2 * e] * bf16_lo(cs[e])) + round_bf16(sign * bf16_lo(pb[e]) * bf16_lo(sn[e])));
    const float o1 =
        round_bf16(round_bf16(y[2 * e + 1] * bf16_hi(cs[e])) + round_bf16(sign * bf16_hi(pb[e]) * bf16_hi(sn[e])));
    o[e] = pack_bf16x2(o0, o1);
  }
  if (!live) return;
  if (is_q) {
    *reinterpret_cast<u32x4*>(a.q_out + (t * a.q_heads + h) * 128 + 8 * j) = o;
    return;
  }
  int64_t slot = -1;
  if (a.slot_mapping) {
    slot = a.slot_mapping[t * a.slot_stride];
    if (slot < 0 || slot >= a.num_slots) slot = -1;
  }
  const u32x4 v = *reinterpret_cast<const u32x4*>(a.v + t * a.v_stride + h * 128 + 8 * j);
  if (a.k_out) {  // the token's rows
    *reinterpret_cast<u32x4*>(a.k_out + (t * a.kv_heads + h) * 128 + 8 * j) = o;
    *reinterpret_cast<u32x4*>(a.v_out + (t * a.kv_heads + h) * 128 + 8 * j) = v;
  }
  if (slot >= 0) {  // and / or its pool slot
    *reinterpret_cast<u32x4*>(a.key_pool + (slot * a.kv_heads + h) * 128 + 8 * j) = o;
    *reinterpret_cast<u32x4*>(a.value_pool + (slot * a.kv_heads + h) * 128 + 8 * j) = v;
  }
}

// ------------------------------------------------------------------------------ SwiGLU
struct SiluArgs {
  uint16_t* out;
  const uint16_t* gate;
  const uint16_t* up;
  int64_t rows;
  int64_t gate_stride, up_stride, out_stride;
  int32_t pieces_per_row;  // cols / 8
};

__device__ __forceinline__ float silu_bf16(float g) { return round_bf16(g / (1.0f + expf(-g))); }

__global__ __launch_bounds__(kThreads) void silu_mul_kernel(const SiluArgs a) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
  if (i >= a.rows * a.pieces_per_row) return;
  const int64_t row = i / a.pieces_per_row;
  const int64_t col = (i % a.pieces_per_row) * 8;
  const u32x4 g = *reinterpret_cast<const u32x4*>(a.gate + row * a.gate_stride + col);
  const u32x4 u = *reinterpret_cast<const u32x4*>(a.up + row * a.up_stride + col);
  u32x4 o;
#pragma unroll
  for (int j = 0; j < 4; ++j)
    o[j] = pack_bf16x2(silu_bf16(bf16_lo(g[j])) * bf16_lo(u[j]), silu_bf16(bf16_hi(g[j])) * bf16_hi(u[j]));
  *reinterpret_cast<u32x4*>(a.out + row * a.out_stride + col) = o;
}

bool aligned(const void* p) { return p == nullptr || aligned16(p); }

}  // namespace
}  // namespace mi

extern "C" int32_t mi_rms_norm(void* out, const void* x, const void* residual, void* residual_out,
                               const void* weight, int64_t rows, int32_t hidden, float eps, void* stream) {
  using namespace mi;
  if (rows < 0 || hidden <= 0) return fail(MI_ERR_INVALID_ARGUMENT, "mi_rms_norm: bad size (rows %lld, hidden %d)",
                                           static_cast<long long>(rows), hidden);
  if (rows == 0) return ok();
  if (!out || !x || !weight || (residual && !residual_out))
    return fail(MI_ERR_INVALID_ARGUMENT, "mi_rms_norm: null pointer argument");
  if (hidden % 8 != 0 || hidden > 8 * 64 * 8)
    return fail(MI_ERR_UNSUPPORTED, "mi_rms_norm: hidden %d must be a multiple of 8 and at most 4096", hidden);
  if (!aligned(out) || !aligned(x) || !aligned(residual) || !aligned(residual_out) || !aligned(weight))
    return fail(MI_ERR_INVALID_ARGUMENT, "mi_rms_norm: pointers must be 16-byte aligned");
  NormArgs a{static_cast<uint16_t*>(out), static_cast<const uint16_t*>(x), static_cast<const uint16_t*>(residual),
             static_cast<uint16_t*>(residual_out), static_cast<const uint16_t*>(weight), rows, hidden, eps};
  const int64_t groups = (rows + kThreads / kWave - 1) / (kThreads / kWave);
  if (groups > 0x7fffffff) return fail(MI_ERR_UNSUPPORTED, "mi_rms_norm: too many rows");
  hipStream_t s = as_stream(stream);
  const int pieces = (hidden / 8 + kWave - 1) / kWave;
  if (pieces <= 1)
    rms_norm_kernel<1><<<static_cast<uint32_t>(groups), kThreads, 0, s>>>(a);
  else if (pieces <= 2)
    rms_norm_kernel<2><<<static_cast<uint32_t>(groups), kThreads, 0, s>>>(a);
  else if (pieces <= 4)
    rms_norm_kernel<4><<<static_cast<uint32_t>(groups), kThreads, 0, s>>>(a);
  else
    rms_norm_kernel<8><<<static_cast<uint32_t>(groups), kThreads, 0, s>>>(a);
  return check_launch("mi_rms_norm");
}

extern "C" int32_t mi_qk_norm_rope(void* q_out, void* k_out, void* v_out, const void* q, int64_t q_stride,
                                   const void* k, int64_t k_stride, const void* v, int64_t v_stride,
                                   const void* q_weight, const void* k_weight, const void* cos, const void* sin,
                                   int64_t num_tokens, int32_t num_heads, int32_t num_kv_heads, int32_t head_dim,
                                   float eps, const int64_t* slot_mapping, int64_t slot_stride, void* key_pool,
                                   void* value_pool, int64_t num_slots, void* stream) {
  using namespace mi;
  if (num_tokens < 0 || num_heads <= 0 || num_kv_heads <= 0)
    return fail(MI_ERR_INVALID_ARGUMENT, "mi_qk_norm_rope: bad size");
  if (head_dim != 128) return fail(MI_ERR_UNSUPPORTED, "mi_qk_norm_rope: head_dim %d (only 128)", head_dim);
  if (num_tokens == 0) return ok();
  if (!q_out || !q || !k || !v || !q_weight || !k_weight || !cos || !sin)
    return fail(MI_ERR_INVALID_ARGUMENT, "mi_qk_norm_rope: null pointer argument");
  if (!k_out != !v_out) return fail(MI_ERR_INVALID_ARGUMENT, "mi_qk_norm_rope: give both k_out and v_out or neither");
  if (!slot_mapping && !k_out)
    return fail(MI_ERR_INVALID_ARGUMENT, "mi_qk_norm_rope: give k_out and v_out, slot_mapping and pools, or both");
  if (slot_mapping && (!key_pool || !value_pool || num_slots < 0 || slot_stride <= 0))
    return fail(MI_ERR_INVALID_ARGUMENT, "mi_qk_norm_rope: slot_mapping needs both pools, num_slots and a stride");
  if (q_stride < num_heads * 128 || k_stride < num_kv_heads * 128 || v_stride < num_kv_heads * 128)
    return fail(MI_ERR_INVALID_ARGUMENT, "mi_qk_norm_rope: row strides shorter than a row");
  QkArgs a{static_cast<uint16_t*>(q_out), static_cast<uint16_t*>(k_out), static_cast<uint16_t*>(v_out),
           static_cast<const uint16_t*>(q), static_cast<const uint16_t*>(k), static_cast<const uint16_t*>(v),
           q_stride, k_stride, v_stride, static_cast<const uint16_t*>(q_weight),
           static_cast<const uint16_t*>(k_weight), static_cast<const uint16_t*>(cos),
           static_cast<const uint16_t*>(sin), slot_mapping, slot_stride, static_cast<uint16_t*>(key_pool),
           static_cast<uint16_t*>(value_pool), num_slots, num_tokens, num_heads, num_kv_heads, eps};
  // 16-byte rows everywhere: the vector form (four heads per wavefront); else one head per wavefront.
  const bool vec = aligned16(q_out) && aligned16(q) && aligned16(k) && aligned16(v) && aligned(k_out) &&
                   aligned(v_out) && aligned(key_pool) && aligned(value_pool) && aligned16(q_weight) &&
                   aligned16(k_weight) && aligned16(cos) && aligned16(sin) && q_stride % 8 == 0 &&
                   k_stride % 8 == 0 && v_stride % 8 == 0;
  const int64_t per_token = vec ? (num_heads + num_kv_heads + 3) / 4 : num_heads + num_kv_heads;
  const int64_t groups = (num_tokens * per_token + kThreads / kWave - 1) / (kThreads / kWave);
  if (groups > 0x7fffffff) return fail(MI_ERR_UNSUPPORTED, "mi_qk_norm_rope: too many tokens");
  if (vec)
    qk_norm_rope_vec_kernel<<<static_cast<uint32_t>(groups), kThreads, 0, as_stream(stream)>>>(a);
  else
    qk_norm_rope_kernel<<<static_cast<uint32_t>(groups), kThreads, 0, as_stream(stream)>>>(a);
  return check_launch("mi_qk_norm_rope");
}

extern "C" int32_t mi_silu_mul(void* out, int64_t out_stride, const void* gate, int64_t gate_stride, const void* up,
                               int64_t up_stride, int64_t rows, int32_t cols, void* stream) {
  using namespace mi;
  if (rows < 0 || cols <= 0) return fail(MI_ERR_INVALID_ARGUMENT, "mi_silu_mul: bad size");
  if (rows == 0) return ok();
  if (!out || !gate || !up) return fail(MI_ERR_INVALID_ARGUMENT, "mi_silu_mul: null pointer argument");
  if (cols % 8 || out_stride % 8 || gate_stride % 8 || up_stride % 8 || !aligned16(out) || !aligned16(gate) ||
      !aligned16(up))
    return fail(MI_ERR_UNSUPPORTED, "mi_silu_mul: columns, strides and pointers must be 16-byte multiples");
  SiluArgs a{static_cast<uint16_t*>(out), static_cast<const uint16_t*>(gate), static_cast<const uint16_t*>(up),
             rows, gate_stride, up_stride, out_stride, cols / 8};
  const int64_t groups = (rows * (cols / 8) + kThreads - 1) / kThreads;
  if (groups > 0x7fffffff) return fail(MI_ERR_UNSUPPORTED, "mi_silu_mul: too many elements");
  silu_mul_kernel<<<static_cast<uint32_t>(groups), kThreads, 0, as_stream(stream)>>>(a);
  return check_launch("mi_silu_mul");
}
