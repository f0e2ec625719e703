// Attention with the reference's rounding points and exactly accumulated sums.
//
// The reference attends with (src/mini_infra/model/qwen3.py:219-255)
//   scores = bf16(Q K^T) * scale          -> bf16 matmul output, then a bf16 product
//   probs  = softmax(scores, fp32).to(bf16)
//   out    = bf16(probs V)
// Each of its sums (the dot products, the softmax denominator, the P V products) is an fp32 sum
// in whatever order ATen's kernels pick, and that order differs between devices, libraries and
// batch shapes, so the last bits of every rounding point depend on it.  The kernels here keep
// the reference's rounding points and make every sum exact instead:
//   s_t  = bf16(bf16(fp32(sum_d q_d k_td)) * scale)       exact dot product, rounded to fp32, bf16
//   m    = max_t s_t
//   e_t  = fp32(exp(fp32(s_t - m)))                       exp evaluated in fp64, rounded once
//   l    = fp32(sum_t e_t)                                exact sum (split_add below)
//   p_t  = bf16(fp32(e_t / l))                            division correctly rounded
//   o_d  = bf16(fp32(sum_t p_t v_td))                     exact sum
// over the visible keys t.  Products of two bf16 values are exact in fp64, and fp64 sums of the
// terms met here are exact or off by far less than the final roundings can see, so the results
// do not depend on how the work is split over lanes, wavefronts or workgroups, nor on the device:
// the oracle computes the same definitions with torch ops and gets the same bits.  That is what
// makes a whole model bit-identical to its oracle, and greedy decoding token-identical (a bf16
// logit tie over a 151,936-token vocabulary is common, so any one-ulp difference anywhere in the
// forward eventually flips a token).
//
// Cost: fp64 arithmetic instead of bf16 / fp32, and two or three passes over the keys (scores and
// their maximum, the denominators, then P V), the scores cached in LDS between them.  These kernels
// serve the model's forward, where attention is latency-bound (small decode batches, prompts of a
// few hundred tokens); the bandwidth kernels (paged_decode_attention.hip,
// chunked_prefill_attention.hip) keep fp32 online softmax for large batches and long prompts.
//
// Decode (q_len 1): one workgroup of 8 wavefronts per (sequence, KV head) serves the G query
// heads of the GQA group; wavefront w takes blocks w, w + 8, ...  Lane 16 r + d holds dims
// [8 d, 8 d + 8) of tokens 4 i + r of a 16-token block (one 16-byte load per lane per i), the
// layout of the bandwidth kernels.  The scores go to LDS as bf16 (exact: they are bf16 values),
// are replaced by the probabilities once m and l are known, and are read back for P V.  A
// context too long for the LDS cache recomputes the scores in each pass instead.  Small batches
// split each sequence's blocks over several workgroups (three launches, merged exactly).
//
// Prefill (chunked, with history from the pool): the dot products and P V on the fp64 matrix
// cores, one workgroup of 4 wavefronts per 16 (query, head) columns of a (row, KV head), the
// wavefronts splitting the keys; the layout is described at the kernel.
#include <algorithm>
#include <math.h>
#include <mutex>

#include "mi_common.h"

namespace mi {
namespace {

constexpr int kHeadDim = 128;
constexpr int kBlockSize = 16;

// ---------------------------------------------------------------- shared arithmetic ---
// The bf16 matmul output (the exact dot product rounded to fp32, then to bf16), times the scale
// with one more bf16 rounding (qwen3.py:243).
__device__ __forceinline__ float exact_score(double dot, float scale) {
  return round_bf16(round_bf16(static_cast<float>(dot)) * scale);
}

// e = fp32(exp(fp32(s - m))): the fp32 difference of two bf16 values, exponential in fp64.
__device__ __forceinline__ float exact_exp(float s, float m) {
  const float d = s - m;
  return static_cast<float>(exp(static_cast<double>(d)));
}

// Order-independent sum of values in [0, 1]: x splits into h, x rounded to a multiple of 2^-32
// ((x + 1.5 * 2^20) - 1.5 * 2^20 in fp64: the sum's ulp is 2^-32), and the remainder x - h.
// The h parts add exactly in fp64 for up to 2^20 terms; the remainders are below 2^-33, so their
// fp64 sum is off by ~2^-77 at most.  The total is fp32(fp64(sum h + sum lo)).
constexpr double kSplit = 1572864.0;
__device__ __forceinline__ void split_add(float e, double& hi, double& lo) {
  const double x = e;
  const double h = (x + kSplit) - kSplit;
  hi += h;
  lo += x - h;
}

// p = bf16(fp32(e / l)): an fp64 quotient of two fp32 values rounds to the correctly rounded
// fp32 quotient (53 >= 2 * 24 + 2 bits).
__device__ __forceinline__ float exact_prob(float e, float l) {
  return round_bf16(static_cast<float>(static_cast<double>(e) / static_cast<double>(l)));
}

__device__ __forceinline__ uint16_t bf16_bits(float f) { return static_cast<uint16_t>(f32_to_bf16_bits(f)); }

__device__ __forceinline__ float wave_max(float v) {
  v = fmaxf(v, dpp_f32<0xB1>(v));
  v = fmaxf(v, dpp_f32<0x4E>(v));
  v = fmaxf(v, dpp_f32<0x141>(v));
  v = fmaxf(v, dpp_f32<0x140>(v));
  return xmax32(xmax16(v));
}

// Eight bf16 values of a 16-byte piece as doubles (exact).
__device__ __forceinline__ void unpack8(const u32x4 v, double (&d)[8]) {
#pragma unroll
  for (int w = 0; w < 4; ++w) {
    const uint32_t x = v[w];
    d[2 * w] = bf16_lo(x);
    d[2 * w + 1] = bf16_hi(x);
  }
}

// ------------------------------------------------------------------------ decode ---
constexpr int kDecWaves = 8;
constexpr int kDecThreads = 64 * kDecWaves;
constexpr int kDecCacheBytes = 128 * 1024;  // score cache (dynamic LDS) of one workgroup, at most
#ifndef MI_EXACT_DECODE_GROUP
#define MI_EXACT_DECODE_GROUP 2
#endif
// Blocks a wavefront loads before using them: MI_EXACT_DECODE_GROUP for GQA groups up to 2, one
// block for larger groups, whose fp64 accumulators leave no registers for more (more spills to
// scratch).
template <int kG>
constexpr int dec_group() {
  return kG <= 2 ? MI_EXACT_DECODE_GROUP : 1;
}

struct ExactDecodeArgs {
  uint16_t* out;
  int64_t out_row;
  const uint16_t* q;       // rotated queries [B, H, 128] (plain form) or raw q projection rows (prologue)
  int64_t q_row, q_head;
  const uint16_t* k_new;   // prologue: raw k / v projection rows of the new tokens; plain form with
  const uint16_t* v_new;   // slot_mapping: their rotated rows, KV head h at h * k_head / v_head
  int64_t k_row, v_row;
  int64_t k_head, v_head;
  const uint16_t* q_weight;
  const uint16_t* k_weight;
  const uint16_t* cos;     // [B, 128]
  const uint16_t* sin;
  float eps;
  const int64_t* slot_mapping;
  int64_t slot_stride;
  int64_t num_slots;
  uint16_t* key_pool;
  uint16_t* value_pool;
  int64_t num_blocks;
  int32_t kv_heads;
  const int64_t* block_tables;
  int64_t bt_stride;
  int32_t max_blocks;
  const int64_t* context_lens;
  int64_t ctx_stride;
  float scale;
  int32_t cache_tokens;    // tokens the LDS score cache holds per head (0: recompute the scores)
};

// LDS of the decode body, carved from the workgroup's dynamic LDS: queries, per-wavefront maxima,
// denominators and outputs, then the score cache [cache_tokens][kG] (bf16 scores, then
// probabilities).
template <int kG, int kWaves>
struct DecodeLds {
  static constexpr int kQ = kG * kHeadDim * 4;
  static constexpr int kM = kWaves * kG * 4;
  static constexpr int kL = kWaves * kG * 2 * 8;
  static constexpr int kO = kWaves * kHeadDim * 8;
  static constexpr int kFixed = (kQ + kM + 7) / 8 * 8 + kL + kO;  // bytes before the cache
};

// Exact decode attention of sequence b, KV head g, by the workgroup's kWaves wavefronts.  kPrologue:
// q / k RMSNorm + RoPE from the raw projection rows and the K/V append.  Plain form: rotated
// queries; with a.slot_mapping set the rows a.k_new / a.v_new (already rotated) are appended first.
template <int kG, bool kPrologue, int kWaves>
__device__ void exact_decode_body(const ExactDecodeArgs& a, const int b, const int g, unsigned char* smem) {
  constexpr int kDecWaves = kWaves;
  constexpr int kDecThreads = 64 * kWaves;
  constexpr int kGrp = dec_group<kG>();
  using Lds = DecodeLds<kG, kWaves>;
  auto s_q = reinterpret_cast<float (*)[kHeadDim]>(smem);
  auto s_m = reinterpret_cast<float (*)[kG]>(smem + Lds::kQ);
  auto s_l = reinterpret_cast<double (*)[kG][2]>(smem + (Lds::kQ + Lds::kM + 7) / 8 * 8);
  auto s_o = reinterpret_cast<double (*)[kHeadDim]>(smem + (Lds::kQ + Lds::kM + 7) / 8 * 8 + Lds::kL);
  uint16_t* s_cache = reinterpret_cast<uint16_t*>(smem + Lds::kFixed);

  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const int dl = lane & 15;
  const int r = lane >> 4;
  const int64_t row_elems = static_cast<int64_t>(a.kv_heads) * kHeadDim;

  if constexpr (kPrologue) {
    // Unit u < kG: query head g kG + u, normalised and rotated into LDS; unit kG: key head g,
    // written with value head g into the sequence's new slot (the K/V append).
    for (int u = w; u <= kG; u += kDecWaves) {
      const bool is_q = u < kG;
      const uint16_t* src = is_q ? a.q + b * a.q_row + (g * kG + u) * kHeadDim : a.k_new + b * a.k_row + g * kHeadDim;
      float o0, o1;
      norm_rope_head(src, is_q ? a.q_weight : a.k_weight, a.cos + b * kHeadDim, a.sin + b * kHeadDim, a.eps, lane,
                     o0, o1);
      if (is_q) {
        s_q[u][lane] = o0;
        s_q[u][lane + 64] = o1;
      } else {
        // Context 0 marks a padding row: no append (as in the plain and mixed forms).
        const int64_t slot = a.slot_mapping[b * a.slot_stride];
        if (slot >= 0 && slot < a.num_slots && a.context_lens[b * a.ctx_stride] > 0) {
          uint16_t* kd = a.key_pool + slot * row_elems + g * kHeadDim;
          uint16_t* vd = a.value_pool + slot * row_elems + g * kHeadDim;
          const uint16_t* vs = a.v_new + b * a.v_row + g * kHeadDim;
          kd[lane] = bf16_bits(o0);
          kd[lane + 64] = bf16_bits(o1);
          vd[lane] = vs[lane];
          vd[lane + 64] = vs[lane + 64];
        }
      }
    }
  } else {
    for (int i = threadIdx.x; i < kG * kHeadDim; i += kDecThreads) {
      const int j = i / kHeadDim, d = i - j * kHeadDim;
      s_q[j][d] = bf16_bits_to_f32(a.q[b * a.q_row + (g * kG + j) * a.q_head + d]);
    }
    if (a.slot_mapping && threadIdx.x < 32) {  // append the token's rotated K and V rows of KV head g
      const int64_t slot = a.slot_mapping[b * a.slot_stride];
      const int64_t ctx = a.context_lens[b * a.ctx_stride];
      if (ctx > 0 && slot >= 0 && slot < a.num_slots) {
        const int piece = (threadIdx.x & 15) * 8;
        const uint16_t* src = threadIdx.x < 16 ? a.k_new + b * a.k_row + g * a.k_head : a.v_new + b * a.v_row + g * a.v_head;
        uint16_t* dst = (threadIdx.x < 16 ? a.key_pool : a.value_pool) + slot * row_elems + g * kHeadDim;
        *reinterpret_cast<uint4*>(dst + piece) = *reinterpret_cast<const uint4*>(src + piece);
      }
    }
  }
  // The barrier also orders the append before this workgroup's loads of the new token's block
  // (no other workgroup reads KV head g of this sequence, and those lines were not read before).
  __syncthreads();

  int64_t n64 = a.context_lens[b * a.ctx_stride];
  n64 = min(n64, static_cast<int64_t>(a.max_blocks) * kBlockSize);
  const int n = n64 > 0 ? static_cast<int>(n64) : 0;
  const int nblk = (n + kBlockSize - 1) / kBlockSize;
  uint16_t* out_b = a.out + b * a.out_row + (g * kG) * kHeadDim;
  if (nblk == 0) {  // empty context: zero rows (uniform)
    if (threadIdx.x < kG * 16) *reinterpret_cast<uint4*>(out_b + 8 * threadIdx.x) = uint4{0, 0, 0, 0};
    return;
  }
  const bool cached = n <= a.cache_tokens;  // uniform
  const int cnt = nblk > w ? (nblk - 1 - w) / kDecWaves + 1 : 0;  // blocks w + 8 i of this wavefront
  const float scale = a.scale;

  // Lane offset inside a block: token 4 i + r (i = 0..3), dims 8 dl .. +8 of KV head g.
  const int64_t lane_off = r * row_elems + g * kHeadDim + 8 * dl;
  // The wavefront's block ids (blocks w + kDecWaves i), fetched with one load, lane i holding id i
  // (i < 64), and broadcast with readlane; ids outside the pool read block 0.  Blocks are then read
  // kGrp at a time, all loads of a group issued before any is used, so a pass costs about one
  // memory round trip per group instead of two per block.
  int64_t lane_id = 0;
  if (lane < cnt) {
    lane_id = a.block_tables[b * a.bt_stride + w + kDecWaves * lane];
    if (lane_id < 0 || lane_id >= a.num_blocks) lane_id = 0;
  }
  auto block_id = [&](int i) -> int64_t {  // i is wave-uniform
    if (i < 64) {
      const uint32_t lo = __builtin_amdgcn_readlane(static_cast<uint32_t>(lane_id), i);
      const uint32_t hi = __builtin_amdgcn_readlane(static_cast<uint32_t>(static_cast<uint64_t>(lane_id) >> 32), i);
      return static_cast<int64_t>((static_cast<uint64_t>(hi) << 32) | lo);
    }
    const int64_t id = a.block_tables[b * a.bt_stride + w + kDecWaves * i];
    return id < 0 || id >= a.num_blocks ? 0 : id;
  };
  // Blocks i0 .. i0 + kGrp - 1 of the wavefront (indices past its last block reload the last
  // one, so every load is unconditional; those are not used).
  auto load_group = [&](const uint16_t* pool, int i0, u32x4 (&buf)[kGrp][4]) {
#pragma unroll
    for (int q = 0; q < kGrp; ++q) {
      const uint16_t* p = pool + block_id(min(i0 + q, cnt - 1)) * kBlockSize * row_elems + lane_off;
#pragma unroll
      for (int t = 0; t < 4; ++t) buf[q][t] = *reinterpret_cast<const u32x4*>(p + 4 * t * row_elems);
    }
  };
  // Scores of the lane row's 4 tokens of block i against the kG queries (equal in the 16 lanes of
  // the row after the butterfly).
  auto block_scores = [&](const u32x4 (&kb)[4], float (&s)[4][kG]) {
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      double kd[8];
      unpack8(kb[t], kd);
#pragma unroll
      for (int j = 0; j < kG; ++j) {
        const float4 q0 = *reinterpret_cast<const float4*>(&s_q[j][8 * dl]);
        const float4 q1 = *reinterpret_cast<const float4*>(&s_q[j][8 * dl + 4]);
        double acc = static_cast<double>(q0.x) * kd[0];
        acc = fma(static_cast<double>(q0.y), kd[1], acc);
        acc = fma(static_cast<double>(q0.z), kd[2], acc);
        acc = fma(static_cast<double>(q0.w), kd[3], acc);
        acc = fma(static_cast<double>(q1.x), kd[4], acc);
        acc = fma(static_cast<double>(q1.y), kd[5], acc);
        acc = fma(static_cast<double>(q1.z), kd[6], acc);
        acc = fma(static_cast<double>(q1.w), kd[7], acc);
        s[t][j] = exact_score(dpp_sum16_f64(acc), scale);
      }
    }
  };

  // ---- pass 1: scores, their maximum per head (and the cache)
  float mloc[kG];
#pragma unroll
  for (int j = 0; j < kG; ++j) mloc[j] = -INFINITY;
  for (int i0 = 0; i0 < cnt; i0 += kGrp) {
    u32x4 kb[kGrp][4];
    load_group(a.key_pool, i0, kb);
#pragma unroll
    for (int q = 0; q < kGrp; ++q) {
      if (i0 + q >= cnt) break;
      float s[4][kG];
      block_scores(kb[q], s);
      const int tok0 = (w + kDecWaves * (i0 + q)) * kBlockSize + r;
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        const int tok = tok0 + 4 * t;
        if (tok < n) {
#pragma unroll
          for (int j = 0; j < kG; ++j) {
            mloc[j] = fmaxf(mloc[j], s[t][j]);
            if (cached && dl == j) s_cache[tok * kG + j] = bf16_bits(s[t][j]);
          }
        }
      }
    }
  }
#pragma unroll
  for (int j = 0; j < kG; ++j) {
    const float mw = wave_max(mloc[j]);
    if (lane == 0) s_m[w][j] = mw;
  }
  __syncthreads();
  float M[kG];
#pragma unroll
  for (int j = 0; j < kG; ++j) {
    float mx = -INFINITY;
#pragma unroll
    for (int v = 0; v < kDecWaves; ++v) mx = fmaxf(mx, s_m[v][j]);
    M[j] = mx;
  }
  // With the scores cached, pass 2 works in LDS only: the first V blocks load meanwhile.
  u32x4 vb[kGrp][4];
  if (cached && cnt > 0) load_group(a.value_pool, 0, vb);

  // ---- pass 2: the softmax denominators
  double hi[kG], lo[kG];
#pragma unroll
  for (int j = 0; j < kG; ++j) hi[j] = lo[j] = 0.0;
  if (cached) {
    for (int tok = threadIdx.x; tok < n; tok += kDecThreads) {
#pragma unroll
      for (int j = 0; j < kG; ++j) split_add(exact_exp(bf16_bits_to_f32(s_cache[tok * kG + j]), M[j]), hi[j], lo[j]);
    }
  } else {
    for (int i0 = 0; i0 < cnt; i0 += kGrp) {
      u32x4 kb[kGrp][4];
      load_group(a.key_pool, i0, kb);
#pragma unroll
      for (int q = 0; q < kGrp; ++q) {
        if (i0 + q >= cnt) break;
        float s[4][kG];
        block_scores(kb[q], s);
        const int tok0 = (w + kDecWaves * (i0 + q)) * kBlockSize + r;
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          if (tok0 + 4 * t < n) {
#pragma unroll
            for (int j = 0; j < kG; ++j)
              if (dl == j) split_add(exact_exp(s[t][j], M[j]), hi[j], lo[j]);
          }
        }
      }
    }
  }
#pragma unroll
  for (int j = 0; j < kG; ++j) {
    const double h = wave_sum64_f64(hi[j]), l = wave_sum64_f64(lo[j]);
    if (lane == 0) {
      s_l[w][j][0] = h;
      s_l[w][j][1] = l;
    }
  }
  __syncthreads();
  float L[kG];
#pragma unroll
  for (int j = 0; j < kG; ++j) {
    double h = 0.0, l = 0.0;
#pragma unroll
    for (int v = 0; v < kDecWaves; ++v) {
      h += s_l[v][j][0];
      l += s_l[v][j][1];
    }
    L[j] = static_cast<float>(h + l);
  }
  if (cached) {  // scores -> probabilities in place
    for (int tok = threadIdx.x; tok < n; tok += kDecThreads) {
#pragma unroll
      for (int j = 0; j < kG; ++j) {
        const float s = bf16_bits_to_f32(s_cache[tok * kG + j]);
        s_cache[tok * kG + j] = bf16_bits(exact_prob(exact_exp(s, M[j]), L[j]));
      }
    }
    __syncthreads();
  }

  // ---- pass 3: P V (lane: tokens 4 i + r of each block, dims 8 dl .. +8)
  double acc[kG][8];
#pragma unroll
  for (int j = 0; j < kG; ++j)
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[j][e] = 0.0;
  for (int i0 = 0; i0 < cnt; i0 += kGrp) {
    if (!cached || i0 > 0) load_group(a.value_pool, i0, vb);
    u32x4 kb[kGrp][4];
    if (!cached) load_group(a.key_pool, i0, kb);
#pragma unroll
    for (int q = 0; q < kGrp; ++q) {
      if (i0 + q >= cnt) break;
      float p[4][kG];
      const int tok0 = (w + kDecWaves * (i0 + q)) * kBlockSize + r;
      if (cached) {
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          const int tok = tok0 + 4 * t;
#pragma unroll
          for (int j = 0; j < kG; ++j) p[t][j] = tok < n ? bf16_bits_to_f32(s_cache[tok * kG + j]) : 0.0f;
        }
      } else {
        float s[4][kG];
        block_scores(kb[q], s);
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          const bool valid = tok0 + 4 * t < n;
#pragma unroll
          for (int j = 0; j < kG; ++j) p[t][j] = valid ? exact_prob(exact_exp(s[t][j], M[j]), L[j]) : 0.0f;
        }
      }
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        double vd[8];
        unpack8(vb[q][t], vd);
#pragma unroll
        for (int j = 0; j < kG; ++j) {
          const double pj = p[t][j];
#pragma unroll
          for (int e = 0; e < 8; ++e) acc[j][e] = fma(pj, vd[e], acc[j][e]);
        }
      }
    }
  }
  // rows of the wavefront, then the wavefronts (one head at a time through LDS)
#pragma unroll
  for (int j = 0; j < kG; ++j) {
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      double x = acc[j][e];
      x = xsum32_f64(xsum16_f64(x));
      acc[j][e] = x;
    }
  }
#pragma unroll
  for (int j = 0; j < kG; ++j) {
    if (r == 0) {
#pragma unroll
      for (int e = 0; e < 8; ++e) s_o[w][8 * dl + e] = acc[j][e];
    }
    __syncthreads();
    if (threadIdx.x < kHeadDim) {
      double o = 0.0;
#pragma unroll
      for (int v = 0; v < kDecWaves; ++v) o += s_o[v][threadIdx.x];
      out_b[j * kHeadDim + threadIdx.x] = bf16_bits(static_cast<float>(o));
    }
    __syncthreads();
  }
}

template <int kG, bool kPrologue>
__global__ __launch_bounds__(kDecThreads) void exact_decode_kernel(const ExactDecodeArgs a) {
  extern __shared__ __align__(16) unsigned char s_dec[];
  exact_decode_body<kG, kPrologue, kDecWaves>(a, blockIdx.x, blockIdx.y, s_dec);
}

// ------------------------------------------------------------------ split decode ---
// The same decode, cut over splits of each sequence's blocks so that small batches fill the GPU:
//   kernel 1 (sequence, KV head, split): the split's scores, into the workspace (bf16 bits);
//   kernel 2 (sequence, KV head, split): the maximum and the exact denominator over all of the
//     sequence's scores (each split reads them all: a few thousand values), then P V over the
//     split's own blocks as fp64 partial sums;
//   kernel 3 (sequence, KV head): the partials summed in split order, rounded once to bf16.
// Every sum is exact (or off by far less than the final roundings can see), so the split gives the
// single-kernel results.  kernel 1 also runs the prologue (q rotation into LDS; the split holding
// the sequence's last block appends the new K/V row before it reads that block).
constexpr int kSplitWaves = 4;
constexpr int kSplitThreads = 64 * kSplitWaves;
constexpr int kSplitInflight = 2;  // blocks a wavefront loads before using them
constexpr int kMaxSplits = 32;

struct ExactSplitArgs {
  ExactDecodeArgs d;
  uint16_t* scores;   // [batch, kv_heads, ctx_cap, kG] bf16 bits
  double* partial;    // [batch, kv_heads, splits, kG, 128]
  int32_t ctx_cap;    // max_blocks * 16
  int32_t splits;
};

struct SplitRange {
  int n, nblk, lo, hi;
};

__device__ __forceinline__ SplitRange split_range(const ExactDecodeArgs& a, int b, int sp, int splits) {
  int64_t n64 = a.context_lens[b * a.ctx_stride];
  n64 = min(n64, static_cast<int64_t>(a.max_blocks) * kBlockSize);
  SplitRange r;
  r.n = n64 > 0 ? static_cast<int>(n64) : 0;
  r.nblk = (r.n + kBlockSize - 1) / kBlockSize;
  r.lo = static_cast<int>(static_cast<int64_t>(sp) * r.nblk / splits);
  r.hi = static_cast<int>(static_cast<int64_t>(sp + 1) * r.nblk / splits);
  return r;
}

template <int kG, bool kPrologue>
__global__ __launch_bounds__(kSplitThreads) void exact_split_scores_kernel(const ExactSplitArgs sa) {
  const ExactDecodeArgs& a = sa.d;
  const int b = blockIdx.x, g = blockIdx.y, sp = blockIdx.z;
  const SplitRange rg = split_range(a, b, sp, sa.splits);
  if (rg.lo >= rg.hi) return;  // uniform
  __shared__ __align__(16) float s_q[kG][kHeadDim];
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const int dl = lane & 15;
  const int r = lane >> 4;
  const int64_t row_elems = static_cast<int64_t>(a.kv_heads) * kHeadDim;
  if constexpr (kPrologue) {
    // Units u < kG: query head g kG + u rotated into LDS; unit kG (split holding the last block
    // only): key head g rotated and written with value head g into the sequence's new slot.
    const bool appends = rg.hi == rg.nblk;
    for (int u = w; u <= kG; u += kSplitWaves) {
      const bool is_q = u < kG;
      if (!is_q && !appends) continue;
      const uint16_t* src = is_q ? a.q + b * a.q_row + (g * kG + u) * kHeadDim : a.k_new + b * a.k_row + g * kHeadDim;
      float o0, o1;
      norm_rope_head(src, is_q ? a.q_weight : a.k_weight, a.cos + b * kHeadDim, a.sin + b * kHeadDim, a.eps, lane,
                     o0, o1);
      if (is_q) {
        s_q[u][lane] = o0;
        s_q[u][lane + 64] = o1;
      } else {
        const int64_t slot = a.slot_mapping[b * a.slot_stride];
        if (slot >= 0 && slot < a.num_slots) {  // context > 0 here: the split has blocks
          uint16_t* kd = a.key_pool + slot * row_elems + g * kHeadDim;
          uint16_t* vd = a.value_pool + slot * row_elems + g * kHeadDim;
          const uint16_t* vs = a.v_new + b * a.v_row + g * kHeadDim;
          kd[lane] = bf16_bits(o0);
          kd[lane + 64] = bf16_bits(o1);
          vd[lane] = vs[lane];
          vd[lane + 64] = vs[lane + 64];
        }
      }
    }
  } else {
    for (int i = threadIdx.x; i < kG * kHeadDim; i += kSplitThreads) {
      const int j = i / kHeadDim, d = i - j * kHeadDim;
      s_q[j][d] = bf16_bits_to_f32(a.q[b * a.q_row + (g * kG + j) * a.q_head + d]);
    }
  }
  // Orders the append before this workgroup's loads of the last block (no other workgroup reads
  // it in this kernel).
  __syncthreads();

  const int64_t lane_off = r * row_elems + g * kHeadDim + 8 * dl;
  uint16_t* out_scores = sa.scores + (static_cast<int64_t>(b) * a.kv_heads + g) * sa.ctx_cap * kG;
  const int cnt = rg.hi - rg.lo > w ? (rg.hi - rg.lo - 1 - w) / kSplitWaves + 1 : 0;  // blocks lo + w + 4 i
  for (int i0 = 0; i0 < cnt; i0 += kSplitInflight) {
    u32x4 kb[kSplitInflight][4];
#pragma unroll
    for (int q = 0; q < kSplitInflight; ++q) {
      if (i0 + q >= cnt) break;
      const int blk = rg.lo + w + kSplitWaves * (i0 + q);
      int64_t id = a.block_tables[b * a.bt_stride + blk];
      if (id < 0 || id >= a.num_blocks) id = 0;
      const uint16_t* p = a.key_pool + id * kBlockSize * row_elems + lane_off;
#pragma unroll
      for (int t = 0; t < 4; ++t) kb[q][t] = *reinterpret_cast<const u32x4*>(p + 4 * t * row_elems);
    }
#pragma unroll
    for (int q = 0; q < kSplitInflight; ++q) {
      if (i0 + q >= cnt) break;
      const int tok0 = (rg.lo + w + kSplitWaves * (i0 + q)) * kBlockSize + r;
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        double kd[8];
        unpack8(kb[q][t], kd);
        const int tok = tok0 + 4 * t;
#pragma unroll
        for (int j = 0; j < kG; ++j) {
          const float4 q0 = *reinterpret_cast<const float4*>(&s_q[j][8 * dl]);
          const float4 q1 = *reinterpret_cast<const float4*>(&s_q[j][8 * dl + 4]);
          double acc = static_cast<double>(q0.x) * kd[0];
          acc = fma(static_cast<double>(q0.y), kd[1], acc);
          acc = fma(static_cast<double>(q0.z), kd[2], acc);
          acc = fma(static_cast<double>(q0.w), kd[3], acc);
          acc = fma(static_cast<double>(q1.x), kd[4], acc);
          acc = fma(static_cast<double>(q1.y), kd[5], acc);
          acc = fma(static_cast<double>(q1.z), kd[6], acc);
          acc = fma(static_cast<double>(q1.w), kd[7], acc);
          acc = dpp_sum16_f64(acc);
          if (dl == j && tok < rg.n) out_scores[tok * kG + j] = bf16_bits(exact_score(acc, a.scale));
        }
      }
    }
  }
}

template <int kG>
__global__ __launch_bounds__(kSplitThreads) void exact_split_pv_kernel(const ExactSplitArgs sa) {
  const ExactDecodeArgs& a = sa.d;
  const int b = blockIdx.x, g = blockIdx.y, sp = blockIdx.z;
  const SplitRange rg = split_range(a, b, sp, sa.splits);
  if (rg.lo >= rg.hi) return;  // uniform
  __shared__ float s_m[kSplitWaves][kG];
  __shared__ double s_l[kSplitWaves][kG][2];
  __shared__ double s_o[kSplitWaves][kHeadDim];
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const int dl = lane & 15;
  const int r = lane >> 4;
  const int64_t row_elems = static_cast<int64_t>(a.kv_heads) * kHeadDim;
  const int64_t lane_off = r * row_elems + g * kHeadDim + 8 * dl;
  const int cnt = rg.hi - rg.lo > w ? (rg.hi - rg.lo - 1 - w) / kSplitWaves + 1 : 0;
  // The first V blocks go out before the softmax statistics are formed.
  u32x4 vb[kSplitInflight][4];
  auto load_v = [&](int i0) {
#pragma unroll
    for (int q = 0; q < kSplitInflight; ++q) {
      if (i0 + q >= cnt) break;
      const int blk = rg.lo + w + kSplitWaves * (i0 + q);
      int64_t id = a.block_tables[b * a.bt_stride + blk];
      if (id < 0 || id >= a.num_blocks) id = 0;
      const uint16_t* p = a.value_pool + id * kBlockSize * row_elems + lane_off;
#pragma unroll
      for (int t = 0; t < 4; ++t) vb[q][t] = *reinterpret_cast<const u32x4*>(p + 4 * t * row_elems);
    }
  };
  load_v(0);

  // Maximum and exact denominator over all of the sequence's scores.
  const uint16_t* sc = sa.scores + (static_cast<int64_t>(b) * a.kv_heads + g) * sa.ctx_cap * kG;
  float mloc[kG];
#pragma unroll
  for (int j = 0; j < kG; ++j) mloc[j] = -INFINITY;
  for (int tok = threadIdx.x; tok < rg.n; tok += kSplitThreads) {
#pragma unroll
    for (int j = 0; j < kG; ++j) mloc[j] = fmaxf(mloc[j], bf16_bits_to_f32(sc[tok * kG + j]));
  }
#pragma unroll
  for (int j = 0; j < kG; ++j) {
    const float mw = wave_max(mloc[j]);
    if (lane == 0) s_m[w][j] = mw;
  }
  __syncthreads();
  float M[kG];
#pragma unroll
  for (int j = 0; j < kG; ++j) {
    float mx = -INFINITY;
#pragma unroll
    for (int v = 0; v < kSplitWaves; ++v) mx = fmaxf(mx, s_m[v][j]);
    M[j] = mx;
  }
  double hi[kG], lo[kG];
#pragma unroll
  for (int j = 0; j < kG; ++j) hi[j] = lo[j] = 0.0;
  for (int tok = threadIdx.x; tok < rg.n; tok += kSplitThreads) {
#pragma unroll
    for (int j = 0; j < kG; ++j) split_add(exact_exp(bf16_bits_to_f32(sc[tok * kG + j]), M[j]), hi[j], lo[j]);
  }
#pragma unroll
  for (int j = 0; j < kG; ++j) {
    const double h = wave_sum64_f64(hi[j]), l = wave_sum64_f64(lo[j]);
    if (lane == 0) {
      s_l[w][j][0] = h;
      s_l[w][j][1] = l;
    }
  }
  __syncthreads();
  float L[kG];
#pragma unroll
  for (int j = 0; j < kG; ++j) {
    double h = 0.0, l = 0.0;
#pragma unroll
    for (int v = 0; v < kSplitWaves; ++v) {
      h += s_l[v][j][0];
      l += s_l[v][j][1];
    }
    L[j] = static_cast<float>(h + l);
  }

  // P V over the split's blocks (lane: tokens 4 i + r of each block, dims 8 dl .. +8).
  double acc[kG][8];
#pragma unroll
  for (int j = 0; j < kG; ++j)
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[j][e] = 0.0;
  for (int i0 = 0; i0 < cnt; i0 += kSplitInflight) {
    if (i0 > 0) load_v(i0);
#pragma unroll
    for (int q = 0; q < kSplitInflight; ++q) {
      if (i0 + q >= cnt) break;
      const int tok0 = (rg.lo + w + kSplitWaves * (i0 + q)) * kBlockSize + r;
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        const int tok = tok0 + 4 * t;
        double vd[8];
        unpack8(vb[q][t], vd);
#pragma unroll
        for (int j = 0; j < kG; ++j) {
          const double pj = tok < rg.n ? exact_prob(exact_exp(bf16_bits_to_f32(sc[tok * kG + j]), M[j]), L[j]) : 0.0;
#pragma unroll
          for (int e = 0; e < 8; ++e) acc[j][e] = fma(pj, vd[e], acc[j][e]);
        }
      }
    }
  }
  // rows of the wavefront, then the wavefronts (one head at a time through LDS)
#pragma unroll
  for (int j = 0; j < kG; ++j) {
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      double x = acc[j][e];
      x = xsum32_f64(xsum16_f64(x));
      acc[j][e] = x;
    }
  }
  double* part = sa.partial + ((static_cast<int64_t>(b) * a.kv_heads + g) * sa.splits + sp) * kG * kHeadDim;
#pragma unroll
  for (int j = 0; j < kG; ++j) {
    if (r == 0) {
#pragma unroll
      for (int e = 0; e < 8; ++e) s_o[w][8 * dl + e] = acc[j][e];
    }
    __syncthreads();
    if (threadIdx.x < kHeadDim) {
      double o = 0.0;
#pragma unroll
      for (int v = 0; v < kSplitWaves; ++v) o += s_o[v][threadIdx.x];
      part[j * kHeadDim + threadIdx.x] = o;
    }
    __syncthreads();
  }
}

template <int kG>
__global__ __launch_bounds__(kHeadDim) void exact_split_merge_kernel(const ExactSplitArgs sa) {
  const ExactDecodeArgs& a = sa.d;
  const int b = blockIdx.x, g = blockIdx.y;
  uint16_t* out_b = a.out + b * a.out_row + (g * kG) * kHeadDim;
  const double* part = sa.partial + (static_cast<int64_t>(b) * a.kv_heads + g) * sa.splits * kG * kHeadDim;
  const SplitRange rg = split_range(a, b, 0, sa.splits);
#pragma unroll
  for (int j = 0; j < kG; ++j) {
    double o = 0.0;
    for (int sp = 0; sp < sa.splits; ++sp) {
      const int lo = static_cast<int>(static_cast<int64_t>(sp) * rg.nblk / sa.splits);
      const int hi = static_cast<int>(static_cast<int64_t>(sp + 1) * rg.nblk / sa.splits);
      if (lo < hi) o += part[(static_cast<int64_t>(sp) * kG + j) * kHeadDim + threadIdx.x];
    }
    out_b[j * kHeadDim + threadIdx.x] = bf16_bits(static_cast<float>(o));  // zero rows for empty contexts
  }
}

// ----------------------------------------------------------------------- prefill ---
// Chunked prefill (history from the pool, then the causal chunk) on the fp64 matrix cores
// (v_mfma_f64_16x16x4f64: D[16][16] += A[16][4] B[4][16] in fp64).  Products of bf16 values are
// exact in fp64 and the sums are exact, so the matrix cores give the same bits as any other order.
//
// A workgroup takes 16 (query, head) columns of one (row, KV head): 16 / G query positions times
// the G query heads of the group (15 columns for G = 5).  Its 4 wavefronts split the 16-key tiles
// of the keys (wavefront w: tiles w, w + 4, ...) and merge their maxima, sums and outputs through
// LDS, so the heaviest query tile of a chunk is spread over four SIMDs.  Per 16-key tile a
// wavefront runs
//   S^T = K Q^T   32 MFMAs over the 128 dims: A = K, the tile's key rho(c) = 4 (c % 4) + c / 4 in
//                 row c; B = Q^T; the k index of MFMA t is dim 32 (lane / 16) + t, so a lane reads
//                 64 contiguous bytes of its key and query.  D row l / 16 + 4 r holds key
//                 rho(l / 16 + 4 r) = 4 (l / 16) + r: lane l ends up with keys 4 (l / 16) .. + 3 of
//                 column l % 16 in its four result registers.
//   O += P V      32 MFMAs: A = P, lane l supplying column l % 16 and key 4 (l / 16) + u (its own
//                 register u) in MFMA u; B = V, whose column j of output tile dt is dim 8 j + dt, so
//                 a lane reads the 16 bytes of dims 8 (l % 16) .. + 7 of each of its four keys and
//                 writes 16 contiguous output bytes per column.
// The passes are those of the decode body: scores and their maxima (the bf16 scores cached in
// LDS, 8 bytes per lane and tile, when the launch's longest row fits), the exact denominators,
// then the probabilities and P V.  Rows too long for the cache recompute S in each pass.
//
// Measured on one MI355X (G = 2, 8 KV heads; TFLOP/s of QK + PV as 4 x 128 flops per visible
// (query head, key) pair; v_mfma_f64_16x16x4f64 alone peaks near 46 TFLOP/s in a loop of
// independent accumulators, v_mfma_f64_4x4x4f64 near 72, but forms on the latter ran no faster:
// the fp64 exponentials, divisions and operand conversions bound this kernel): one 2048-token row 471-476 us (36.1-36.5 TFLOP/s), two 1024-token rows 235-236 us,
// four rows of ~512 tokens 168 us, 1000 history + 1024 chunk tokens 374-378 us, with the queries
// read by 16-byte loads (2-byte loads: 484 / 249 / 184 / 387 us).  The fp64 FMA form this replaces
// (one lane per key, query rows broadcast from LDS, one wavefront per SIMD) took 3106 / 934 / 499 /
// 1845 us.  A timing copy without the cross-wavefront merge of the outputs ran about 1% faster.
constexpr int kPfWaves = 4;
constexpr int kPfThreads = 64 * kPfWaves;
constexpr int kPfCols = 16;                                    // (query, head) columns of a workgroup
constexpr int kPfTileKeys = 16;                                // keys of one MFMA tile
constexpr int kPfCacheTileBytes = 64 * 8;                      // one wavefront's scores of one tile
constexpr int kPfRedBytes = kPfWaves * kPfCols * (4 + 16);     // per-wavefront maxima and hi / lo sums
constexpr int kPfMergeBytes = 2 * 32 * 64 * 8;                 // two wavefronts' partial outputs
constexpr int kPfLdsBytes = 160 * 1024;
constexpr int kPfMaxCacheTiles = (kPfLdsBytes - kPfRedBytes) / (kPfWaves * kPfCacheTileBytes);  // per wavefront

struct ExactPrefillArgs {
  uint16_t* out;
  int64_t out_row, out_tok;
  const uint16_t* q;
  int64_t q_row, q_head, q_tok;
  const uint16_t* k;
  int64_t k_row, k_head, k_tok;
  const uint16_t* v;
  int64_t v_row, v_head, v_tok;
  uint16_t* key_pool;
  uint16_t* value_pool;
  int64_t num_blocks;
  int32_t kv_heads;
  const int64_t* history;
  int64_t hist_stride;
  int32_t max_hist_blocks;
  const int64_t* start_lens;
  const int64_t* chunk_lens;
  int64_t lens_stride;
  int32_t padded_len;
  float scale;
  int32_t cache_tiles;     // key tiles per wavefront the LDS score cache holds (cached form)
  int32_t tiles;           // query tiles per row
  int32_t batch;           // rows
  int32_t groups;          // workgroups of these rows: tiles x kv_heads x batch
  int32_t q_vec;           // query rows 16-byte aligned (pointer and strides): 16-byte loads
  // Decode rows (a mixed step's single new tokens, padded_len 1): start_lens holds each row's
  // context length including its token, so the history is the context minus one and the chunk key
  // is the token itself; a row with context 0 is padding.  The token's K/V row of each KV head is
  // also appended to pool slot slot_mapping[b] (skipped when outside the pool).
  int32_t decode_rows;
  const int64_t* slot_mapping;
  int64_t slot_stride;
  // Ragged chunk rows (a mixed step's chunks packed back to back): when set, the clen real tokens
  // of row b are flat tokens row_first[b] .. row_first[b] + clen - 1 of q / k / v / out (the token
  // strides apply, the row strides are unused; row_first[b] is clamped to [0, row_tokens - clen]),
  // and padding positions are neither read nor written.
  const int64_t* row_first;
  int64_t row_tokens;
};

typedef double f64x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ f64x4 mfma_f64(double a, double b, f64x4 c) {
  return __builtin_amdgcn_mfma_f64_16x16x4f64(a, b, c, 0, 0, 0);
}

// Element e of eight bf16 values held as a 16-byte piece, as a double (exact).
__device__ __forceinline__ double bf16_at(const u32x4 v, int e) {
  const uint32_t x = v[e >> 1];
  return (e & 1) ? bf16_hi(x) : bf16_lo(x);
}

// One launch serves a mixed step: the first a1.groups workgroups take the decode rows of a1 as
// one-token chunks (history: the context but the token; each as heavy as the chunk's heaviest
// query tiles, so dispatched first), the rest the chunk rows of a0 -- the sums are exact, so the
// decode rows get the bits of the exact decode body.
template <int kG, bool kCached>
__global__ __launch_bounds__(kPfThreads) void exact_prefill_kernel(const ExactPrefillArgs a0, const ExactPrefillArgs a1) {
  constexpr int kQP = kPfCols / kG;  // query positions of a workgroup
  constexpr int kCols = kQP * kG;    // columns in use (15 for G = 5)
  extern __shared__ __align__(16) unsigned char s_raw[];
  const bool decode = static_cast<int>(blockIdx.x) < a1.groups;  // uniform
  const ExactPrefillArgs a = decode ? a1 : a0;
  float* sM = reinterpret_cast<float*>(s_raw);                                    // [waves][16]
  double* sL = reinterpret_cast<double*>(s_raw + kPfWaves * kPfCols * 4);          // [waves][16][hi, lo]
  uint2* sC = reinterpret_cast<uint2*>(s_raw + kPfRedBytes);                      // [waves][cache_tiles][64]
  double* sO = reinterpret_cast<double*>(s_raw + kPfRedBytes);                    // [2][32][64], after the cache

  // Workgroup order: query tiles from the last (most keys) to the first across every row and KV
  // head, the KV head fastest, so consecutive workgroups (round-robin over the XCDs) keep one KV
  // head's keys on one XCD when there are 8 KV heads.
  const int lin = static_cast<int>(blockIdx.x) - (decode ? 0 : a1.groups);
  const int g = lin % a.kv_heads;
  const int b = (lin / a.kv_heads) % a.batch;
  const int qt = a.tiles - 1 - lin / (a.kv_heads * a.batch);
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const int q4 = lane >> 4, c = lane & 15;
  const int L = a.padded_len;
  int64_t clen, nh64;
  if (a.decode_rows) {
    const int64_t ctx = a.start_lens[b * a.lens_stride];
    clen = ctx > 0 ? 1 : 0;
    nh64 = ctx - 1;
  } else {
    clen = a.chunk_lens[b * a.lens_stride];
    nh64 = a.start_lens[b * a.lens_stride];
  }
  clen = clen < 0 ? 0 : (clen > L ? L : clen);
  const int pad = L - static_cast<int>(clen);
  nh64 = nh64 < 0 ? 0 : min(nh64, static_cast<int64_t>(a.max_hist_blocks) * kBlockSize);
  const int nh = static_cast<int>(nh64);
  const int i0 = qt * kQP;
  const int i_last = min(i0 + kQP - 1, L - 1);
  const int64_t row_elems = static_cast<int64_t>(a.kv_heads) * kHeadDim;
  // Element offset of padded position rpad of row b (its first stored token): position i >= rpad
  // of a tensor with row / token strides (r, t) is at base + (i - rpad) t.
  const bool ragged = a.row_first != nullptr;  // uniform
  if (ragged && clen == 0) return;              // an empty ragged row stores nothing
  int64_t first = 0;
  if (ragged) {
    first = a.row_first[b];
    first = first < 0 ? 0 : (first > a.row_tokens - clen ? a.row_tokens - clen : first);
  }
  const int rpad = ragged ? pad : 0;
  const int64_t q_base = ragged ? first * a.q_tok : b * a.q_row;
  const int64_t k_base = ragged ? first * a.k_tok : b * a.k_row;
  const int64_t v_base = ragged ? first * a.v_tok : b * a.v_row;
  const int64_t o_base = ragged ? first * a.out_tok : b * a.out_row;

  if (a.decode_rows && clen > 0 && threadIdx.x < 32) {  // append the token's K and V rows of KV head g
    const int64_t slot = a.slot_mapping[b * a.slot_stride];
    if (slot >= 0 && slot < a.num_blocks * kBlockSize) {
      const int piece = (threadIdx.x & 15) * 8;
      const uint16_t* src = threadIdx.x < 16 ? a.k + b * a.k_row + g * a.k_head : a.v + b * a.v_row + g * a.v_head;
      uint16_t* dst = (threadIdx.x < 16 ? a.key_pool : a.value_pool) + slot * row_elems + g * kHeadDim;
      *reinterpret_cast<uint4*>(dst + piece) = *reinterpret_cast<const uint4*>(src + piece);
    }
  }

  if (i_last < pad) {  // every query of the tile is padding: zero rows (uniform; a ragged row stores none)
    if (ragged) return;
    const int col = threadIdx.x >> 4, piece = threadIdx.x & 15;
    const int i = i0 + col / kG;
    if (col < kCols && i < L)
      *reinterpret_cast<uint4*>(a.out + b * a.out_row + i * a.out_tok + (g * kG + col % kG) * kHeadDim + 8 * piece) =
          uint4{0, 0, 0, 0};
    return;
  }
  const int nkeys = nh + i_last - pad + 1;  // keys any column of the tile sees
  const int ntiles = (nkeys + kPfTileKeys - 1) / kPfTileKeys;

  // This lane's column: query position i0 + c / G, query head g G + c % G.  Key kk (history slots
  // first, then chunk positions pad, pad + 1, ...) is visible to it iff kk <= kmax.
  const int ci = i0 + c / kG;
  const int kmax = (c < kCols && ci < L && ci >= pad) ? nh + ci - pad : -1;

  // Q^T operand: dims 32 q4 .. + 31 of column c, as doubles (zeros for unused columns).
  double qd[32];
  {
    const bool live = c < kCols && ci < L;
    const int cq = max(min(ci, L - 1), rpad);  // unused columns read a stored row and keep zeros
    const uint16_t* qrow = a.q + q_base + (g * kG + c % kG) * a.q_head + static_cast<int64_t>(cq - rpad) * a.q_tok + 32 * q4;
    if (a.q_vec) {  // uniform
      u32x4 qv[4];
#pragma unroll
      for (int x = 0; x < 4; ++x) qv[x] = reinterpret_cast<const u32x4*>(qrow)[x];
#pragma unroll
      for (int t = 0; t < 32; ++t) qd[t] = live ? bf16_at(qv[t >> 3], t & 7) : 0.0;
    } else {
#pragma unroll
      for (int t = 0; t < 32; ++t) qd[t] = live ? static_cast<double>(bf16_bits_to_f32(qrow[t])) : 0.0;
    }
  }

  // Row of key kk (clamped to the last key any column sees; such keys are masked or zeroed).
  auto key_row = [&](int kk, bool values) -> const uint16_t* {
    const int kc = min(kk, nkeys - 1);
    if (kc < nh) {
      int64_t id = a.history[b * a.hist_stride + kc / kBlockSize];
      if (id < 0 || id >= a.num_blocks) id = 0;
      return (values ? a.value_pool : a.key_pool) + (id * kBlockSize + kc % kBlockSize) * row_elems + g * kHeadDim;
    }
    const int p = pad + (kc - nh) - rpad;  // from the row's first stored position
    return values ? a.v + v_base + g * a.v_head + static_cast<int64_t>(p) * a.v_tok
                  : a.k + k_base + g * a.k_head + static_cast<int64_t>(p) * a.k_tok;
  };
  // Scores of keys 16 kt + 4 q4 + r (r = 0..3) against column c.
  auto tile_scores = [&](int kt, float (&sc)[4]) {
    const u32x4* krow = reinterpret_cast<const u32x4*>(key_row(kPfTileKeys * kt + 4 * (c & 3) + (c >> 2), false) + 32 * q4);
    u32x4 kr[4];
#pragma unroll
    for (int x = 0; x < 4; ++x) kr[x] = krow[x];
    f64x4 s0 = {0.0, 0.0, 0.0, 0.0}, s1 = {0.0, 0.0, 0.0, 0.0};
#pragma unroll
    for (int t = 0; t < 32; t += 2) {
      s0 = mfma_f64(bf16_at(kr[t >> 3], t & 7), qd[t], s0);
      s1 = mfma_f64(bf16_at(kr[(t + 1) >> 3], (t + 1) & 7), qd[t + 1], s1);
    }
#pragma unroll
    for (int r = 0; r < 4; ++r) sc[r] = exact_score(s0[r] + s1[r], a.scale);  // both halves exact
  };
  auto cache_slot = [&](int lt) -> uint2* { return sC + (static_cast<int64_t>(w) * a.cache_tiles + lt) * 64 + lane; };
  auto tile_scores_any = [&](int kt, int lt, float (&sc)[4]) {
    if constexpr (kCached) {
      const uint2 x = *cache_slot(lt);
      sc[0] = bf16_lo(x.x);
      sc[1] = bf16_hi(x.x);
      sc[2] = bf16_lo(x.y);
      sc[3] = bf16_hi(x.y);
    } else {
      tile_scores(kt, sc);
    }
  };

  // ---- pass 1: scores and the column maxima
  float mloc = -INFINITY;
  for (int kt = w, lt = 0; kt < ntiles; kt += kPfWaves, ++lt) {
    float sc[4];
    tile_scores(kt, sc);
    const int kb = kPfTileKeys * kt + 4 * q4;
#pragma unroll
    for (int r = 0; r < 4; ++r)
      if (kb + r <= kmax) mloc = fmaxf(mloc, sc[r]);
    if constexpr (kCached)
      *cache_slot(lt) = uint2{static_cast<uint32_t>(bf16_bits(sc[0])) | (static_cast<uint32_t>(bf16_bits(sc[1])) << 16),
                              static_cast<uint32_t>(bf16_bits(sc[2])) | (static_cast<uint32_t>(bf16_bits(sc[3])) << 16)};
  }
  mloc = xmax32(xmax16(mloc));
  if (q4 == 0) sM[w * kPfCols + c] = mloc;
  __syncthreads();
  float M = sM[c];
#pragma unroll
  for (int x = 1; x < kPfWaves; ++x) M = fmaxf(M, sM[x * kPfCols + c]);

  // ---- pass 2: denominators
  double hi = 0.0, lo = 0.0;
  for (int kt = w, lt = 0; kt < ntiles; kt += kPfWaves, ++lt) {
    float sc[4];
    tile_scores_any(kt, lt, sc);
    const int kb = kPfTileKeys * kt + 4 * q4;
#pragma unroll
    for (int r = 0; r < 4; ++r)
      if (kb + r <= kmax) split_add(exact_exp(sc[r], M), hi, lo);
  }
  hi = xsum32_f64(xsum16_f64(hi));
  lo = xsum32_f64(xsum16_f64(lo));
  if (q4 == 0) {
    sL[(w * kPfCols + c) * 2] = hi;
    sL[(w * kPfCols + c) * 2 + 1] = lo;
  }
  __syncthreads();
  double hsum = 0.0, lsum = 0.0;
#pragma unroll
  for (int x = 0; x < kPfWaves; ++x) {
    hsum += sL[(x * kPfCols + c) * 2];
    lsum += sL[(x * kPfCols + c) * 2 + 1];
  }
  const float Lc = static_cast<float>(hsum + lsum);

  // ---- pass 3: probabilities and P V
  f64x4 o[8];
#pragma unroll
  for (int dt = 0; dt < 8; ++dt) o[dt] = f64x4{0.0, 0.0, 0.0, 0.0};
  for (int kt = w, lt = 0; kt < ntiles; kt += kPfWaves, ++lt) {
    const int kb = kPfTileKeys * kt + 4 * q4;
    u32x4 vr[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      vr[u] = *reinterpret_cast<const u32x4*>(key_row(kb + u, true) + 8 * c);
      if (kb + u >= nkeys) vr[u] = u32x4{0u, 0u, 0u, 0u};
    }
    float sc[4];
    tile_scores_any(kt, lt, sc);
    double p[4];
#pragma unroll
    for (int u = 0; u < 4; ++u)
      p[u] = kb + u <= kmax ? static_cast<double>(exact_prob(exact_exp(sc[u], M), Lc)) : 0.0;
#pragma unroll
    for (int dt = 0; dt < 8; ++dt) {
#pragma unroll
      for (int u = 0; u < 4; ++u) o[dt] = mfma_f64(p[u], bf16_at(vr[u], dt), o[dt]);
    }
  }

  // ---- merge the four wavefronts' partial outputs: (O0 + O2) + (O1 + O3)
  __syncthreads();  // the cache, which the merge area overlays, is no longer read
  if (w >= 2) {
#pragma unroll
    for (int e = 0; e < 32; ++e) sO[((w - 2) * 32 + e) * 64 + lane] = o[e >> 2][e & 3];
  }
  __syncthreads();
  if (w < 2) {
#pragma unroll
    for (int e = 0; e < 32; ++e) o[e >> 2][e & 3] += sO[(w * 32 + e) * 64 + lane];
  }
  __syncthreads();
  if (w == 1) {
#pragma unroll
    for (int e = 0; e < 32; ++e) sO[e * 64 + lane] = o[e >> 2][e & 3];
  }
  __syncthreads();
  if (w != 0) return;
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int col = q4 + 4 * r;
    const int i = i0 + col / kG;
    if (col >= kCols || i >= L || i < rpad) continue;
    uint32_t word[4];
#pragma unroll
    for (int h = 0; h < 4; ++h) {
      const double x0 = o[2 * h][r] + sO[((2 * h) * 4 + r) * 64 + lane];
      const double x1 = o[2 * h + 1][r] + sO[((2 * h + 1) * 4 + r) * 64 + lane];
      word[h] = i < pad ? 0u
                        : static_cast<uint32_t>(bf16_bits(static_cast<float>(x0))) |
                              (static_cast<uint32_t>(bf16_bits(static_cast<float>(x1))) << 16);
    }
    *reinterpret_cast<uint4*>(a.out + o_base + static_cast<int64_t>(i - rpad) * a.out_tok +
                              (g * kG + col % kG) * kHeadDim + 8 * c) = uint4{word[0], word[1], word[2], word[3]};
  }
}

// ------------------------------------------------------------------------- host ---
bool group_ok(int g) { return g == 1 || g == 2 || g == 4 || g == 5 || g == 8; }

template <typename Kernel>
int32_t allow_lds(Kernel kernel, int bytes, const char* what) {
  // Dynamic LDS above 64 KiB must be allowed per kernel (gfx950 has 160 KiB per workgroup).
  const hipError_t err = hipFuncSetAttribute(reinterpret_cast<const void*>(kernel),
                                             hipFuncAttributeMaxDynamicSharedMemorySize, bytes);
  if (err != hipSuccess) return fail(MI_ERR_DEVICE, "%s: hipFuncSetAttribute: %s", what, hipGetErrorString(err));
  return MI_OK;
}

template <int kG, bool kPrologue>
int32_t launch_exact_decode(const ExactDecodeArgs& a, int32_t batch, hipStream_t s) {
  static std::once_flag once;
  static int32_t attr_rc = MI_OK;
  using Lds = DecodeLds<kG, kDecWaves>;
  std::call_once(once, [] {
    attr_rc = allow_lds(exact_decode_kernel<kG, kPrologue>, Lds::kFixed + kDecCacheBytes, "mi_paged_decode_attention_exact");
  });
  if (attr_rc != MI_OK) return attr_rc;
  const size_t lds = Lds::kFixed + static_cast<size_t>(a.cache_tokens) * kG * sizeof(uint16_t);
  exact_decode_kernel<kG, kPrologue><<<dim3(batch, a.kv_heads), kDecThreads, lds, s>>>(a);
  return check_launch("mi_paged_decode_attention_exact");
}

template <int kG, bool kPrologue>
int32_t launch_exact_split(const ExactSplitArgs& sa, int32_t batch, hipStream_t s) {
  const dim3 grid(batch, sa.d.kv_heads, sa.splits);
  exact_split_scores_kernel<kG, kPrologue><<<grid, kSplitThreads, 0, s>>>(sa);
  if (const int32_t rc = check_launch("mi_paged_decode_attention_exact(scores)")) return rc;
  exact_split_pv_kernel<kG><<<grid, kSplitThreads, 0, s>>>(sa);
  if (const int32_t rc = check_launch("mi_paged_decode_attention_exact(pv)")) return rc;
  exact_split_merge_kernel<kG><<<dim3(batch, sa.d.kv_heads), kHeadDim, 0, s>>>(sa);
  return check_launch("mi_paged_decode_attention_exact(merge)");
}

template <bool kPrologue>
int32_t dispatch_exact_split(const ExactSplitArgs& sa, int32_t batch, int group, hipStream_t s) {
  switch (group) {
    case 1: return launch_exact_split<1, kPrologue>(sa, batch, s);
    case 2: return launch_exact_split<2, kPrologue>(sa, batch, s);
    case 4: return launch_exact_split<4, kPrologue>(sa, batch, s);
    case 5: return launch_exact_split<5, kPrologue>(sa, batch, s);
    default: return launch_exact_split<8, kPrologue>(sa, batch, s);
  }
}

// Splits of each sequence for the split decode: enough (sequence, KV head, split) workgroups for
// two per CU, at most one per 4 table blocks (so the 4 wavefronts of a split have blocks to read)
// and at most kMaxSplits; 1 = the single-kernel form.  Only launches of at most kMaxSplitPairs
// (sequence, KV head) pairs split: measured on MI355X (28 layers in a HIP graph, contexts U[200,
// 1150], GQA group 2), µs per layer single / split: batch 1 24.4 / 21.2, 4 30.4 / 24.5,
// 9 27.8 / 33.6, 16 36.2 / 45.8, 24 36.5 / 59.6, 32 38.0 / 67.6 -- three dependent launches cost
// more than one launch's idle CUs once the batch gives a workgroup to a fifth of them.
constexpr int64_t kMaxSplitPairs = 48;
int32_t exact_decode_splits(int32_t batch, int32_t max_blocks, int32_t num_kv_heads) {
  const int64_t pairs = static_cast<int64_t>(batch) * num_kv_heads;
  if (pairs <= 0 || pairs > kMaxSplitPairs || batch > 65535) return 1;
  int64_t splits = (2 * static_cast<int64_t>(device_cus()) + pairs - 1) / pairs;
  splits = std::min<int64_t>(splits, kMaxSplits);
  splits = std::min<int64_t>(splits, max_blocks / kSplitWaves);
  return splits < 2 ? 1 : static_cast<int32_t>(splits);
}

// Workspace of the split decode: the scores [batch, kv_heads, max_blocks * 16, G] bf16, then the
// partials [batch, kv_heads, splits, G, 128] fp64 (256-byte aligned).
struct ExactSplitLayout {
  int32_t splits;
  int64_t scores_bytes, bytes;
};
ExactSplitLayout exact_split_layout(int32_t batch, int32_t max_blocks, int32_t num_heads, int32_t num_kv_heads) {
  ExactSplitLayout l{1, 0, 0};
  if (batch <= 0 || max_blocks <= 0 || num_kv_heads <= 0 || num_heads % num_kv_heads != 0) return l;
  l.splits = exact_decode_splits(batch, max_blocks, num_kv_heads);
  if (l.splits < 2) return l;
  const int64_t group = num_heads / num_kv_heads;
  const int64_t pairs = static_cast<int64_t>(batch) * num_kv_heads;
  l.scores_bytes = (pairs * max_blocks * kBlockSize * group * 2 + 255) / 256 * 256;
  l.bytes = l.scores_bytes + pairs * l.splits * group * kHeadDim * 8;
  return l;
}

template <bool kPrologue>
int32_t dispatch_exact_decode(const ExactDecodeArgs& a, int32_t batch, int group, hipStream_t s) {
  switch (group) {
    case 1: return launch_exact_decode<1, kPrologue>(a, batch, s);
    case 2: return launch_exact_decode<2, kPrologue>(a, batch, s);
    case 4: return launch_exact_decode<4, kPrologue>(a, batch, s);
    case 5: return launch_exact_decode<5, kPrologue>(a, batch, s);
    default: return launch_exact_decode<8, kPrologue>(a, batch, s);
  }
}

template <int kG, bool kCached>
int32_t launch_exact_prefill(const ExactPrefillArgs& a0, const ExactPrefillArgs& a1, const char* what, hipStream_t s) {
  static std::once_flag once;
  static int32_t attr_rc = MI_OK;
  std::call_once(once, [] { attr_rc = allow_lds(exact_prefill_kernel<kG, kCached>, kPfLdsBytes, "exact_prefill_kernel"); });
  if (attr_rc != MI_OK) return attr_rc;
  if (a0.groups < 0 || a1.groups < 0 || static_cast<int64_t>(a0.groups) + a1.groups > 0x3fffffff)
    return fail(MI_ERR_UNSUPPORTED, "%s: too many workgroups", what);
  const int groups = a0.groups + a1.groups;
  if (groups == 0) return ok();
  const size_t lds = static_cast<size_t>(kPfRedBytes) +
                     std::max(static_cast<size_t>(kPfMergeBytes),
                              kCached ? static_cast<size_t>(a0.cache_tiles) * kPfWaves * kPfCacheTileBytes : size_t{0});
  exact_prefill_kernel<kG, kCached><<<groups, kPfThreads, lds, s>>>(a0, a1);
  return check_launch(what);
}

// Both row sets share one score-cache size (the larger of the two; the recomputing form when
// either set's rows are too long for the cache).
int32_t dispatch_exact_prefill(ExactPrefillArgs a0, ExactPrefillArgs a1, int group, const char* what, hipStream_t s) {
  const bool cached = (a0.groups == 0 || a0.cache_tiles > 0) && (a1.groups == 0 || a1.cache_tiles > 0);
  const int32_t tiles = cached ? std::max(a0.groups > 0 ? a0.cache_tiles : 0, a1.groups > 0 ? a1.cache_tiles : 0) : 0;
  a0.cache_tiles = a1.cache_tiles = tiles;
  switch (group) {
    case 1: return cached ? launch_exact_prefill<1, true>(a0, a1, what, s) : launch_exact_prefill<1, false>(a0, a1, what, s);
    case 2: return cached ? launch_exact_prefill<2, true>(a0, a1, what, s) : launch_exact_prefill<2, false>(a0, a1, what, s);
    case 4: return cached ? launch_exact_prefill<4, true>(a0, a1, what, s) : launch_exact_prefill<4, false>(a0, a1, what, s);
    case 5: return cached ? launch_exact_prefill<5, true>(a0, a1, what, s) : launch_exact_prefill<5, false>(a0, a1, what, s);
    default: return cached ? launch_exact_prefill<8, true>(a0, a1, what, s) : launch_exact_prefill<8, false>(a0, a1, what, s);
  }
}

// Row-independent fields: grid shape and the LDS score cache for rows of up to `keys` keys (the
// cached form when each wavefront's share of them fits, else the recomputing form).
void exact_rows(ExactPrefillArgs& a, int32_t batch, int32_t padded_len, int32_t num_heads, int32_t num_kv_heads,
                int64_t keys, float scale) {
  const int group = num_heads / num_kv_heads;
  a.batch = batch;
  a.padded_len = padded_len;
  a.kv_heads = num_kv_heads;
  a.scale = scale;
  const int q_per_group = kPfCols / group;
  a.tiles = (padded_len + q_per_group - 1) / q_per_group;
  const int64_t groups = static_cast<int64_t>(a.tiles) * num_kv_heads * batch;
  a.groups = groups > 0x3fffffff ? -1 : static_cast<int32_t>(groups);
  const int64_t key_tiles = (keys + kPfTileKeys - 1) / kPfTileKeys;
  const int64_t per_wave = (key_tiles + kPfWaves - 1) / kPfWaves;
  a.cache_tiles = per_wave <= kPfMaxCacheTiles ? static_cast<int32_t>(per_wave) : 0;
}

int32_t check_exact_heads(const char* what, int32_t num_heads, int32_t num_kv_heads, int32_t head_dim,
                          int32_t block_size) {
  if (head_dim != kHeadDim || block_size != kBlockSize || num_kv_heads <= 0 || num_heads <= 0 ||
      num_heads % num_kv_heads != 0 || !group_ok(num_heads / num_kv_heads))
    return fail(MI_ERR_UNSUPPORTED,
                "%s: needs head_dim %d, block_size %d and %s (got head_dim %d, block_size %d, heads %d/%d)", what,
                kHeadDim, kBlockSize, "1, 2, 4, 5 or 8 query heads per KV head", head_dim, block_size, num_heads,
                num_kv_heads);
  if (num_kv_heads > 65535) return fail(MI_ERR_UNSUPPORTED, "%s: too many KV heads", what);
  return MI_OK;
}

}  // namespace
}  // namespace mi

extern "C" int32_t mi_paged_decode_attention_exact(
    void* out, int64_t out_row_stride, const void* q, int64_t q_row_stride, int64_t q_head_stride, const void* k,
    int64_t k_row_stride, const void* v, int64_t v_row_stride, const void* q_weight, const void* k_weight,
    const void* cos, const void* sin, float eps, const int64_t* slot_mapping, int64_t slot_stride, void* key_pool,
    void* value_pool, int64_t num_blocks, const int64_t* block_tables, int64_t block_table_stride, int32_t max_blocks,
    const int64_t* context_lens, int64_t context_lens_stride, int32_t batch, int32_t num_heads, int32_t num_kv_heads,
    int32_t head_dim, int32_t block_size, float scale, void* workspace, int64_t workspace_bytes, void* stream) {
  using namespace mi;
  const char* what = "mi_paged_decode_attention_exact";
  if (batch < 0 || max_blocks < 0 || num_blocks < 0) return fail(MI_ERR_INVALID_ARGUMENT, "%s: negative size", what);
  if (batch == 0) return ok();
  if (const int32_t rc = reject_empty_pool(what, num_blocks, max_blocks > 0)) return rc;
  if (const int32_t rc = check_exact_heads(what, num_heads, num_kv_heads, head_dim, block_size)) return rc;
  const bool prologue = q_weight != nullptr;
  if (!out || !q || !key_pool || !value_pool || !context_lens || (max_blocks > 0 && !block_tables))
    return fail(MI_ERR_INVALID_ARGUMENT, "%s: null pointer argument", what);
  if (prologue && (!k || !v || !k_weight || !cos || !sin || !slot_mapping))
    return fail(MI_ERR_INVALID_ARGUMENT, "%s: the prologue form needs k, v, k_weight, cos, sin and slot_mapping", what);
  if (!aligned16(out) || out_row_stride % 8 != 0 || !aligned16(key_pool) || !aligned16(value_pool))
    return fail(MI_ERR_UNSUPPORTED, "%s: out and pools must be 16-byte aligned", what);
  if ((max_blocks > 0 && block_table_stride < max_blocks) || context_lens_stride <= 0 ||
      (prologue && (q_row_stride < static_cast<int64_t>(num_heads) * head_dim ||
                    k_row_stride < static_cast<int64_t>(num_kv_heads) * head_dim ||
                    v_row_stride < static_cast<int64_t>(num_kv_heads) * head_dim)))
    return fail(MI_ERR_INVALID_ARGUMENT, "%s: bad stride", what);
  if (num_blocks > INT64_MAX / (kBlockSize * static_cast<int64_t>(num_kv_heads) * head_dim))
    return fail(MI_ERR_INVALID_ARGUMENT, "%s: pool too large", what);
  const int group = num_heads / num_kv_heads;
  ExactDecodeArgs a{};
  a.out = static_cast<uint16_t*>(out);
  a.out_row = out_row_stride;
  a.q = static_cast<const uint16_t*>(q);
  a.q_row = q_row_stride;
  a.q_head = prologue ? head_dim : q_head_stride;
  a.k_new = static_cast<const uint16_t*>(k);
  a.v_new = static_cast<const uint16_t*>(v);
  a.k_row = k_row_stride;
  a.v_row = v_row_stride;
  a.q_weight = static_cast<const uint16_t*>(q_weight);
  a.k_weight = static_cast<const uint16_t*>(k_weight);
  a.cos = static_cast<const uint16_t*>(cos);
  a.sin = static_cast<const uint16_t*>(sin);
  a.eps = eps;
  // The plain form appends nothing: k, v and slot_mapping are ignored without the prologue.
  a.slot_mapping = prologue ? slot_mapping : nullptr;
  a.slot_stride = slot_stride;
  a.num_slots = num_blocks * kBlockSize;
  a.key_pool = static_cast<uint16_t*>(key_pool);
  a.value_pool = static_cast<uint16_t*>(value_pool);
  a.num_blocks = num_blocks;
  a.kv_heads = num_kv_heads;
  a.block_tables = block_tables;
  a.bt_stride = block_table_stride;
  a.max_blocks = max_blocks;
  a.context_lens = context_lens;
  a.ctx_stride = context_lens_stride;
  a.scale = scale;
  const int64_t tokens = static_cast<int64_t>(max_blocks) * kBlockSize;
  a.cache_tokens = tokens * group * static_cast<int64_t>(sizeof(uint16_t)) <= kDecCacheBytes ? static_cast<int32_t>(tokens) : 0;
  hipStream_t s = as_stream(stream);
  if (workspace_bytes < 0 || (workspace_bytes > 0 && !workspace))
    return fail(MI_ERR_INVALID_ARGUMENT, "%s: bad workspace", what);
  if (workspace) {  // the split form when the batch is small enough to gain from it
    const ExactSplitLayout layout = exact_split_layout(batch, max_blocks, num_heads, num_kv_heads);
    if (layout.splits > 1) {
      if (workspace_bytes < layout.bytes)
        return fail(MI_ERR_WORKSPACE, "%s: workspace of %lld bytes, the split form needs %lld", what,
                    static_cast<long long>(workspace_bytes), static_cast<long long>(layout.bytes));
      if (reinterpret_cast<uintptr_t>(workspace) % 256 != 0)
        return fail(MI_ERR_INVALID_ARGUMENT, "%s: workspace must be 256-byte aligned", what);
      ExactSplitArgs sa{};
      sa.d = a;
      sa.d.cache_tokens = 0;
      sa.scores = static_cast<uint16_t*>(workspace);
      sa.partial = reinterpret_cast<double*>(static_cast<char*>(workspace) + layout.scores_bytes);
      sa.ctx_cap = static_cast<int32_t>(tokens);
      sa.splits = layout.splits;
      const int32_t rc = prologue ? dispatch_exact_split<true>(sa, batch, group, s)
                                  : dispatch_exact_split<false>(sa, batch, group, s);
      return rc == MI_OK ? ok() : rc;
    }
  }
  // One launch per 65535 sequences (grid y holds the KV heads, x the sequences).
  for (int32_t b0 = 0; b0 < batch; b0 += 65535) {
    const int32_t nb = batch - b0 < 65535 ? batch - b0 : 65535;
    ExactDecodeArgs c = a;
    c.out = a.out + b0 * out_row_stride;
    c.q = a.q + b0 * q_row_stride;
    c.context_lens = context_lens + b0 * context_lens_stride;
    c.block_tables = block_tables ? block_tables + b0 * block_table_stride : nullptr;
    if (prologue) {
      c.k_new = a.k_new + b0 * k_row_stride;
      c.v_new = a.v_new + b0 * v_row_stride;
      c.cos = a.cos + b0 * static_cast<int64_t>(head_dim);
      c.sin = a.sin + b0 * static_cast<int64_t>(head_dim);
      c.slot_mapping = slot_mapping + b0 * slot_stride;
    }
    const int32_t rc = prologue ? dispatch_exact_decode<true>(c, nb, group, s) : dispatch_exact_decode<false>(c, nb, group, s);
    if (rc != MI_OK) return rc;
  }
  return ok();
}

extern "C" int64_t mi_paged_decode_exact_workspace_bytes(int32_t batch, int32_t max_blocks, int32_t num_heads,
                                                         int32_t num_kv_heads) {
  return mi::exact_split_layout(batch, max_blocks, num_heads, num_kv_heads).bytes;
}

extern "C" int32_t mi_chunked_prefill_attention_exact(
    void* out, int64_t out_row_stride, int64_t out_tok_stride, const void* query, int64_t query_row_stride,
    int64_t query_head_stride, int64_t query_tok_stride, const void* key, int64_t key_row_stride,
    int64_t key_head_stride, int64_t key_tok_stride, const void* value, int64_t value_row_stride,
    int64_t value_head_stride, int64_t value_tok_stride, const void* key_pool, const void* value_pool,
    int64_t num_blocks, const int64_t* history_blocks, int64_t history_stride, int32_t max_history_blocks,
    const int64_t* start_lens, const int64_t* chunk_lens, int64_t lens_stride, int32_t batch, int32_t padded_len,
    int32_t num_heads, int32_t num_kv_heads, int32_t head_dim, int32_t block_size, float scale, void* stream) {
  using namespace mi;
  const char* what = "mi_chunked_prefill_attention_exact";
  if (batch < 0 || padded_len < 0 || max_history_blocks < 0 || num_blocks < 0)
    return fail(MI_ERR_INVALID_ARGUMENT, "%s: negative size", what);
  if (batch == 0 || padded_len == 0) return ok();
  if (const int32_t rc = reject_empty_pool(what, num_blocks, max_history_blocks > 0)) return rc;
  if (const int32_t rc = check_exact_heads(what, num_heads, num_kv_heads, head_dim, block_size)) return rc;
  if (!out || !query || !key || !value || !start_lens || !chunk_lens ||
      (max_history_blocks > 0 && (!history_blocks || !key_pool || !value_pool)))
    return fail(MI_ERR_INVALID_ARGUMENT, "%s: null pointer argument", what);
  if (!aligned16(out) || !aligned16(key) || !aligned16(value) || (max_history_blocks > 0 &&
      (!aligned16(key_pool) || !aligned16(value_pool))) || out_row_stride % 8 != 0 || out_tok_stride % 8 != 0 ||
      key_row_stride % 8 != 0 || key_head_stride % 8 != 0 || key_tok_stride % 8 != 0 || value_row_stride % 8 != 0 ||
      value_head_stride % 8 != 0 || value_tok_stride % 8 != 0)
    return fail(MI_ERR_UNSUPPORTED, "%s: out / key / value / pools need 16-byte alignment and strides of 8 elements", what);
  if (lens_stride <= 0 || (max_history_blocks > 0 && history_stride < max_history_blocks))
    return fail(MI_ERR_INVALID_ARGUMENT, "%s: bad stride", what);
  if (batch > 65535 || num_kv_heads > 65535) return fail(MI_ERR_UNSUPPORTED, "%s: batch above 65535", what);
  const int group = num_heads / num_kv_heads;
  ExactPrefillArgs a{};
  a.out = static_cast<uint16_t*>(out);
  a.out_row = out_row_stride;
  a.out_tok = out_tok_stride;
  a.q = static_cast<const uint16_t*>(query);
  a.q_row = query_row_stride;
  a.q_head = query_head_stride;
  a.q_tok = query_tok_stride;
  a.k = static_cast<const uint16_t*>(key);
  a.k_row = key_row_stride;
  a.k_head = key_head_stride;
  a.k_tok = key_tok_stride;
  a.v = static_cast<const uint16_t*>(value);
  a.v_row = value_row_stride;
  a.v_head = value_head_stride;
  a.v_tok = value_tok_stride;
  a.key_pool = static_cast<uint16_t*>(const_cast<void*>(key_pool));
  a.value_pool = static_cast<uint16_t*>(const_cast<void*>(value_pool));
  a.num_blocks = num_blocks;
  a.history = history_blocks;
  a.hist_stride = history_stride;
  a.max_hist_blocks = max_history_blocks;
  a.start_lens = start_lens;
  a.chunk_lens = chunk_lens;
  a.lens_stride = lens_stride;
  a.q_vec = aligned16(query) && query_row_stride % 8 == 0 && query_head_stride % 8 == 0 && query_tok_stride % 8 == 0;
  // Keys a row can see: its history (at most the table's) plus the chunk up to it.
  exact_rows(a, batch, padded_len, num_heads, num_kv_heads,
             static_cast<int64_t>(max_history_blocks) * kBlockSize + padded_len, scale);
  const int32_t rc = dispatch_exact_prefill(a, ExactPrefillArgs{}, group, what, as_stream(stream));
  return rc == MI_OK ? ok() : rc;
}

extern "C" int32_t mi_mixed_paged_attention_exact(
    void* out, int64_t out_tok_stride, const void* query, int64_t query_tok_stride, int64_t query_head_stride,
    const void* key, int64_t key_tok_stride, int64_t key_head_stride, const void* value, int64_t value_tok_stride,
    int64_t value_head_stride, void* key_pool, void* value_pool, int64_t num_blocks, int32_t prefill_rows,
    int32_t prefill_width, int64_t chunk_tokens, const int64_t* chunk_first, const int64_t* history_blocks,
    int64_t history_stride, int32_t max_history_blocks, const int64_t* start_lens, const int64_t* chunk_lens,
    int64_t lens_stride, int32_t decode_rows, const int64_t* block_tables, int64_t block_table_stride,
    int32_t max_blocks, const int64_t* context_lens, int64_t context_lens_stride, const int64_t* slot_mapping,
    int64_t slot_stride, int32_t num_heads, int32_t num_kv_heads, int32_t head_dim, int32_t block_size, float scale,
    void* stream) {
  using namespace mi;
  const char* what = "mi_mixed_paged_attention_exact";
  if (prefill_rows < 0 || prefill_width < 0 || decode_rows < 0 || max_history_blocks < 0 || max_blocks < 0 ||
      num_blocks < 0 || (chunk_first && chunk_tokens < 0))
    return fail(MI_ERR_INVALID_ARGUMENT, "%s: negative size", what);
  const bool chunks = prefill_rows > 0 && prefill_width > 0;
  const bool ragged = chunk_first && chunk_tokens > 0;  // writes a zero row for every uncovered token
  if (!chunks && decode_rows == 0 && !ragged) return ok();
  if (const int32_t rc = reject_empty_pool(what, num_blocks, (chunks && max_history_blocks > 0) ||
                                                                 (decode_rows > 0 && max_blocks > 0)))
    return rc;
  if (const int32_t rc = check_exact_heads(what, num_heads, num_kv_heads, head_dim, block_size)) return rc;
  const bool pools = decode_rows > 0 || max_history_blocks > 0;
  if (!out || !query || !key || !value || (chunks && (!start_lens || !chunk_lens)) ||
      (chunks && max_history_blocks > 0 && !history_blocks) ||
      (decode_rows > 0 && (!context_lens || !slot_mapping || (max_blocks > 0 && !block_tables))) ||
      (pools && (!key_pool || !value_pool)))
    return fail(MI_ERR_INVALID_ARGUMENT, "%s: null pointer argument", what);
  if (!aligned16(out) || !aligned16(key) || !aligned16(value) || (pools && (!aligned16(key_pool) || !aligned16(value_pool))) ||
      out_tok_stride % 8 != 0 || key_tok_stride % 8 != 0 || key_head_stride % 8 != 0 || value_tok_stride % 8 != 0 ||
      value_head_stride % 8 != 0)
    return fail(MI_ERR_UNSUPPORTED, "%s: out / key / value / pools need 16-byte alignment and strides of 8 elements", what);
  if ((chunks && (lens_stride <= 0 || (max_history_blocks > 0 && history_stride < max_history_blocks))) ||
      (decode_rows > 0 && (context_lens_stride <= 0 || slot_stride <= 0 ||
                           (max_blocks > 0 && block_table_stride < max_blocks))))
    return fail(MI_ERR_INVALID_ARGUMENT, "%s: bad stride", what);
  if (prefill_rows > 65535 || decode_rows > 65535) return fail(MI_ERR_UNSUPPORTED, "%s: more than 65535 rows", what);
  if (num_blocks > INT64_MAX / (kBlockSize * static_cast<int64_t>(num_kv_heads) * head_dim))
    return fail(MI_ERR_INVALID_ARGUMENT, "%s: pool too large", what);

  // Chunk rows: tokens [0, P L), row b at token b L, or with chunk_first the ragged rows of tokens
  // [0, chunk_tokens).  Decode rows: the D tokens after them, one each.
  const int64_t n = chunk_first ? chunk_tokens : (chunks ? static_cast<int64_t>(prefill_rows) * prefill_width : 0);
  auto fill = [&](ExactPrefillArgs& a, int64_t tok0, int64_t row_tokens) {
    a.out = static_cast<uint16_t*>(out) + tok0 * out_tok_stride;
    a.out_row = row_tokens * out_tok_stride;
    a.out_tok = out_tok_stride;
    a.q = static_cast<const uint16_t*>(query) + tok0 * query_tok_stride;
    a.q_row = row_tokens * query_tok_stride;
    a.q_head = query_head_stride;
    a.q_tok = query_tok_stride;
    a.k = static_cast<const uint16_t*>(key) + tok0 * key_tok_stride;
    a.k_row = row_tokens * key_tok_stride;
    a.k_head = key_head_stride;
    a.k_tok = key_tok_stride;
    a.v = static_cast<const uint16_t*>(value) + tok0 * value_tok_stride;
    a.v_row = row_tokens * value_tok_stride;
    a.v_head = value_head_stride;
    a.v_tok = value_tok_stride;
    a.key_pool = static_cast<uint16_t*>(key_pool);
    a.value_pool = static_cast<uint16_t*>(value_pool);
    a.num_blocks = num_blocks;
  };
  ExactPrefillArgs a0{};
  if (chunks) {
    fill(a0, 0, prefill_width);
    a0.q_vec = aligned16(query) && query_tok_stride % 8 == 0 && query_head_stride % 8 == 0;
    a0.history = history_blocks;
    a0.hist_stride = history_stride;
    a0.max_hist_blocks = max_history_blocks;
    a0.start_lens = start_lens;
    a0.chunk_lens = chunk_lens;
    a0.lens_stride = lens_stride;
    a0.row_first = chunk_first;
    a0.row_tokens = chunk_tokens;
    exact_rows(a0, prefill_rows, prefill_width, num_heads, num_kv_heads,
               static_cast<int64_t>(max_history_blocks) * kBlockSize + prefill_width, scale);
  } else {
    a0.kv_heads = num_kv_heads;
  }
  // Decode rows: one-token chunks at the D tokens after the chunk rows, whose history is the
  // context minus the token (the block table), appending each row's rotated K/V to its slot.
  const int group = num_heads / num_kv_heads;
  ExactPrefillArgs a1{};
  if (decode_rows > 0) {
    fill(a1, n, 1);
    a1.q_vec = aligned16(query) && query_tok_stride % 8 == 0 && query_head_stride % 8 == 0;
    a1.history = block_tables;
    a1.hist_stride = block_table_stride;
    a1.max_hist_blocks = max_blocks;
    a1.start_lens = context_lens;
    a1.chunk_lens = context_lens;
    a1.lens_stride = context_lens_stride;
    a1.decode_rows = 1;
    a1.slot_mapping = slot_mapping;
    a1.slot_stride = slot_stride;
    exact_rows(a1, decode_rows, 1, num_heads, num_kv_heads, static_cast<int64_t>(max_blocks) * kBlockSize + 1, scale);
  }
  if (ragged) {
    if (const int32_t rc = zero_uncovered_tokens(what, out, out_tok_stride, num_heads * head_dim, chunk_first, chunk_lens,
                                                 lens_stride, chunks ? prefill_rows : 0, prefill_width, chunk_tokens,
                                                 stream))
      return rc;
  }
  const int32_t rc = dispatch_exact_prefill(a0, a1, group, what, as_stream(stream));
  return rc == MI_OK ? ok() : rc;
}
