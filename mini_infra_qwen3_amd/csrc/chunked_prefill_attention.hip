// Kernel 4: chunked-prefill attention on MFMA, history read straight from the paged pool.
//
// Behaviour of a chunked-prefill layer of the reference: the history gather of
// PagedKVCachePool.gather_blocks (src/mini_infra/worker/paged_kv_cache.py:54-72), the concat of
// history and chunk in Qwen3Attention.forward (src/mini_infra/model/qwen3.py:325-330), the visibility
// mask of PagedRunner.run_prefill_chunk_step (src/mini_infra/worker/paged_runner.py:179-187) with the
// causal mask of Qwen3Model._prepare_position_ids_and_allowed_mask (qwen3.py:477-484), and
// Qwen3Attention._attend (qwen3.py:219-255) -- as one flash-style kernel.
//
// Row b of the batch: chunk of padded length L whose last len_b positions are real (left
// padding), logical start start_b, history = the first nh = min(start_b, 16 * max_history_blocks)
// pool slots of its block table.  Query i (i >= L - len_b) sees every history slot k < nh and
// chunk keys j with L - len_b <= j <= i.  Rows i < L - len_b (padding) get a zero output.
//
// Tiling for gfx950 (v_mfma_f32_16x16x32_bf16, 64-lane wavefronts):
//  * workgroup = (row b, KV head g, 64-query tile), 4 wavefronts: wave w serves query head
//    2 g + (w >> 1) and queries [32 (w & 1), +32) of the tile, so the two GQA heads share
//    every K/V tile staged in LDS.
//  * KV tiles of 64 keys: history tiles first (pool blocks through the block table -- the
//    gather is fused, nothing is materialised), then chunk tiles up to the causal limit.
//    K is staged row-major, V transposed (V^T) in double-buffered LDS; the next tile's global
//    loads are in flight while the current one is multiplied.
//  * S^T = K Q^T: A = K rows from LDS, B = Q^T from registers (loaded once), C lane layout =
//    (query = lane % 16, keys 4 (lane / 16) + i).  Each query's softmax state lives in the
//    lanes of its column; the row max needs two cross-lane steps, the row sum is deferred.
//  * O^T = V^T P^T: the probabilities of a 32-key step are already in the B-operand lanes if
//    the MFMA's k index is read as key 16 (k' / 4) + 4 (lane / 16) + k' % 4; the A operand
//    (V^T) is read from LDS with the same permutation (two 8-byte reads).
//  * Scores keep the reference's bf16 rounding points (bf16 product, bf16 scale); softmax
//    and accumulation are fp32; lazy rescaling of the running max as in the decode kernel.
#include "mi_common.h"

namespace mi {
namespace {

constexpr int kHeadDim = 128;
constexpr int kBlockSize = 16;
constexpr int kGroup = 2;
constexpr int kQTile = 64;                 // queries per head per workgroup
constexpr int kKTile = 64;                 // keys per KV tile
constexpr int kKStride = kHeadDim + 8;     // LDS row of K (elements): 272 B
constexpr int kVStride = kKTile + 4;       // LDS row of V^T (elements): 136 B
constexpr int kThreads = 256;
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kRescaleSlack = 8.0f;

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x8 __attribute__((ext_vector_type(8)));

struct PrefillArgs {
  uint16_t* out;
  int64_t out_row, out_tok;                 // elements
  const uint16_t* query;
  int64_t q_row, q_head, q_tok;
  const uint16_t* key;
  int64_t k_row, k_head, k_tok;
  const uint16_t* value;
  int64_t v_row, v_head, v_tok;
  const uint16_t* key_pool;
  const uint16_t* value_pool;
  int64_t num_blocks;
  const int64_t* history_blocks;
  int64_t history_stride;
  int32_t max_history_blocks;
  const int64_t* start_lens;
  const int64_t* chunk_lens;
  int64_t lens_stride;
  int32_t padded_len;
  float scale;
};

__device__ __forceinline__ float score_log2(float dot, float scale) {
  const float s = static_cast<float>(static_cast<__bf16>(static_cast<float>(static_cast<__bf16>(dot)) * scale));
  return s * kLog2e;
}

__device__ __forceinline__ uint32_t perm(uint32_t hi_src, uint32_t lo_src, uint32_t sel) {
  return __builtin_amdgcn_perm(hi_src, lo_src, sel);
}

template <int kKvHeads>
__global__ __launch_bounds__(kThreads, 2) void chunked_prefill_kernel(const PrefillArgs a) {
  __shared__ __align__(16) uint16_t sK[2][kKTile * kKStride];
  __shared__ __align__(16) uint16_t sV[2][kHeadDim * kVStride];

  const int b = blockIdx.z;
  const int g = blockIdx.y;
  const int qt = gridDim.x - 1 - blockIdx.x;  // heaviest (latest) query tiles start first
  const int q0 = qt * kQTile;
  const int L = a.padded_len;
  int64_t len64 = a.chunk_lens[b * a.lens_stride];
  len64 = len64 < 0 ? 0 : (len64 > L ? L : len64);
  const int pad = L - static_cast<int>(len64);
  int64_t start64 = a.start_lens[b * a.lens_stride];
  start64 = start64 < 0 ? 0 : start64;
  const int64_t hist_cap = static_cast<int64_t>(a.max_history_blocks) * kBlockSize;
  const int nh = static_cast<int>(start64 < hist_cap ? start64 : hist_cap);

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int w = tid >> 6;
  const int hh = w >> 1;
  const int qs = w & 1;
  const int h = g * kGroup + hh;
  const int ql = lane & 15;
  const int gq = lane >> 4;

  uint16_t* out_b = a.out + b * a.out_row;
  if (q0 + kQTile <= pad) {  // the whole tile is padding: zero rows
    for (int c = tid; c < kQTile * kGroup * (kHeadDim / 8); c += kThreads) {
      const int qi = q0 + c / (kGroup * (kHeadDim / 8));
      const int rem = c % (kGroup * (kHeadDim / 8));
      const int head = g * kGroup + rem / (kHeadDim / 8);
      if (qi < L)
        *reinterpret_cast<uint4*>(out_b + qi * a.out_tok + head * kHeadDim + (rem % (kHeadDim / 8)) * 8) =
            uint4{0, 0, 0, 0};
    }
    return;
  }

  // ---- Q^T fragments (B operand): query column n = ql of n-tile nt, dims 32 ks + 8 gq .. +8
  bf16x8 qf[2][4];
  const int qw0 = q0 + 32 * qs;  // first query of this wave
#pragma unroll
  for (int nt = 0; nt < 2; ++nt) {
    const int qi = qw0 + 16 * nt + ql;
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      uint4 v = uint4{0, 0, 0, 0};
      if (qi < L) v = *reinterpret_cast<const uint4*>(a.query + b * a.q_row + h * a.q_head + qi * a.q_tok + ks * 32 + gq * 8);
      qf[nt][ks] = __builtin_bit_cast(bf16x8, v);
    }
  }

  const int n_hist_tiles = (nh + kKTile - 1) / kKTile;
  const int c_lo = pad / kKTile;
  const int last_q = min(q0 + kQTile, L) - 1;
  const int c_hi = last_q / kKTile;
  const int n_tiles = n_hist_tiles + (c_hi - c_lo + 1);

  // ---- tile loader: thread owns 4 K pieces (key, 8 dims) and 2 V key-pairs (2 keys, 8 dims)
  uint4 kreg[4], vreg[2][2];
  auto src_row = [&](int t, int key, bool is_value, bool& ok) -> const uint16_t* {
    if (t < n_hist_tiles) {
      const int kpos = t * kKTile + key;
      ok = kpos < nh;
      if (!ok) return nullptr;
      int64_t bid = a.history_blocks[b * a.history_stride + kpos / kBlockSize];
      if (bid < 0 || bid >= a.num_blocks) bid = 0;
      const uint16_t* pool = is_value ? a.value_pool : a.key_pool;
      return pool + ((bid * kBlockSize + kpos % kBlockSize) * kKvHeads + g) * kHeadDim;
    }
    const int j = (c_lo + t - n_hist_tiles) * kKTile + key;
    ok = j < L;
    if (!ok) return nullptr;
    return is_value ? a.value + b * a.v_row + g * a.v_head + j * a.v_tok
                    : a.key + b * a.k_row + g * a.k_head + j * a.k_tok;
  };
  auto load_tile = [&](int t) {
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
      const int c = tid + kThreads * kk;
      bool ok;
      const uint16_t* p = src_row(t, c >> 4, false, ok);
      kreg[kk] = ok ? *reinterpret_cast<const uint4*>(p + (c & 15) * 8) : uint4{0, 0, 0, 0};
    }
#pragma unroll
    for (int kk = 0; kk < 2; ++kk) {
      const int it = tid + kThreads * kk;
      const int kp = it >> 4, dg = it & 15;
#pragma unroll
      for (int e = 0; e < 2; ++e) {
        bool ok;
        const uint16_t* p = src_row(t, 2 * kp + e, true, ok);
        vreg[kk][e] = ok ? *reinterpret_cast<const uint4*>(p + dg * 8) : uint4{0, 0, 0, 0};
      }
    }
  };
  auto store_tile = [&](int buf) {
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
      const int c = tid + kThreads * kk;
      *reinterpret_cast<uint4*>(&sK[buf][(c >> 4) * kKStride + (c & 15) * 8]) = kreg[kk];
    }
#pragma unroll
    for (int kk = 0; kk < 2; ++kk) {
      const int it = tid + kThreads * kk;
      const int kp = it >> 4, dg = it & 15;
      const uint32_t x[4] = {vreg[kk][0].x, vreg[kk][0].y, vreg[kk][0].z, vreg[kk][0].w};
      const uint32_t y[4] = {vreg[kk][1].x, vreg[kk][1].y, vreg[kk][1].z, vreg[kk][1].w};
#pragma unroll
      for (int d2 = 0; d2 < 4; ++d2) {
        // dims 2 d2 and 2 d2 + 1 of keys (2 kp, 2 kp + 1) -> two V^T words
        const uint32_t lo = perm(y[d2], x[d2], 0x05040100u);
        const uint32_t hi = perm(y[d2], x[d2], 0x07060302u);
        *reinterpret_cast<uint32_t*>(&sV[buf][(dg * 8 + 2 * d2) * kVStride + 2 * kp]) = lo;
        *reinterpret_cast<uint32_t*>(&sV[buf][(dg * 8 + 2 * d2 + 1) * kVStride + 2 * kp]) = hi;
      }
    }
  };

  f32x4 oacc[8][2];
#pragma unroll
  for (int dt = 0; dt < 8; ++dt)
#pragma unroll
    for (int nt = 0; nt < 2; ++nt) oacc[dt][nt] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  float m_run[2] = {-INFINITY, -INFINITY};
  float l_part[2] = {0.0f, 0.0f};
  const float scale = a.scale;

  if (n_tiles > 0) {
    load_tile(0);
    store_tile(0);
  }
  __syncthreads();

  for (int t = 0; t < n_tiles; ++t) {
    const int buf = t & 1;
    if (t + 1 < n_tiles) load_tile(t + 1);

    // ---- S^T = K Q^T for 64 keys x 32 queries
    f32x4 sacc[4][2];
#pragma unroll
    for (int mt = 0; mt < 4; ++mt)
#pragma unroll
      for (int nt = 0; nt < 2; ++nt) sacc[mt][nt] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
#pragma unroll
      for (int mt = 0; mt < 4; ++mt) {
        const bf16x8 kf = *reinterpret_cast<const bf16x8*>(&sK[buf][(mt * 16 + ql) * kKStride + ks * 32 + gq * 8]);
#pragma unroll
        for (int nt = 0; nt < 2; ++nt)
          sacc[mt][nt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kf, qf[nt][ks], sacc[mt][nt], 0, 0, 0);
      }
    }

    // ---- scores, masks (uniform branch: only edge tiles need them)
    const bool is_hist = t < n_hist_tiles;
    const int key0 = is_hist ? t * kKTile : (c_lo + t - n_hist_tiles) * kKTile;
    bool need_mask;
    if (is_hist) {
      need_mask = key0 + kKTile > nh || qw0 < pad || qw0 + 31 >= L;
    } else {
      need_mask = key0 + kKTile - 1 > qw0 || key0 < pad || qw0 < pad || qw0 + 31 >= L;
    }
#pragma unroll
    for (int mt = 0; mt < 4; ++mt)
#pragma unroll
      for (int nt = 0; nt < 2; ++nt)
#pragma unroll
        for (int i = 0; i < 4; ++i) sacc[mt][nt][i] = score_log2(sacc[mt][nt][i], scale);
    if (need_mask) {
#pragma unroll
      for (int nt = 0; nt < 2; ++nt) {
        const int qi = qw0 + 16 * nt + ql;
        const bool row_ok = qi >= pad && qi < L;
#pragma unroll
        for (int mt = 0; mt < 4; ++mt)
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const int kpos = key0 + mt * 16 + 4 * gq + i;
            const bool vis = row_ok && (is_hist ? kpos < nh : (kpos >= pad && kpos <= qi));
            sacc[mt][nt][i] = vis ? sacc[mt][nt][i] : -INFINITY;
          }
      }
    }

    // ---- online softmax per query column (lanes ql, ql+16, ql+32, ql+48 hold its 64 keys)
    float mx[2];
#pragma unroll
    for (int nt = 0; nt < 2; ++nt) {
      float v = -INFINITY;
#pragma unroll
      for (int mt = 0; mt < 4; ++mt)
#pragma unroll
        for (int i = 0; i < 4; ++i) v = fmaxf(v, sacc[mt][nt][i]);
      v = fmaxf(v, __shfl_xor(v, 16));
      v = fmaxf(v, __shfl_xor(v, 32));
      mx[nt] = v;
    }
    const bool grow = mx[0] > m_run[0] + kRescaleSlack || mx[1] > m_run[1] + kRescaleSlack;
    if (__builtin_amdgcn_ballot_w64(grow) != 0) {
#pragma unroll
      for (int nt = 0; nt < 2; ++nt) {
        const float mn = fmaxf(m_run[nt], mx[nt]);
        const float alpha = mn == -INFINITY ? 1.0f : __builtin_amdgcn_exp2f(m_run[nt] - mn);
        m_run[nt] = mn;
        l_part[nt] *= alpha;
#pragma unroll
        for (int dt = 0; dt < 8; ++dt) oacc[dt][nt] *= alpha;
      }
    }
    bf16x8 pf[2][2];  // [nt][ks2]
#pragma unroll
    for (int nt = 0; nt < 2; ++nt) {
      const float ref = m_run[nt] == -INFINITY ? 0.0f : m_run[nt];
      float sum = 0.0f;
#pragma unroll
      for (int mt = 0; mt < 4; ++mt)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float p = __builtin_amdgcn_exp2f(sacc[mt][nt][i] - ref);
          sacc[mt][nt][i] = p;
          sum += p;
        }
      l_part[nt] += sum;
#pragma unroll
      for (int ks2 = 0; ks2 < 2; ++ks2) {
        const f32x8 pv = {sacc[2 * ks2][nt][0], sacc[2 * ks2][nt][1], sacc[2 * ks2][nt][2], sacc[2 * ks2][nt][3],
                          sacc[2 * ks2 + 1][nt][0], sacc[2 * ks2 + 1][nt][1], sacc[2 * ks2 + 1][nt][2],
                          sacc[2 * ks2 + 1][nt][3]};
        pf[nt][ks2] = __builtin_convertvector(pv, bf16x8);
      }
    }

    // ---- O^T += V^T P^T
#pragma unroll
    for (int ks2 = 0; ks2 < 2; ++ks2) {
#pragma unroll
      for (int dt = 0; dt < 8; ++dt) {
        const uint16_t* vrow = &sV[buf][(dt * 16 + ql) * kVStride + 32 * ks2 + 4 * gq];
        const bf16x4 v0 = *reinterpret_cast<const bf16x4*>(vrow);
        const bf16x4 v1 = *reinterpret_cast<const bf16x4*>(vrow + 16);
        const bf16x8 vf = {v0[0], v0[1], v0[2], v0[3], v1[0], v1[1], v1[2], v1[3]};
#pragma unroll
        for (int nt = 0; nt < 2; ++nt)
          oacc[dt][nt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(vf, pf[nt][ks2], oacc[dt][nt], 0, 0, 0);
      }
    }

    if (t + 1 < n_tiles) store_tile(buf ^ 1);
    __syncthreads();
  }

  // ---- normalise and write: lane holds query qw0 + 16 nt + ql, dims 16 dt + 4 gq + i
#pragma unroll
  for (int nt = 0; nt < 2; ++nt) {
    float lt = l_part[nt];
    lt += __shfl_xor(lt, 16);
    lt += __shfl_xor(lt, 32);
    const float inv = lt > 0.0f ? 1.0f / lt : 0.0f;
    const int qi = qw0 + 16 * nt + ql;
    if (qi >= L) continue;
    uint16_t* orow = out_b + qi * a.out_tok + h * kHeadDim + 4 * gq;
#pragma unroll
    for (int dt = 0; dt < 8; ++dt) {
      uint2 v;
      v.x = pack_bf16x2(oacc[dt][nt][0] * inv, oacc[dt][nt][1] * inv);
      v.y = pack_bf16x2(oacc[dt][nt][2] * inv, oacc[dt][nt][3] * inv);
      *reinterpret_cast<uint2*>(orow + dt * 16) = v;
    }
  }
}

}  // namespace
}  // namespace mi

extern "C" int32_t mi_chunked_prefill_attention(
    void* out, int64_t out_row_stride, int64_t out_tok_stride, const void* query, int64_t query_row_stride,
    int64_t query_head_stride, int64_t query_tok_stride, const void* key, int64_t key_row_stride,
    int64_t key_head_stride, int64_t key_tok_stride, const void* value, int64_t value_row_stride,
    int64_t value_head_stride, int64_t value_tok_stride, const void* key_pool, const void* value_pool,
    int64_t num_blocks, const int64_t* history_blocks, int64_t history_stride, int32_t max_history_blocks,
    const int64_t* start_lens, const int64_t* chunk_lens, int64_t lens_stride, int32_t batch, int32_t padded_len,
    int32_t num_heads, int32_t num_kv_heads, int32_t head_dim, int32_t block_size, float scale, void* stream) {
  using namespace mi;
  if (batch < 0 || padded_len < 0 || max_history_blocks < 0 || num_blocks < 0)
    return fail(MI_ERR_INVALID_ARGUMENT, "mi_chunked_prefill_attention: negative size");
  if (batch == 0 || padded_len == 0) return ok();
  if (!out || !query || !key || !value || !start_lens || !chunk_lens ||
      (max_history_blocks > 0 && (!history_blocks || !key_pool || !value_pool)))
    return fail(MI_ERR_INVALID_ARGUMENT, "mi_chunked_prefill_attention: null pointer argument");
  if (head_dim != kHeadDim || block_size != kBlockSize || num_kv_heads <= 0 || num_heads != kGroup * num_kv_heads)
    return fail(MI_ERR_UNSUPPORTED,
                "mi_chunked_prefill_attention: needs head_dim %d, block_size %d, num_heads = %d * num_kv_heads "
                "(got head_dim %d, block_size %d, heads %d/%d)",
                kHeadDim, kBlockSize, kGroup, head_dim, block_size, num_heads, num_kv_heads);
  if (num_kv_heads != 1 && num_kv_heads != 2 && num_kv_heads != 4 && num_kv_heads != 8)
    return fail(MI_ERR_UNSUPPORTED, "mi_chunked_prefill_attention: num_kv_heads %d not in {1,2,4,8}", num_kv_heads);
  const int64_t strides[] = {out_row_stride, out_tok_stride, query_row_stride, query_head_stride, query_tok_stride,
                             key_row_stride, key_head_stride, key_tok_stride, value_row_stride, value_head_stride,
                             value_tok_stride};
  for (int64_t s : strides)
    if (s % 8 != 0) return fail(MI_ERR_UNSUPPORTED, "mi_chunked_prefill_attention: strides must be multiples of 8");
  if (!aligned16(out) || !aligned16(query) || !aligned16(key) || !aligned16(value) ||
      (max_history_blocks > 0 && (!aligned16(key_pool) || !aligned16(value_pool))))
    return fail(MI_ERR_UNSUPPORTED, "mi_chunked_prefill_attention: tensors must be 16-byte aligned");
  if (max_history_blocks > 0 && history_stride < max_history_blocks)
    return fail(MI_ERR_INVALID_ARGUMENT, "mi_chunked_prefill_attention: history_stride < max_history_blocks");
  if (lens_stride <= 0) return fail(MI_ERR_INVALID_ARGUMENT, "mi_chunked_prefill_attention: lens_stride must be > 0");
  if (batch > 65535) return fail(MI_ERR_UNSUPPORTED, "mi_chunked_prefill_attention: batch > 65535");

  PrefillArgs a{};
  a.out = static_cast<uint16_t*>(out);
  a.out_row = out_row_stride;
  a.out_tok = out_tok_stride;
  a.query = static_cast<const uint16_t*>(query);
  a.q_row = query_row_stride;
  a.q_head = query_head_stride;
  a.q_tok = query_tok_stride;
  a.key = static_cast<const uint16_t*>(key);
  a.k_row = key_row_stride;
  a.k_head = key_head_stride;
  a.k_tok = key_tok_stride;
  a.value = static_cast<const uint16_t*>(value);
  a.v_row = value_row_stride;
  a.v_head = value_head_stride;
  a.v_tok = value_tok_stride;
  a.key_pool = static_cast<const uint16_t*>(key_pool);
  a.value_pool = static_cast<const uint16_t*>(value_pool);
  a.num_blocks = num_blocks;
  a.history_blocks = history_blocks;
  a.history_stride = history_stride;
  a.max_history_blocks = max_history_blocks;
  a.start_lens = start_lens;
  a.chunk_lens = chunk_lens;
  a.lens_stride = lens_stride;
  a.padded_len = padded_len;
  a.scale = scale;

  dim3 grid((padded_len + kQTile - 1) / kQTile, num_kv_heads, batch);
  hipStream_t s = as_stream(stream);
  switch (num_kv_heads) {
    case 1: chunked_prefill_kernel<1><<<grid, kThreads, 0, s>>>(a); break;
    case 2: chunked_prefill_kernel<2><<<grid, kThreads, 0, s>>>(a); break;
    case 4: chunked_prefill_kernel<4><<<grid, kThreads, 0, s>>>(a); break;
    default: chunked_prefill_kernel<8><<<grid, kThreads, 0, s>>>(a); break;
  }
  return check_launch("mi_chunked_prefill_attention");
}
