// Kernel 3: paged GQA decode attention (one query token per sequence).
//
// Behaviour of the reference's paged decode branch: the pool gather of
// Qwen3Attention._apply_paged_kv_pool (src/mini_infra/model/qwen3.py:285-292), the context-length
// bias of Qwen3Model._build_paged_inputs (:513-528) and Qwen3Attention._attend with
// _repeat_key_value (:219-255, :147-156) -- computed straight from the pool, without
// materialising the padded history or the repeated K/V.
//
// Work decomposition (MI355X: 256 CUs, 64-lane wavefronts, bandwidth-bound):
//  * A workgroup owns one sequence b, one partition of kPartBlocks pool blocks of its
//    context, and kWaves consecutive KV heads.  Wavefront w serves KV head g and both query
//    heads 2g, 2g+1 that share it (GQA group 2), so every K/V byte is loaded exactly once.
//  * Inside a wavefront, lane = 16 * row + dl.  Lane dl holds dims [8 dl, 8 dl + 8) of the
//    two query rows; row r owns tokens 4 i + r (i = 0..3) of every 16-token block.  One
//    16-byte load per lane per i brings four 256-byte (token, head) rows per instruction.
//  * QK^T: bf16 v_dot2 on packed pairs, then a 16-lane DPP butterfly (quad_perm, half-row
//    mirror, row mirror) leaves the full dot product in every lane of the row.
//  * Each row keeps its own online-softmax state (running max m, sum l, fp32 accumulator
//    of 2 heads x 8 dims), so no cross-row traffic happens inside the block loop.  The max
//    is rescaled lazily: only when a new score exceeds the running max by more than
//    kRescaleSlack (log2 units) -- exact, since l and the accumulator share the same m.
//  * PV: probabilities of token pairs are packed to bf16 and v_perm regroups V so that one
//    v_dot2 covers two tokens of one dim.
//  * K/V of the next kDepth-1 blocks are in flight in registers while the current block
//    is computed (a register ring: the VGPR file is 512 KiB per CU, LDS is 160 KiB).
//  * Rows merge at the end of the partition (log-sum-exp).  A sequence with one partition
//    writes bf16 output directly; otherwise (m, l, acc) go to the caller's workspace and
//    a second kernel merges partitions.
#include "mi_common.h"

namespace mi {
namespace {

constexpr int kHeadDim = 128;
constexpr int kBlockSize = 16;
constexpr int kGroup = 2;          // query heads per KV head
constexpr int kPartBlocks = 16;    // pool blocks per partition (256 tokens)
constexpr int kPartTokens = kPartBlocks * kBlockSize;
constexpr int kDepth = 2;          // register ring depth (blocks in flight incl. current)
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kRescaleSlack = 8.0f;

typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float f32x2 __attribute__((ext_vector_type(2)));

struct DecodeArgs {
  uint16_t* out;
  int64_t out_row;                 // elements
  const uint16_t* query;
  int64_t q_row, q_head;           // elements
  const uint16_t* key_pool;
  const uint16_t* value_pool;
  int64_t num_blocks;
  const int64_t* block_tables;
  int64_t bt_stride;
  const int64_t* context_lens;
  int64_t ctx_stride;
  int32_t max_blocks;
  int32_t max_parts;               // partitions per sequence the workspace is sized for
  float scale;                     // softmax scale (natural units)
  float* ws_acc;                   // [batch, max_parts, heads, 128]
  float* ws_ml;                    // [batch, max_parts, heads, 2] = (m, l) in log2 units
};

__device__ __forceinline__ float dpp_sum16(float x) {
  // Butterfly over the 16 lanes of a DPP row: xor 1, xor 2, 8-lane mirror, 16-lane mirror.
  x += __builtin_amdgcn_update_dpp(0.0f, x, 0xB1, 0xf, 0xf, false);   // quad_perm [1,0,3,2]
  x += __builtin_amdgcn_update_dpp(0.0f, x, 0x4E, 0xf, 0xf, false);   // quad_perm [2,3,0,1]
  x += __builtin_amdgcn_update_dpp(0.0f, x, 0x141, 0xf, 0xf, false);  // row_half_mirror
  x += __builtin_amdgcn_update_dpp(0.0f, x, 0x140, 0xf, 0xf, false);  // row_mirror
  return x;
}

__device__ __forceinline__ float dot8(const uint4 q, const uint4 k) {
  float d = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, q.x), __builtin_bit_cast(bf16x2, k.x), 0.0f, false);
  d = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, q.y), __builtin_bit_cast(bf16x2, k.y), d, false);
  d = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, q.z), __builtin_bit_cast(bf16x2, k.z), d, false);
  d = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, q.w), __builtin_bit_cast(bf16x2, k.w), d, false);
  return d;
}

// Reference rounding points: the bf16 matmul output, then the bf16 product with the
// scale (src/mini_infra/model/qwen3.py:243).  Returned in log2 units for exp2.
__device__ __forceinline__ float score_log2(float dot, float scale) {
  const float s = static_cast<float>(static_cast<__bf16>(static_cast<float>(static_cast<__bf16>(dot)) * scale));
  return s * kLog2e;
}

__device__ __forceinline__ uint32_t pack_p(float lo, float hi) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2){lo, hi}, bf16x2));
}

__device__ __forceinline__ float fdot2(uint32_t a, uint32_t b, float c) {
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, a), __builtin_bit_cast(bf16x2, b), c, false);
}

template <int kKvHeads, int kWaves>
__global__ __launch_bounds__(64 * kWaves) void paged_decode_kernel(const DecodeArgs a) {
  constexpr int kRowElems = kKvHeads * kHeadDim;     // elements of one pool row (token)
  constexpr int kBlockElems = kBlockSize * kRowElems;
  constexpr int kHeadGroups = kKvHeads / kWaves;
  constexpr int kHeads = kKvHeads * kGroup;

  const int b = blockIdx.y;
  const int part = blockIdx.x / kHeadGroups;
  const int g = (blockIdx.x - part * kHeadGroups) * kWaves + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const int dl = lane & 15;
  const int r = lane >> 4;

  int64_t n = a.context_lens[b * a.ctx_stride];
  n = min(n, static_cast<int64_t>(a.max_blocks) * kBlockSize);
  const int64_t t_begin = static_cast<int64_t>(part) * kPartTokens;
  if (t_begin >= n) {
    if (part == 0 && r < kGroup) {  // empty context: zero output row
      uint16_t* o = a.out + b * a.out_row + (g * kGroup + r) * kHeadDim + 8 * dl;
      *reinterpret_cast<uint4*>(o) = uint4{0, 0, 0, 0};
    }
    return;
  }
  const int nparts = static_cast<int>((n + kPartTokens - 1) / kPartTokens);
  const int blk0 = part * kPartBlocks;
  const int nblk = static_cast<int>(min(static_cast<int64_t>(kPartBlocks), (n - t_begin + kBlockSize - 1) / kBlockSize));

  // Block ids of this partition, one per lane; ids out of range read block 0.
  int64_t my_bid = 0;
  if (lane < nblk) {
    my_bid = a.block_tables[b * a.bt_stride + blk0 + lane];
    if (my_bid < 0 || my_bid >= a.num_blocks) my_bid = 0;
  }
  const uint32_t bid_lo = static_cast<uint32_t>(my_bid);
  const uint32_t bid_hi = static_cast<uint32_t>(static_cast<uint64_t>(my_bid) >> 32);

  const uint16_t* qp = a.query + b * a.q_row + (g * kGroup) * a.q_head + 8 * dl;
  const uint4 q0 = *reinterpret_cast<const uint4*>(qp);
  const uint4 q1 = *reinterpret_cast<const uint4*>(qp + a.q_head);

  // Lane offset (elements) of its piece of token 4 i + r inside a block.
  const int lane_off = r * kRowElems + g * kHeadDim + 8 * dl;

  auto block_base = [&](int j) -> int64_t {
    const uint32_t lo = __builtin_amdgcn_readlane(bid_lo, j);
    const uint32_t hi = __builtin_amdgcn_readlane(bid_hi, j);
    return static_cast<int64_t>((static_cast<uint64_t>(hi) << 32) | lo) * kBlockElems;
  };

  uint4 kbuf[kDepth][4], vbuf[kDepth][4];
  auto issue = [&](int slot, int j) {
    const int64_t base = block_base(min(j, nblk - 1));
    const uint16_t* kp = a.key_pool + base + lane_off;
    const uint16_t* vp = a.value_pool + base + lane_off;
#pragma unroll
    for (int i = 0; i < 4; ++i) kbuf[slot][i] = *reinterpret_cast<const uint4*>(kp + i * 4 * kRowElems);
#pragma unroll
    for (int i = 0; i < 4; ++i) vbuf[slot][i] = *reinterpret_cast<const uint4*>(vp + i * 4 * kRowElems);
  };

  float m0 = -INFINITY, m1 = -INFINITY, l0 = 0.0f, l1 = 0.0f;
  float acc0[8], acc1[8];
#pragma unroll
  for (int d = 0; d < 8; ++d) acc0[d] = acc1[d] = 0.0f;

  const float scale = a.scale;
#pragma unroll
  for (int s = 0; s < kDepth - 1; ++s) issue(s, s);

  for (int j0 = 0; j0 < nblk; j0 += kDepth) {
#pragma unroll
    for (int s = 0; s < kDepth; ++s) {
      const int j = j0 + s;
      if (j >= nblk) break;
      issue((s + kDepth - 1) % kDepth, j + kDepth - 1);

      // ---- scores of tokens 4 i + r of block j, both query heads
      const int64_t tok0 = t_begin + static_cast<int64_t>(j) * kBlockSize + r;
      float s0[4], s1[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float d0 = dpp_sum16(dot8(q0, kbuf[s][i]));
        const float d1 = dpp_sum16(dot8(q1, kbuf[s][i]));
        const bool valid = tok0 + 4 * i < n;
        s0[i] = valid ? score_log2(d0, scale) : -INFINITY;
        s1[i] = valid ? score_log2(d1, scale) : -INFINITY;
      }
      const float mb0 = fmaxf(fmaxf(s0[0], s0[1]), fmaxf(s0[2], s0[3]));
      const float mb1 = fmaxf(fmaxf(s1[0], s1[1]), fmaxf(s1[2], s1[3]));

      // ---- lazy rescale (wave-uniform branch)
      const bool grow = (mb0 > m0 + kRescaleSlack) || (mb1 > m1 + kRescaleSlack);
      if (__builtin_amdgcn_ballot_w64(grow) != 0) {
        const float n0 = fmaxf(m0, mb0), n1 = fmaxf(m1, mb1);
        const float a0 = (n0 == -INFINITY) ? 1.0f : __builtin_amdgcn_exp2f(m0 - n0);
        const float a1 = (n1 == -INFINITY) ? 1.0f : __builtin_amdgcn_exp2f(m1 - n1);
        m0 = n0;
        m1 = n1;
        l0 *= a0;
        l1 *= a1;
#pragma unroll
        for (int d = 0; d < 8; ++d) {
          acc0[d] *= a0;
          acc1[d] *= a1;
        }
      }
      float p0[4], p1[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        p0[i] = (s0[i] == -INFINITY) ? 0.0f : __builtin_amdgcn_exp2f(s0[i] - m0);
        p1[i] = (s1[i] == -INFINITY) ? 0.0f : __builtin_amdgcn_exp2f(s1[i] - m1);
      }
      l0 += (p0[0] + p0[1]) + (p0[2] + p0[3]);
      l1 += (p1[0] + p1[1]) + (p1[2] + p1[3]);

      // ---- P V over token pairs (0,1) and (2,3)
#pragma unroll
      for (int pr = 0; pr < 2; ++pr) {
        const uint32_t ph0 = pack_p(p0[2 * pr], p0[2 * pr + 1]);
        const uint32_t ph1 = pack_p(p1[2 * pr], p1[2 * pr + 1]);
        const uint4 va = vbuf[s][2 * pr];
        const uint4 vc = vbuf[s][2 * pr + 1];
        const uint32_t aw[4] = {va.x, va.y, va.z, va.w};
        const uint32_t cw[4] = {vc.x, vc.y, vc.z, vc.w};
#pragma unroll
        for (int w = 0; w < 4; ++w) {
          const uint32_t lo = __builtin_amdgcn_perm(cw[w], aw[w], 0x05040100u);  // (a.lo, c.lo)
          const uint32_t hi = __builtin_amdgcn_perm(cw[w], aw[w], 0x07060302u);  // (a.hi, c.hi)
          acc0[2 * w] = fdot2(ph0, lo, acc0[2 * w]);
          acc0[2 * w + 1] = fdot2(ph0, hi, acc0[2 * w + 1]);
          acc1[2 * w] = fdot2(ph1, lo, acc1[2 * w]);
          acc1[2 * w + 1] = fdot2(ph1, hi, acc1[2 * w + 1]);
        }
      }
    }
  }

  // ---- merge the four rows (log-sum-exp)
  float M0 = fmaxf(m0, __shfl_xor(m0, 16));
  M0 = fmaxf(M0, __shfl_xor(M0, 32));
  float M1 = fmaxf(m1, __shfl_xor(m1, 16));
  M1 = fmaxf(M1, __shfl_xor(M1, 32));
  const float w0 = (m0 == -INFINITY) ? 0.0f : __builtin_amdgcn_exp2f(m0 - M0);
  const float w1 = (m1 == -INFINITY) ? 0.0f : __builtin_amdgcn_exp2f(m1 - M1);
  l0 *= w0;
  l1 *= w1;
  l0 += __shfl_xor(l0, 16);
  l0 += __shfl_xor(l0, 32);
  l1 += __shfl_xor(l1, 16);
  l1 += __shfl_xor(l1, 32);
#pragma unroll
  for (int d = 0; d < 8; ++d) {
    acc0[d] *= w0;
    acc1[d] *= w1;
    acc0[d] += __shfl_xor(acc0[d], 16);
    acc0[d] += __shfl_xor(acc0[d], 32);
    acc1[d] += __shfl_xor(acc1[d], 16);
    acc1[d] += __shfl_xor(acc1[d], 32);
  }

  // Row 0 writes query head 2g, row 1 writes 2g + 1.
  if (r >= kGroup) return;
  const int h = g * kGroup + r;
  float o[8];
#pragma unroll
  for (int d = 0; d < 8; ++d) o[d] = r == 0 ? acc0[d] : acc1[d];
  if (nparts == 1) {
    const float inv = 1.0f / (r == 0 ? l0 : l1);
    uint4 v;
    v.x = pack_bf16x2(o[0] * inv, o[1] * inv);
    v.y = pack_bf16x2(o[2] * inv, o[3] * inv);
    v.z = pack_bf16x2(o[4] * inv, o[5] * inv);
    v.w = pack_bf16x2(o[6] * inv, o[7] * inv);
    *reinterpret_cast<uint4*>(a.out + b * a.out_row + h * kHeadDim + 8 * dl) = v;
  } else {
    const int64_t slot = (static_cast<int64_t>(b) * a.max_parts + part) * kHeads + h;
    float4* dst = reinterpret_cast<float4*>(a.ws_acc + slot * kHeadDim + 8 * dl);
    dst[0] = make_float4(o[0], o[1], o[2], o[3]);
    dst[1] = make_float4(o[4], o[5], o[6], o[7]);
    if (dl == 0) {
      a.ws_ml[slot * 2 + 0] = r == 0 ? M0 : M1;
      a.ws_ml[slot * 2 + 1] = r == 0 ? l0 : l1;
    }
  }
}

// Merge the partitions of sequences longer than one partition.
// grid: batch; block: heads * 16 lanes, lane (h, dl) owns dims [8 dl, 8 dl + 8) of head h.
template <int kHeads>
__global__ __launch_bounds__(kHeads * 16) void paged_decode_reduce_kernel(const DecodeArgs a) {
  const int b = blockIdx.x;
  const int h = threadIdx.x >> 4;
  const int dl = threadIdx.x & 15;
  int64_t n = a.context_lens[b * a.ctx_stride];
  n = min(n, static_cast<int64_t>(a.max_blocks) * kBlockSize);
  const int nparts = n <= 0 ? 0 : static_cast<int>((n + kPartTokens - 1) / kPartTokens);
  if (nparts <= 1) return;
  const int64_t base = static_cast<int64_t>(b) * a.max_parts * kHeads + h;
  float M = -INFINITY;
  for (int p = 0; p < nparts; ++p) M = fmaxf(M, a.ws_ml[(base + p * kHeads) * 2]);
  float L = 0.0f, o[8];
#pragma unroll
  for (int d = 0; d < 8; ++d) o[d] = 0.0f;
  for (int p = 0; p < nparts; ++p) {
    const int64_t slot = base + p * kHeads;
    const float m = a.ws_ml[slot * 2];
    const float w = (m == -INFINITY) ? 0.0f : __builtin_amdgcn_exp2f(m - M);
    L += w * a.ws_ml[slot * 2 + 1];
    const float4* src = reinterpret_cast<const float4*>(a.ws_acc + slot * kHeadDim + 8 * dl);
    const float4 x = src[0], y = src[1];
    o[0] += w * x.x; o[1] += w * x.y; o[2] += w * x.z; o[3] += w * x.w;
    o[4] += w * y.x; o[5] += w * y.y; o[6] += w * y.z; o[7] += w * y.w;
  }
  const float inv = 1.0f / L;
  uint4 v;
  v.x = pack_bf16x2(o[0] * inv, o[1] * inv);
  v.y = pack_bf16x2(o[2] * inv, o[3] * inv);
  v.z = pack_bf16x2(o[4] * inv, o[5] * inv);
  v.w = pack_bf16x2(o[6] * inv, o[7] * inv);
  *reinterpret_cast<uint4*>(a.out + b * a.out_row + h * kHeadDim + 8 * dl) = v;
}

template <int kKvHeads>
int32_t launch_decode(const DecodeArgs& a, int batch, hipStream_t s) {
  constexpr int kWaves = kKvHeads < 4 ? kKvHeads : 4;
  dim3 grid(a.max_parts * (kKvHeads / kWaves), batch);
  paged_decode_kernel<kKvHeads, kWaves><<<grid, 64 * kWaves, 0, s>>>(a);
  int32_t rc = check_launch("mi_paged_decode_attention");
  if (rc != MI_OK || a.max_parts <= 1) return rc;
  paged_decode_reduce_kernel<kKvHeads * kGroup><<<batch, kKvHeads * kGroup * 16, 0, s>>>(a);
  return check_launch("mi_paged_decode_attention(reduce)");
}

int64_t parts_for(int32_t max_blocks) { return (static_cast<int64_t>(max_blocks) + kPartBlocks - 1) / kPartBlocks; }

}  // namespace
}  // namespace mi

extern "C" int64_t mi_paged_decode_workspace_bytes(int32_t batch, int32_t max_blocks, int32_t num_heads,
                                                   int32_t head_dim, int32_t block_size) {
  if (batch <= 0 || max_blocks <= 0 || num_heads <= 0 || head_dim <= 0 || block_size != mi::kBlockSize) return 0;
  const int64_t parts = mi::parts_for(max_blocks);
  if (parts <= 1) return 0;
  return static_cast<int64_t>(batch) * parts * num_heads * (head_dim + 2) * static_cast<int64_t>(sizeof(float));
}

extern "C" int32_t mi_paged_decode_attention(void* out, int64_t out_row_stride, const void* query,
                                             int64_t query_row_stride, int64_t query_head_stride,
                                             const void* key_pool, const void* value_pool, int64_t num_blocks,
                                             const int64_t* block_tables, int64_t block_table_stride,
                                             int32_t max_blocks, const int64_t* context_lens,
                                             int64_t context_lens_stride, int32_t batch, int32_t num_heads,
                                             int32_t num_kv_heads, int32_t head_dim, int32_t block_size, float scale,
                                             void* workspace, int64_t workspace_bytes, void* stream) {
  using namespace mi;
  if (batch < 0 || max_blocks < 0 || num_blocks < 0)
    return fail(MI_ERR_INVALID_ARGUMENT, "mi_paged_decode_attention: negative size");
  if (batch == 0) return ok();
  if (!out || !query || !key_pool || !value_pool || !context_lens || (max_blocks > 0 && !block_tables))
    return fail(MI_ERR_INVALID_ARGUMENT, "mi_paged_decode_attention: null pointer argument");
  if (head_dim != kHeadDim || block_size != kBlockSize || num_kv_heads <= 0 || num_heads != kGroup * num_kv_heads)
    return fail(MI_ERR_UNSUPPORTED,
                "mi_paged_decode_attention: needs head_dim %d, block_size %d, num_heads = %d * num_kv_heads "
                "(got head_dim %d, block_size %d, heads %d/%d)",
                kHeadDim, kBlockSize, kGroup, head_dim, block_size, num_heads, num_kv_heads);
  if (num_kv_heads != 1 && num_kv_heads != 2 && num_kv_heads != 4 && num_kv_heads != 8)
    return fail(MI_ERR_UNSUPPORTED, "mi_paged_decode_attention: num_kv_heads %d not in {1,2,4,8}", num_kv_heads);
  if (!aligned16(out) || !aligned16(query) || !aligned16(key_pool) || !aligned16(value_pool) ||
      out_row_stride % 8 != 0 || query_row_stride % 8 != 0 || query_head_stride % 8 != 0)
    return fail(MI_ERR_UNSUPPORTED, "mi_paged_decode_attention: query/out/pools must be 16-byte aligned");
  if (max_blocks > 0 && block_table_stride < max_blocks)
    return fail(MI_ERR_INVALID_ARGUMENT, "mi_paged_decode_attention: block_table_stride < max_blocks");
  if (context_lens_stride <= 0)
    return fail(MI_ERR_INVALID_ARGUMENT, "mi_paged_decode_attention: context_lens_stride must be > 0");

  DecodeArgs a{};
  a.out = static_cast<uint16_t*>(out);
  a.out_row = out_row_stride;
  a.query = static_cast<const uint16_t*>(query);
  a.q_row = query_row_stride;
  a.q_head = query_head_stride;
  a.key_pool = static_cast<const uint16_t*>(key_pool);
  a.value_pool = static_cast<const uint16_t*>(value_pool);
  a.num_blocks = num_blocks;
  a.block_tables = block_tables;
  a.bt_stride = block_table_stride;
  a.context_lens = context_lens;
  a.ctx_stride = context_lens_stride;
  a.max_blocks = max_blocks;
  a.scale = scale;
  const int64_t parts = max_blocks > 0 ? parts_for(max_blocks) : 1;
  a.max_parts = static_cast<int32_t>(parts);
  if (parts > 1) {
    const int64_t need = mi_paged_decode_workspace_bytes(batch, max_blocks, num_heads, head_dim, block_size);
    if (!workspace || workspace_bytes < need)
      return fail(MI_ERR_WORKSPACE, "mi_paged_decode_attention: workspace of %lld bytes needed, got %lld",
                  static_cast<long long>(need), static_cast<long long>(workspace_bytes));
    if (!aligned16(workspace))
      return fail(MI_ERR_UNSUPPORTED, "mi_paged_decode_attention: workspace must be 16-byte aligned");
    a.ws_acc = static_cast<float*>(workspace);
    a.ws_ml = a.ws_acc + static_cast<int64_t>(batch) * parts * num_heads * kHeadDim;
  }
  if (parts * (num_kv_heads / (num_kv_heads < 4 ? num_kv_heads : 4)) > 0x7fffffff || batch > 65535)
    return fail(MI_ERR_UNSUPPORTED, "mi_paged_decode_attention: grid too large");

  hipStream_t s = as_stream(stream);
  switch (num_kv_heads) {
    case 1: return launch_decode<1>(a, batch, s);
    case 2: return launch_decode<2>(a, batch, s);
    case 4: return launch_decode<4>(a, batch, s);
    default: return launch_decode<8>(a, batch, s);
  }
}
