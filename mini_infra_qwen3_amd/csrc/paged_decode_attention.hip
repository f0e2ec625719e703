// Kernel 3: paged GQA decode attention (one query token per sequence).
//
// Behaviour of the reference's paged decode branch: the pool gather of
// Qwen3Attention._apply_paged_kv_pool (src/mini_infra/model/qwen3.py:285-292), the context-length
// bias of Qwen3Model._build_paged_inputs (:513-528) and Qwen3Attention._attend with
// _repeat_key_value (:219-255, :147-156) -- computed straight from the pool, without
// materialising the padded history or the repeated K/V.
//
// Work decomposition (MI355X: 256 CUs, 64-lane wavefronts, bandwidth-bound):
//  * A work unit is (sequence b, partition of kPartBlocks pool blocks of its context,
//    group of kWaves KV heads).  Wavefront w of the group serves KV head g and both query
//    heads 2g, 2g+1 that share it (GQA group 2), so every K/V byte is loaded exactly once.
//  * Persistent workgroups (a few per CU, MI_DECODE_PERSISTENT=1): each workgroup first turns
//    the context lengths into a prefix sum of partitions per sequence in LDS, then walks the
//    compact unit list with a grid stride -- no empty workgroups for short sequences.  With
//    MI_DECODE_PERSISTENT=0 the grid is (partitions x head groups, batch), one unit each.
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
//    writes bf16 output directly.  Otherwise the partition's (m, l, acc) go to the caller's
//    workspace and a second, small kernel merges the partitions.  (Merging inside the first
//    kernel needs device-scope release/acquire fences per partition, and on this GPU each
//    such fence writes back and invalidates a whole XCD L2: far more costly than a launch.)
#include "mi_common.h"

namespace mi {
namespace {

constexpr int kHeadDim = 128;
constexpr int kBlockSize = 16;
constexpr int kGroup = 2;          // query heads per KV head
#ifndef MI_DECODE_PART_BLOCKS
#define MI_DECODE_PART_BLOCKS 32
#endif
#ifndef MI_DECODE_DEPTH
#define MI_DECODE_DEPTH 2
#endif
#ifndef MI_DECODE_MAX_WAVES
#define MI_DECODE_MAX_WAVES 2
#endif
#ifndef MI_DECODE_NT_LOADS
#define MI_DECODE_NT_LOADS 1
#endif
#ifndef MI_DECODE_GROUPS_PER_CU
#define MI_DECODE_GROUPS_PER_CU 4
#endif
#ifndef MI_DECODE_PERSISTENT
#define MI_DECODE_PERSISTENT 1
#endif
constexpr int kPartBlocks = MI_DECODE_PART_BLOCKS;  // pool blocks per partition (512 tokens)
constexpr int kPartTokens = kPartBlocks * kBlockSize;
constexpr int kDepth = MI_DECODE_DEPTH;            // register ring depth (blocks in flight incl. current)
constexpr int kMaxWaves = MI_DECODE_MAX_WAVES;     // wavefronts (KV heads) per workgroup
constexpr bool kNtLoads = MI_DECODE_NT_LOADS != 0; // K/V stream with the non-temporal hint
constexpr int kGroupsPerCu = MI_DECODE_GROUPS_PER_CU;
constexpr bool kPersistent = MI_DECODE_PERSISTENT != 0;
constexpr int kMaxBatchPerLaunch = 4096;           // sequences whose prefix sum one workgroup holds in LDS
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kRescaleSlack = 8.0f;

static_assert(kPartBlocks <= 64, "one block id per lane");

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
  int32_t batch;                   // sequences of this launch
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

__device__ __forceinline__ float dot8(const uint4 q, const u32x4 k) {
  // Elements are copied to scalars before the bit casts: a bit cast of an ext-vector
  // component expression (k.y) must not be used, it can read component 0.
  const uint32_t k0 = k[0], k1 = k[1], k2 = k[2], k3 = k[3];
  float d = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, q.x), __builtin_bit_cast(bf16x2, k0), 0.0f, false);
  d = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, q.y), __builtin_bit_cast(bf16x2, k1), d, false);
  d = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, q.z), __builtin_bit_cast(bf16x2, k2), d, false);
  d = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, q.w), __builtin_bit_cast(bf16x2, k3), d, false);
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

__device__ __forceinline__ int64_t context_of(const DecodeArgs& a, int b) {
  const int64_t n = a.context_lens[b * a.ctx_stride];
  return min(n, static_cast<int64_t>(a.max_blocks) * kBlockSize);
}

// Partitions of a context of n tokens; an empty context still owns one unit (zero output).
__device__ __forceinline__ int parts_of(int64_t n) {
  return n <= 0 ? 1 : static_cast<int>((n + kPartTokens - 1) / kPartTokens);
}

__device__ __forceinline__ void store_bf16x8(uint16_t* dst, const float* o, float inv) {
  uint4 v;
  v.x = pack_bf16x2(o[0] * inv, o[1] * inv);
  v.y = pack_bf16x2(o[2] * inv, o[3] * inv);
  v.z = pack_bf16x2(o[4] * inv, o[5] * inv);
  v.w = pack_bf16x2(o[6] * inv, o[7] * inv);
  *reinterpret_cast<uint4*>(dst) = v;
}

// Exclusive prefix sums of the partitions per sequence into s_off[0..batch]; returns the total.
template <int kThreads>
__device__ int scan_partitions(const DecodeArgs& a, int* s_off, int* s_wave) {
  constexpr int kWavesPerGroup = kThreads / 64;
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  int carry = 0;
  for (int base = 0; base < a.batch; base += kThreads) {
    const int i = base + threadIdx.x;
    int v = i < a.batch ? parts_of(context_of(a, i)) : 0;
    for (int d = 1; d < 64; d <<= 1) {
      const int y = __shfl_up(v, d);
      if (lane >= d) v += y;
    }
    if (lane == 63) s_wave[w] = v;
    __syncthreads();
    int prefix = 0, total = 0;
#pragma unroll
    for (int k = 0; k < kWavesPerGroup; ++k) {
      const int t = s_wave[k];
      prefix += k < w ? t : 0;
      total += t;
    }
    if (i < a.batch) s_off[i + 1] = carry + prefix + v;
    carry += total;
    __syncthreads();
  }
  if (threadIdx.x == 0) s_off[0] = 0;
  __syncthreads();
  return carry;
}

template <int kKvHeads, int kWaves>
// Second bound: minimum wavefronts per SIMD, so that kGroupsPerCu workgroups fit on a CU
// (4 SIMDs per CU) and the persistent grid is fully resident.
__global__ __launch_bounds__(64 * kWaves, (kGroupsPerCu * kWaves + 3) / 4) void paged_decode_kernel(const DecodeArgs a) {
  constexpr int kThreads = 64 * kWaves;
  constexpr int kRowElems = kKvHeads * kHeadDim;     // elements of one pool row (token)
  constexpr int kBlockElems = kBlockSize * kRowElems;
  constexpr int kHeadGroups = kKvHeads / kWaves;
  constexpr int kHeads = kKvHeads * kGroup;

  extern __shared__ int s_off[];                     // [batch + 1] partition prefix sums
  __shared__ int s_wave[kWaves];

  int total_units, first_unit, unit_stride;
  if constexpr (kPersistent) {
    total_units = scan_partitions<kThreads>(a, s_off, s_wave) * kHeadGroups;
    first_unit = blockIdx.x;
    unit_stride = gridDim.x;
  } else {
    total_units = 1;
    first_unit = 0;
    unit_stride = 1;
  }

  const int lane = threadIdx.x & 63;
  const int dl = lane & 15;
  const int r = lane >> 4;
  const float scale = a.scale;

  for (int unit = first_unit; unit < total_units; unit += unit_stride) {
    int b, part, hg;
    if constexpr (kPersistent) {
      hg = unit % kHeadGroups;
      const int pu = unit / kHeadGroups;
      int lo = 0, hi = a.batch;  // s_off[lo] <= pu < s_off[hi]
      while (hi - lo > 1) {
        const int mid = (lo + hi) >> 1;
        if (s_off[mid] <= pu) lo = mid; else hi = mid;
      }
      b = lo;
      part = pu - s_off[b];
    } else {
      b = blockIdx.y;
      part = blockIdx.x / kHeadGroups;
      hg = blockIdx.x - part * kHeadGroups;
    }
    const int g = hg * kWaves + (threadIdx.x >> 6);
    const int64_t n = context_of(a, b);
    const int nparts = parts_of(n);
    if (part >= nparts) continue;  // grid form: partition past this sequence's context

    if (n <= 0) {  // empty context: zero output row for this group's heads
      if (r < kGroup) {
        uint16_t* o = a.out + b * a.out_row + (g * kGroup + r) * kHeadDim + 8 * dl;
        *reinterpret_cast<uint4*>(o) = uint4{0, 0, 0, 0};
      }
      continue;
    }
    const int64_t t_begin = static_cast<int64_t>(part) * kPartTokens;
    const int n32 = static_cast<int>(n);  // contexts are bounded by max_blocks * 16 < 2^31
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
      const uint32_t blo = __builtin_amdgcn_readlane(bid_lo, j);
      const uint32_t bhi = __builtin_amdgcn_readlane(bid_hi, j);
      return static_cast<int64_t>((static_cast<uint64_t>(bhi) << 32) | blo) * kBlockElems;
    };

    u32x4 kbuf[kDepth][4], vbuf[kDepth][4];
    auto issue = [&](int slot, int j) {
      const int64_t base = block_base(min(j, nblk - 1));
      const uint16_t* kp = a.key_pool + base + lane_off;
      const uint16_t* vp = a.value_pool + base + lane_off;
#pragma unroll
      for (int i = 0; i < 4; ++i) kbuf[slot][i] = load_vec<kNtLoads>(reinterpret_cast<const u32x4*>(kp + i * 4 * kRowElems));
#pragma unroll
      for (int i = 0; i < 4; ++i) vbuf[slot][i] = load_vec<kNtLoads>(reinterpret_cast<const u32x4*>(vp + i * 4 * kRowElems));
    };

    float m0 = -INFINITY, m1 = -INFINITY, l0 = 0.0f, l1 = 0.0f;
    float acc0[8], acc1[8];
#pragma unroll
    for (int d = 0; d < 8; ++d) acc0[d] = acc1[d] = 0.0f;

#pragma unroll
    for (int s = 0; s < kDepth - 1; ++s) issue(s, s);

    for (int j0 = 0; j0 < nblk; j0 += kDepth) {
#pragma unroll
      for (int s = 0; s < kDepth; ++s) {
        const int j = j0 + s;
        if (j >= nblk) break;
        issue((s + kDepth - 1) % kDepth, j + kDepth - 1);

        // ---- scores of tokens 4 i + r of block j, both query heads.  Only a partition's
        // last block can reach past the context; full blocks skip the masking (uniform branch).
        float s0[4], s1[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          s0[i] = score_log2(dpp_sum16(dot8(q0, kbuf[s][i])), scale);
          s1[i] = score_log2(dpp_sum16(dot8(q1, kbuf[s][i])), scale);
        }
        const int tok_base = static_cast<int>(t_begin) + j * kBlockSize;
        if (tok_base + kBlockSize > n32) {
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const bool valid = tok_base + 4 * i + r < n32;
            s0[i] = valid ? s0[i] : -INFINITY;
            s1[i] = valid ? s1[i] : -INFINITY;
          }
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
        // exp2(-inf) = 0 covers masked tokens; a row with no valid token yet keeps m = -inf,
        // so the reference point falls back to 0 there to avoid -inf - -inf.
        const float r0 = m0 == -INFINITY ? 0.0f : m0;
        const float r1 = m1 == -INFINITY ? 0.0f : m1;
        float p0[4], p1[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          p0[i] = __builtin_amdgcn_exp2f(s0[i] - r0);
          p1[i] = __builtin_amdgcn_exp2f(s1[i] - r1);
        }
        l0 += (p0[0] + p0[1]) + (p0[2] + p0[3]);
        l1 += (p1[0] + p1[1]) + (p1[2] + p1[3]);

        // ---- P V over token pairs (0,1) and (2,3)
#pragma unroll
        for (int pr = 0; pr < 2; ++pr) {
          const uint32_t ph0 = pack_p(p0[2 * pr], p0[2 * pr + 1]);
          const uint32_t ph1 = pack_p(p1[2 * pr], p1[2 * pr + 1]);
          const u32x4 va = vbuf[s][2 * pr];
          const u32x4 vc = vbuf[s][2 * pr + 1];
          const uint32_t aw[4] = {va[0], va[1], va[2], va[3]};
          const uint32_t cw[4] = {vc[0], vc[1], vc[2], vc[3]};
#pragma unroll
          for (int w = 0; w < 4; ++w) {
            const uint32_t plo = __builtin_amdgcn_perm(cw[w], aw[w], 0x05040100u);  // (a.lo, c.lo)
            const uint32_t phi = __builtin_amdgcn_perm(cw[w], aw[w], 0x07060302u);  // (a.hi, c.hi)
            acc0[2 * w] = fdot2(ph0, plo, acc0[2 * w]);
            acc0[2 * w + 1] = fdot2(ph0, phi, acc0[2 * w + 1]);
            acc1[2 * w] = fdot2(ph1, plo, acc1[2 * w]);
            acc1[2 * w + 1] = fdot2(ph1, phi, acc1[2 * w + 1]);
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

    // Row 0 writes query head 2g, row 1 query head 2g + 1 (every row has both after the merge).
    const int h = g * kGroup + (r & 1);
    float o[8];
#pragma unroll
    for (int d = 0; d < 8; ++d) o[d] = (r & 1) == 0 ? acc0[d] : acc1[d];
    if (nparts == 1) {
      if (r < kGroup) store_bf16x8(a.out + b * a.out_row + h * kHeadDim + 8 * dl, o, 1.0f / ((r & 1) == 0 ? l0 : l1));
      continue;
    }
    if (r < kGroup) {
      const int64_t slot = (static_cast<int64_t>(b) * a.max_parts + part) * kHeads + h;
      float4* dst = reinterpret_cast<float4*>(a.ws_acc + slot * kHeadDim + 8 * dl);
      dst[0] = make_float4(o[0], o[1], o[2], o[3]);
      dst[1] = make_float4(o[4], o[5], o[6], o[7]);
      if (dl == 0) {
        a.ws_ml[slot * 2 + 0] = (r & 1) == 0 ? M0 : M1;
        a.ws_ml[slot * 2 + 1] = (r & 1) == 0 ? l0 : l1;
      }
    }
  }
}

// Merge the partitions of sequences longer than one partition.
// grid: batch; block: heads * 16 lanes, lane (h, dm) owns dims [8 dm, 8 dm + 8) of head h.
// Partials of one sequence are contiguous; kMergeUnroll partitions are loaded per step.
template <int kHeads>
__global__ __launch_bounds__(kHeads * 16) void paged_decode_merge_kernel(const DecodeArgs a) {
  constexpr int kMergeUnroll = 8;
  const int b = blockIdx.x;
  const int h = threadIdx.x >> 4;
  const int dm = threadIdx.x & 15;
  const int nparts = parts_of(context_of(a, b));
  if (context_of(a, b) <= 0 || nparts <= 1) return;
  const int64_t base = static_cast<int64_t>(b) * a.max_parts * kHeads + h;
  float M = -INFINITY;
  for (int p0 = 0; p0 < nparts; p0 += kMergeUnroll) {
    float m[kMergeUnroll];
#pragma unroll
    for (int k = 0; k < kMergeUnroll; ++k)
      m[k] = p0 + k < nparts ? a.ws_ml[(base + (p0 + k) * kHeads) * 2] : -INFINITY;
#pragma unroll
    for (int k = 0; k < kMergeUnroll; ++k) M = fmaxf(M, m[k]);
  }
  float L = 0.0f, acc[8];
#pragma unroll
  for (int d = 0; d < 8; ++d) acc[d] = 0.0f;
  for (int p0 = 0; p0 < nparts; p0 += kMergeUnroll) {
    float4 x[kMergeUnroll], y[kMergeUnroll];
    float m[kMergeUnroll], l[kMergeUnroll];
#pragma unroll
    for (int k = 0; k < kMergeUnroll; ++k) {
      if (p0 + k < nparts) {
        const int64_t slot = base + (p0 + k) * kHeads;
        m[k] = a.ws_ml[slot * 2];
        l[k] = a.ws_ml[slot * 2 + 1];
        const float4* src = reinterpret_cast<const float4*>(a.ws_acc + slot * kHeadDim + 8 * dm);
        x[k] = src[0];
        y[k] = src[1];
      } else {
        m[k] = -INFINITY;
        l[k] = 0.0f;
        x[k] = y[k] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
      }
    }
#pragma unroll
    for (int k = 0; k < kMergeUnroll; ++k) {
      const float w = m[k] == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(m[k] - M);
      L += w * l[k];
      acc[0] += w * x[k].x; acc[1] += w * x[k].y; acc[2] += w * x[k].z; acc[3] += w * x[k].w;
      acc[4] += w * y[k].x; acc[5] += w * y[k].y; acc[6] += w * y[k].z; acc[7] += w * y[k].w;
    }
  }
  store_bf16x8(a.out + b * a.out_row + h * kHeadDim + 8 * dm, acc, 1.0f / L);
}

int device_cus() {
  static int cached[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (cached[dev] == 0) {
    int cus = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0) cus = 256;
    cached[dev] = cus;
  }
  return cached[dev];
}

template <int kKvHeads>
int32_t launch_decode(const DecodeArgs& a, hipStream_t s) {
  constexpr int kWaves = kKvHeads < kMaxWaves ? kKvHeads : kMaxWaves;
  constexpr int kHeadGroups = kKvHeads / kWaves;
  if constexpr (kPersistent) {
    const int64_t units_bound = static_cast<int64_t>(a.batch) * a.max_parts * kHeadGroups;
    const int64_t resident = static_cast<int64_t>(device_cus()) * kGroupsPerCu;
    const uint32_t grid = static_cast<uint32_t>(units_bound < resident ? units_bound : resident);
    const size_t lds = sizeof(int) * (static_cast<size_t>(a.batch) + 1);
    paged_decode_kernel<kKvHeads, kWaves><<<grid, 64 * kWaves, lds, s>>>(a);
  } else {
    dim3 grid(static_cast<uint32_t>(a.max_parts * kHeadGroups), static_cast<uint32_t>(a.batch));
    paged_decode_kernel<kKvHeads, kWaves><<<grid, 64 * kWaves, 0, s>>>(a);
  }
  int32_t rc = check_launch("mi_paged_decode_attention");
  if (rc != MI_OK || a.max_parts <= 1) return rc;
  paged_decode_merge_kernel<kKvHeads * kGroup><<<a.batch, kKvHeads * kGroup * 16, 0, s>>>(a);
  return check_launch("mi_paged_decode_attention(merge)");
}

int64_t parts_for(int32_t max_blocks) { return (static_cast<int64_t>(max_blocks) + kPartBlocks - 1) / kPartBlocks; }

int head_groups_for(int32_t num_kv_heads) {
  const int waves = num_kv_heads < kMaxWaves ? num_kv_heads : kMaxWaves;
  return num_kv_heads / waves;
}

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

  const int64_t parts = max_blocks > 0 ? parts_for(max_blocks) : 1;
  float* ws_acc = nullptr;
  float* ws_ml = nullptr;
  if (parts > 1) {
    const int64_t need = mi_paged_decode_workspace_bytes(batch, max_blocks, num_heads, head_dim, block_size);
    if (!workspace || workspace_bytes < need)
      return fail(MI_ERR_WORKSPACE, "mi_paged_decode_attention: workspace of %lld bytes needed, got %lld",
                  static_cast<long long>(need), static_cast<long long>(workspace_bytes));
    if (!aligned16(workspace))
      return fail(MI_ERR_UNSUPPORTED, "mi_paged_decode_attention: workspace must be 16-byte aligned");
    ws_acc = static_cast<float*>(workspace);
    ws_ml = ws_acc + static_cast<int64_t>(batch) * parts * num_heads * kHeadDim;
  }
  if (static_cast<int64_t>(batch) * parts * head_groups_for(num_kv_heads) > 0x7fffffff ||
      (!kPersistent && batch > 65535))
    return fail(MI_ERR_UNSUPPORTED, "mi_paged_decode_attention: too many work units");

  hipStream_t s = as_stream(stream);
  // Sequences go in slices of at most kMaxBatchPerLaunch (the per-workgroup prefix sum lives in LDS).
  for (int32_t b0 = 0; b0 < batch; b0 += kMaxBatchPerLaunch) {
    const int32_t nb = batch - b0 < kMaxBatchPerLaunch ? batch - b0 : kMaxBatchPerLaunch;
    DecodeArgs a{};
    a.out = static_cast<uint16_t*>(out) + b0 * out_row_stride;
    a.out_row = out_row_stride;
    a.query = static_cast<const uint16_t*>(query) + b0 * query_row_stride;
    a.q_row = query_row_stride;
    a.q_head = query_head_stride;
    a.key_pool = static_cast<const uint16_t*>(key_pool);
    a.value_pool = static_cast<const uint16_t*>(value_pool);
    a.num_blocks = num_blocks;
    a.block_tables = block_tables ? block_tables + b0 * block_table_stride : nullptr;
    a.bt_stride = block_table_stride;
    a.context_lens = context_lens + b0 * context_lens_stride;
    a.ctx_stride = context_lens_stride;
    a.batch = nb;
    a.max_blocks = max_blocks;
    a.max_parts = static_cast<int32_t>(parts);
    a.scale = scale;
    if (parts > 1) {
      a.ws_acc = ws_acc + static_cast<int64_t>(b0) * parts * num_heads * kHeadDim;
      a.ws_ml = ws_ml + static_cast<int64_t>(b0) * parts * num_heads * 2;
    }
    int32_t rc;
    switch (num_kv_heads) {
      case 1: rc = launch_decode<1>(a, s); break;
      case 2: rc = launch_decode<2>(a, s); break;
      case 4: rc = launch_decode<4>(a, s); break;
      default: rc = launch_decode<8>(a, s); break;
    }
    if (rc != MI_OK) return rc;
  }
  return ok();
}
