// Kernel 3: paged GQA decode attention (one query token per sequence).
//
// Behaviour of the reference's paged decode branch: the pool gather of
// Qwen3Attention._apply_paged_kv_pool (src/mini_infra/model/qwen3.py:285-292), the context-length
// bias of Qwen3Model._build_paged_inputs (:513-528) and Qwen3Attention._attend with
// _repeat_key_value (:219-255, :147-156) -- computed straight from the pool, without
// materialising the padded history or the repeated K/V.
//
// Work decomposition (MI355X: 256 CUs in 8 XCDs, 64-lane wavefronts, bandwidth-bound):
//  * The work of one launch is the list of (sequence, pool block) pairs, sequences in order,
//    N blocks in all.  It is cut into `streams` contiguous ranges of N / streams blocks (+-1),
//    and workgroup (stream s, head group hg) streams range s for the kWaves KV heads of hg.
//    Every workgroup gets the same number of blocks whatever the context lengths, and the
//    head groups of one range run side by side (adjacent workgroup ids), so the 2 KiB pool
//    rows of a block are read by concurrent workgroups.  Wavefront w of a group serves KV
//    head g and all G query heads G g .. G g + G - 1 that share it (the GQA group; 2 for
//    Qwen3-0.6B, kernels compiled for G in {1, 2, 4, 5, 8}): every K/V byte is loaded exactly
//    once.
//  * Each workgroup first turns the context lengths into a prefix sum of blocks per sequence
//    in LDS (so a block index maps to its sequence by binary search); block ids of the next
//    64 blocks of the range are fetched one per lane, a window ahead, and broadcast with
//    readlane.
//  * Inside a wavefront, lane = 16 * row + dl.  Lane dl holds dims [8 dl, 8 dl + 8) of the
//    G queries; row r owns tokens 4 i + r (i = 0..3) of every 16-token block.  One
//    16-byte load per lane per i brings four 256-byte (token, head) rows per instruction.
//  * QK^T: bf16 v_dot2 on packed pairs, then a 16-lane DPP butterfly (quad_perm, half-row
//    mirror, row mirror) leaves the full dot product in every lane of the row.
//  * Each row keeps its own online-softmax state (running max m, sum l, fp32 accumulator
//    of G heads x 8 dims), so no cross-row traffic happens inside the block loop.  The max
//    is rescaled lazily: only when a new score exceeds the running max by more than
//    kRescaleSlack (log2 units) -- exact, since l and the accumulator share the same m.
//  * PV: probabilities of token pairs are packed to bf16 and v_perm regroups V so that one
//    v_dot2 covers two tokens of one dim.
//  * K/V of the next kDepth-1 blocks are in flight in registers while the current block
//    is computed (a register ring: the VGPR file is 512 KiB per CU, LDS is 160 KiB).  The
//    ring runs straight across sequence boundaries, so the memory pipeline never drains
//    inside a range.
//  * At the end of a sequence's segment the four rows merge (log-sum-exp).  A sequence whose
//    blocks all lie in one range writes its bf16 output directly.  A sequence cut by a range
//    boundary leaves (m, l, acc) partials: a range holds at most two cut sequences (its first
//    and its last), so the caller's workspace is 2 slots per range per head, whatever the
//    batch and context lengths.  A second, small kernel merges the cut sequences and writes
//    zero rows for empty contexts.  (Merging inside the first kernel needs device-scope
//    release/acquire fences, and on this GPU each such fence writes back and invalidates a
//    whole XCD L2: far more costly than a launch.)
#include <cstdlib>
#include <cstring>
#include <mutex>

#include "mi_common.h"

namespace mi {
namespace {

constexpr int kHeadDim = 128;
constexpr int kBlockSize = 16;
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
constexpr int kDepth = MI_DECODE_DEPTH;            // register ring depth (blocks in flight incl. current)
constexpr int kMaxWaves = MI_DECODE_MAX_WAVES;     // wavefronts (KV heads) per workgroup
constexpr bool kNtLoads = MI_DECODE_NT_LOADS != 0; // K/V stream with the non-temporal hint
constexpr int kGroupsPerCu = MI_DECODE_GROUPS_PER_CU;
#ifndef MI_DECODE_XCD_RUN
#define MI_DECODE_XCD_RUN 0
#endif
// Consecutive stream-kernel workgroups per XCD run (0: launch order, which deals a range's head
// groups to different XCDs).  Unlike the scatter and the gather, decode loses with runs: at batch
// 256 (Σctx 755,887, 28 layers, three repetitions) 461-462 µs per layer without, 476.6-478.0 with
// runs of 4, 8, 16 or 32; four KV heads per workgroup (MI_DECODE_MAX_WAVES=4) 523-526 µs.
constexpr int kXcdRun = MI_DECODE_XCD_RUN;
constexpr int kMaxBatchPerLaunch = 4096;           // sequences whose prefix sum one workgroup holds in LDS
constexpr int kMinBlocksPerStream = 16;            // small launches use fewer, longer ranges
constexpr int kWindow = 64;                        // block ids fetched per window, one per lane
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kRescaleSlack = 8.0f;

static_assert(kDepth >= 2 && kDepth - 1 < kWindow, "the ring looks ahead less than one id window");

typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

#ifndef MI_DECODE_MFMA_GROUP
#define MI_DECODE_MFMA_GROUP 4
#endif
// GQA groups from this size up use the matrix-core form of the stream kernel (at most 16 heads,
// the MFMA's column count); smaller groups (Qwen3-0.6B / 1.7B's 2, multi-head 1) use the
// dot-product form, whose v_dot2 + DPP row reduction needs no zero-padded columns.  Measured at batch 256
// (8 KV heads, Σctx 755,887, attention + merge), TB/s for groups 1 / 2 / 4 / 5 / 8:
// dot-product form 6.75 / 6.67 / 6.40 / 6.27 / 4.67 (its per-token arithmetic grows with the
// group); matrix-core form 6.75 / 6.71 / 6.56 / 6.51 / 6.35.  At group 2, interleaved in one
// process (8 x 20 launches each), the matrix-core form took 461.5 µs (median) against 463.3.
constexpr int kMfmaGroup = MI_DECODE_MFMA_GROUP;
#ifndef MI_DECODE_SEQ_MFMA_GROUP
#define MI_DECODE_SEQ_MFMA_GROUP 2
#endif
// The per-sequence kernel (small launches: latency-bound) takes the matrix-core form from this
// group size up.  At group 2 the matrix-core form measured faster (6.4 against 7.8 µs per layer at
// batch 1, 9.5 against 11.6 at 6, 22.0 against 22.8 at 32; contexts U[32, 1150]); in the
// bandwidth-kernel e2e runs of config 5 (two repetitions each, one machine) the decode step went
// from 2.144-2.145 to 2.104-2.121 ms alternating and from 2.127-2.136 to 2.114-2.118 ms mixed.
constexpr int kSeqMfmaGroup = MI_DECODE_SEQ_MFMA_GROUP;

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
  int32_t streams;                 // block ranges; grid = streams x head groups
  float scale;                     // softmax scale (natural units)
  float* ws_acc;                   // [streams, 2, heads, 128]: slot 0 = range's first (cut) sequence, 1 = last
  float* ws_ml;                    // [streams, 2, heads, 2] = (m, l) in log2 units
  // Fused form of the per-sequence kernel: raw q / k / v projection rows of the new tokens, the
  // q/k norm weights, cos / sin rows [batch, 128] and the slots of the new K/V rows.
  const uint16_t* q_raw;
  const uint16_t* k_raw;
  const uint16_t* v_raw;
  int64_t q_raw_row, k_raw_row, v_raw_row;  // elements
  const uint16_t* q_weight;
  const uint16_t* k_weight;
  const uint16_t* cos;
  const uint16_t* sin;
  const int64_t* slot_mapping;
  int64_t slot_stride;
  int64_t num_slots;
  float eps;
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

// Pool blocks of a context of n tokens (0 for an empty context).
__device__ __forceinline__ int blocks_of(int64_t n) {
  return n <= 0 ? 0 : static_cast<int>((n + kBlockSize - 1) / kBlockSize);
}

// Range holding block x of N: the last s with floor(s N / streams) <= x.
__device__ __forceinline__ int stream_of(int64_t x, int64_t total, int streams) {
  return static_cast<int>(((x + 1) * streams - 1) / total);
}

__device__ __forceinline__ void store_bf16x8(uint16_t* dst, const float* o, float inv) {
  uint4 v;
  v.x = pack_bf16x2(o[0] * inv, o[1] * inv);
  v.y = pack_bf16x2(o[2] * inv, o[3] * inv);
  v.z = pack_bf16x2(o[4] * inv, o[5] * inv);
  v.w = pack_bf16x2(o[6] * inv, o[7] * inv);
  *reinterpret_cast<uint4*>(dst) = v;
}

// Exclusive prefix sums of the blocks per sequence into s_off[0..batch]; returns the total.
template <int kThreads>
__device__ int scan_blocks(const DecodeArgs& a, int* s_off, int* s_wave) {
  constexpr int kWavesPerGroup = kThreads / 64;
  static_assert(kThreads % 64 == 0, "whole wavefronts");
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  int carry = 0;
  for (int base = 0; base < a.batch; base += kThreads) {
    const int i = base + threadIdx.x;
    int v = i < a.batch ? blocks_of(context_of(a, i)) : 0;
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

// Sequence of block x (x < total): the last b with s_off[b] <= x (empty sequences are skipped).
__device__ __forceinline__ int row_of(const int* s_off, int batch, int64_t x) {
  int lo = 0, hi = batch;  // s_off[lo] <= x < s_off[hi]
  while (hi - lo > 1) {
    const int mid = (lo + hi) >> 1;
    if (s_off[mid] <= x) lo = mid; else hi = mid;
  }
  return lo;
}

// Softmax state of one lane row (tokens 4 i + r of every block) for the kG query heads of its KV
// head: running max m (log2 units), sum l and the fp32 accumulator of the lane's 8 dims.
template <int kG>
struct RowState {
  float m[kG], l[kG], acc[kG][8];
  __device__ __forceinline__ void init() {
#pragma unroll
    for (int h = 0; h < kG; ++h) {
      m[h] = -INFINITY;
      l[h] = 0.0f;
#pragma unroll
      for (int d = 0; d < 8; ++d) acc[h][d] = 0.0f;
    }
  }
};

// One 16-token block (first token tok_base of a context of n tokens) for lane row r: scores of
// tokens 4 i + r against the kG queries, lazy rescale, then P V.  Only a sequence's last block
// can reach past its context; full blocks skip the masking (uniform branch).
template <int kG>
__device__ __forceinline__ void attend_block(RowState<kG>& st, const uint4 (&q)[kG], const u32x4 (&kb)[4],
                                             const u32x4 (&vb)[4], float scale, int tok_base, int n, int r) {
  float s[kG][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int h = 0; h < kG; ++h) s[h][i] = score_log2(dpp_sum16(dot8(q[h], kb[i])), scale);
  if (tok_base + kBlockSize > n) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const bool valid = tok_base + 4 * i + r < n;
#pragma unroll
      for (int h = 0; h < kG; ++h) s[h][i] = valid ? s[h][i] : -INFINITY;
    }
  }
  float mb[kG];
  bool grow = false;
#pragma unroll
  for (int h = 0; h < kG; ++h) {
    mb[h] = fmaxf(fmaxf(s[h][0], s[h][1]), fmaxf(s[h][2], s[h][3]));
    grow = grow || mb[h] > st.m[h] + kRescaleSlack;
  }
  if (__builtin_amdgcn_ballot_w64(grow) != 0) {  // lazy rescale (wave-uniform branch)
#pragma unroll
    for (int h = 0; h < kG; ++h) {
      const float nm = fmaxf(st.m[h], mb[h]);
      const float al = (nm == -INFINITY) ? 1.0f : __builtin_amdgcn_exp2f(st.m[h] - nm);
      st.m[h] = nm;
      st.l[h] *= al;
#pragma unroll
      for (int d = 0; d < 8; ++d) st.acc[h][d] *= al;
    }
  }
  // exp2(-inf) = 0 covers masked tokens; a row with no valid token yet keeps m = -inf, so the
  // reference point falls back to 0 there to avoid -inf - -inf.
  uint32_t ph[kG][2];
#pragma unroll
  for (int h = 0; h < kG; ++h) {
    const float ref = st.m[h] == -INFINITY ? 0.0f : st.m[h];
    float p[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) p[i] = __builtin_amdgcn_exp2f(s[h][i] - ref);
    st.l[h] += (p[0] + p[1]) + (p[2] + p[3]);
    ph[h][0] = pack_p(p[0], p[1]);
    ph[h][1] = pack_p(p[2], p[3]);
  }
  // P V over token pairs (0,1) and (2,3): v_perm regroups V so that one v_dot2 covers two tokens
  // of one dim; the regrouped V serves every head of the group.
#pragma unroll
  for (int pr = 0; pr < 2; ++pr) {
    const u32x4 va = vb[2 * pr];
    const u32x4 vc = vb[2 * pr + 1];
    const uint32_t aw[4] = {va[0], va[1], va[2], va[3]};
    const uint32_t cw[4] = {vc[0], vc[1], vc[2], vc[3]};
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      const uint32_t plo = __builtin_amdgcn_perm(cw[w], aw[w], 0x05040100u);  // (a.lo, c.lo)
      const uint32_t phi = __builtin_amdgcn_perm(cw[w], aw[w], 0x07060302u);  // (a.hi, c.hi)
#pragma unroll
      for (int h = 0; h < kG; ++h) {
        st.acc[h][2 * w] = fdot2(ph[h][pr], plo, st.acc[h][2 * w]);
        st.acc[h][2 * w + 1] = fdot2(ph[h][pr], phi, st.acc[h][2 * w + 1]);
      }
    }
  }
}

// Merges the four lane rows of a wavefront (log-sum-exp): afterwards every row holds, per head,
// the wavefront's max M, sum l and accumulator.
template <int kG>
__device__ __forceinline__ void merge_rows(RowState<kG>& st, float (&M)[kG]) {
#pragma unroll
  for (int h = 0; h < kG; ++h) {
    float mx = fmaxf(st.m[h], __shfl_xor(st.m[h], 16));
    mx = fmaxf(mx, __shfl_xor(mx, 32));
    M[h] = mx;
    const float wt = (st.m[h] == -INFINITY) ? 0.0f : __builtin_amdgcn_exp2f(st.m[h] - mx);
    st.l[h] *= wt;
    st.l[h] += __shfl_xor(st.l[h], 16);
    st.l[h] += __shfl_xor(st.l[h], 32);
#pragma unroll
    for (int d = 0; d < 8; ++d) {
      st.acc[h][d] *= wt;
      st.acc[h][d] += __shfl_xor(st.acc[h][d], 16);
      st.acc[h][d] += __shfl_xor(st.acc[h][d], 32);
    }
  }
}

// ---- Matrix-core form (groups of kMfmaGroup..16 query heads).  Per 16-token block and wavefront:
//  * S^T = K Q^T with four v_mfma_f32_16x16x32_bf16 over the 128 dims: A = K (lane: token
//    lane % 16, dims 32 ks + 8 (lane / 16) .. +8), B = Q^T (lane: head lane % 16, zero past the
//    group), C: lane holds head lane % 16, tokens 4 (lane / 16) + i.  K is loaded in whole
//    256-byte token rows, as the dot-product form loads it, and restaged into the A layout
//    through 16 LDS rows per wavefront (A straight from the pool would read 64-byte pieces of 16
//    rows per instruction).
//  * That C layout is the A layout of v_mfma_f32_16x16x16_bf16 (row lane % 16, k = 4 (lane / 16)
//    + i), so the probabilities feed O = P V without moving.  V is loaded as token 4 (lane / 16) + i,
//    dims 8 (lane % 16) .. +8; output tile t takes dim 8 j + t as its column j, so B of tile t is
//    element t of the lane's four V pieces (two v_perm) and the lane ends up holding, for heads
//    4 (lane / 16) + i, dims 8 (lane % 16) .. +8: one 16-byte store per head.
//  * Softmax per head column: the running max m is shared by the column's four lanes (raised
//    lazily, with the column max, as in the dot-product form); each lane sums its own tokens.
struct MfmaState {
  float m;       // running max of head lane % 16 (log2 units), equal in the four lanes of its column
  float l;       // this lane's share of the head's sum
  f32x4 o[8];    // tile t: O[head 4 (lane / 16) + i][dim 8 (lane % 16) + t]
};

constexpr int kKStageRow = kHeadDim + 8;  // LDS row (elements) of a wavefront's K staging: 272 bytes

// kb: the lane's K pieces as the dot-product form loads them (token 4 i + lane / 16, dims
// 8 (lane % 16) .. +8: whole 256-byte rows per instruction); kst: the wavefront's 16-row K staging
// in LDS, through which they reach the MFMA A layout (token lane % 16, dims 32 ks + 8 (lane / 16)).
__device__ __forceinline__ void attend_block_mfma(MfmaState& st, const bf16x8 (&qf)[4], const u32x4 (&kb)[4],
                                                  const u32x4 (&vb)[4], uint16_t* kst, float scale,
                                                  int tok_base, int n, int lane) {
  const int dl = lane & 15, r = lane >> 4;
#pragma unroll
  for (int i = 0; i < 4; ++i) *reinterpret_cast<u32x4*>(kst + (4 * i + r) * kKStageRow + 8 * dl) = kb[i];
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
  for (int ks = 0; ks < 4; ++ks)
    acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(*reinterpret_cast<const bf16x8*>(kst + dl * kKStageRow + 32 * ks + 8 * r),
                                                  qf[ks], acc, 0, 0, 0);
  // The next block's staging stores follow these reads in the wavefront's LDS order.
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  const int tok0 = tok_base + 4 * (lane >> 4);
  float sc[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) sc[i] = score_log2(acc[i], scale);
  if (tok_base + kBlockSize > n) {  // the sequence's last block (uniform branch)
#pragma unroll
    for (int i = 0; i < 4; ++i) sc[i] = tok0 + i < n ? sc[i] : -INFINITY;
  }
  const float mb = fmaxf(fmaxf(sc[0], sc[1]), fmaxf(sc[2], sc[3]));
  if (__builtin_amdgcn_ballot_w64(mb > st.m + kRescaleSlack) != 0) {  // lazy rescale (wave-uniform)
    float cm = fmaxf(mb, __shfl_xor(mb, 16));
    cm = fmaxf(cm, __shfl_xor(cm, 32));
    const float nm = fmaxf(st.m, cm);
    const float al = (nm == -INFINITY) ? 1.0f : __builtin_amdgcn_exp2f(st.m - nm);
    st.m = nm;
    st.l *= al;
#pragma unroll
    for (int i = 0; i < 4; ++i) {  // O rows are heads 4 (lane / 16) + i: lane h holds head h's factor
      const float ai = __shfl(al, 4 * (lane >> 4) + i);
#pragma unroll
      for (int t = 0; t < 8; ++t) st.o[t][i] *= ai;
    }
  }
  const float ref = st.m == -INFINITY ? 0.0f : st.m;
  float p[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) p[i] = __builtin_amdgcn_exp2f(sc[i] - ref);
  st.l += (p[0] + p[1]) + (p[2] + p[3]);
  const bf16x4 pa = __builtin_convertvector((f32x4){p[0], p[1], p[2], p[3]}, bf16x4);
#pragma unroll
  for (int t = 0; t < 8; ++t) {
    const uint32_t sel = (t & 1) ? 0x07060302u : 0x05040100u;
    const uint32_t w01 = __builtin_amdgcn_perm(vb[1][t >> 1], vb[0][t >> 1], sel);  // tokens 0, 1 at dim t
    const uint32_t w23 = __builtin_amdgcn_perm(vb[3][t >> 1], vb[2][t >> 1], sel);  // tokens 2, 3
    const bf16x4 vbf = __builtin_bit_cast(bf16x4, (u32x2){w01, w23});
    st.o[t] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(pa, vbf, st.o[t], 0, 0, 0);
  }
}

template <int kKvHeads, int kWaves, int kG>
// Second bound: minimum wavefronts per SIMD, so that kGroupsPerCu workgroups fit on a CU
// (4 SIMDs per CU) and the whole grid is resident.
__global__ __launch_bounds__(64 * kWaves, (kGroupsPerCu * kWaves + 3) / 4) void paged_decode_kernel(const DecodeArgs a) {
  constexpr int kThreads = 64 * kWaves;
  constexpr int kRowElems = kKvHeads * kHeadDim;     // elements of one pool row (token)
  constexpr int kBlockElems = kBlockSize * kRowElems;
  constexpr int kHeadGroups = kKvHeads / kWaves;
  constexpr int kHeads = kKvHeads * kG;
  constexpr bool kMfma = kG >= kMfmaGroup;
  static_assert(kG <= 16, "at most 16 query heads per KV head");

  extern __shared__ int s_off[];                     // [batch + 1] block prefix sums
  __shared__ int s_wave[kWaves];
  __shared__ __align__(16) uint16_t s_kst[kMfma ? kWaves : 1][kMfma ? kBlockSize * kKStageRow : 8];
  const int total = scan_blocks<kThreads>(a, s_off, s_wave);
  int wg = blockIdx.x;
  if (kXcdRun > 0) {
    // Workgroups go round-robin to the XCDs: within each super-run of kXcds * kXcdRun workgroups,
    // those on XCD i take [i kXcdRun, (i + 1) kXcdRun) in order, so the head groups of a range share
    // an XCD; the partial tail keeps identity.
    constexpr int kSuper = kXcds * kXcdRun;
    const int n = a.streams * kHeadGroups;
    if (wg < n / kSuper * kSuper) {
      const int base = wg / kSuper * kSuper, r = wg - base;
      wg = base + (r % kXcds) * kXcdRun + r / kXcds;
    }
  }
  const int stream = wg / kHeadGroups;
  const int hg = wg - stream * kHeadGroups;
  const int64_t lo = static_cast<int64_t>(stream) * total / a.streams;
  const int64_t hi = static_cast<int64_t>(stream + 1) * total / a.streams;
  if (lo >= hi) return;

  const int lane = threadIdx.x & 63;
  const int dl = lane & 15;
  const int r = lane >> 4;
  const int g = hg * kWaves + (threadIdx.x >> 6);
  const float scale = a.scale;
  // Lane offsets (elements) of its first K and V pieces inside a block, and the step between its
  // four pieces.  K (both forms) and V of the dot-product form: tokens 4 i + r, dims 8 dl .. +8;
  // V of the matrix-core form: token 4 r + i, dims 8 dl .. +8.
  const int k_off = r * kRowElems + g * kHeadDim + 8 * dl;
  const int v_off = kMfma ? 4 * r * kRowElems + g * kHeadDim + 8 * dl : k_off;
  constexpr int kKStep = 4 * kRowElems;
  constexpr int kVStep = kMfma ? kRowElems : 4 * kRowElems;

  // Block ids of window [base, base + 64), one per lane (indices past the range repeat its
  // last block; ids outside the pool read block 0).
  auto fetch_ids = [&](int64_t base, uint32_t& id_lo, uint32_t& id_hi) {
    const int64_t x = min(base + lane, hi - 1);
    const int b = row_of(s_off, a.batch, x);
    int64_t id = a.block_tables[b * a.bt_stride + (x - s_off[b])];
    if (id < 0 || id >= a.num_blocks) id = 0;
    id_lo = static_cast<uint32_t>(id);
    id_hi = static_cast<uint32_t>(static_cast<uint64_t>(id) >> 32);
  };
  int64_t wbase = lo;
  uint32_t cur_lo, cur_hi, nxt_lo, nxt_hi;
  fetch_ids(wbase, cur_lo, cur_hi);
  fetch_ids(wbase + kWindow, nxt_lo, nxt_hi);

  u32x4 kbuf[kDepth][4], vbuf[kDepth][4];
  // Loads block y (clamped to the range) into ring slot `slot`; y never passes the next window.
  auto issue = [&](int slot, int64_t y) {
    y = min(y, hi - 1);
    if (y >= wbase + kWindow) {  // wave-uniform: slide the window, fetch the one after
      wbase += kWindow;
      cur_lo = nxt_lo;
      cur_hi = nxt_hi;
      fetch_ids(wbase + kWindow, nxt_lo, nxt_hi);
    }
    const int j = static_cast<int>(y - wbase);
    const uint32_t blo = __builtin_amdgcn_readlane(cur_lo, j);
    const uint32_t bhi = __builtin_amdgcn_readlane(cur_hi, j);
    const int64_t base = static_cast<int64_t>((static_cast<uint64_t>(bhi) << 32) | blo) * kBlockElems;
    const uint16_t* kp = a.key_pool + base + k_off;
    const uint16_t* vp = a.value_pool + base + v_off;
#pragma unroll
    for (int i = 0; i < 4; ++i) kbuf[slot][i] = load_vec<kNtLoads>(reinterpret_cast<const u32x4*>(kp + i * kKStep));
#pragma unroll
    for (int i = 0; i < 4; ++i) vbuf[slot][i] = load_vec<kNtLoads>(reinterpret_cast<const u32x4*>(vp + i * kVStep));
  };
#pragma unroll
  for (int s = 0; s < kDepth - 1; ++s) issue(s, lo + s);  // ring slot of block x: (x - lo) % kDepth

  int b = row_of(s_off, a.batch, lo);
  int64_t x = lo;
  while (x < hi) {
    const int64_t row_lo = s_off[b], row_hi = s_off[b + 1];
    const int64_t seg_end = min(hi, row_hi);
    const int n32 = static_cast<int>(context_of(a, b));  // contexts are bounded by max_blocks * 16 < 2^31
    const uint16_t* qp = a.query + b * a.q_row + (g * kG) * a.q_head;
    uint4 q[kMfma ? 1 : kG];
    bf16x8 qf[4];
    RowState<kMfma ? 1 : kG> st;
    MfmaState ms;
    if constexpr (kMfma) {  // Q^T fragments: head dl (zero past the group), dims 32 ks + 8 r .. +8
#pragma unroll
      for (int ks = 0; ks < 4; ++ks)
        qf[ks] = dl < kG ? *reinterpret_cast<const bf16x8*>(qp + dl * a.q_head + 32 * ks + 8 * r) : bf16x8{};
      ms.m = -INFINITY;
      ms.l = 0.0f;
#pragma unroll
      for (int t = 0; t < 8; ++t) ms.o[t] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    } else {
#pragma unroll
      for (int j = 0; j < kG; ++j) q[j] = *reinterpret_cast<const uint4*>(qp + j * a.q_head + 8 * dl);
      st.init();
    }

    const int64_t seg_begin = x;
    for (int64_t x0 = x - (x - lo) % kDepth; x0 < seg_end; x0 += kDepth) {
#pragma unroll
      for (int s = 0; s < kDepth; ++s) {
        const int64_t xb = x0 + s;
        if (xb < seg_begin || xb >= seg_end) continue;  // wave-uniform
        issue((s + kDepth - 1) % kDepth, xb + kDepth - 1);
        const int tok_base = static_cast<int>(xb - row_lo) * kBlockSize;
        if constexpr (kMfma)
          attend_block_mfma(ms, qf, kbuf[s], vbuf[s], s_kst[threadIdx.x >> 6], scale, tok_base, n32, lane);
        else
          attend_block<kG>(st, q, kbuf[s], vbuf[s], scale, tok_base, n32, r);
      }
    }
    x = seg_end;
    const bool whole = row_lo >= lo && row_hi <= hi;  // the whole sequence is in this range

    if constexpr (kMfma) {
      // Column sums, then each lane's heads 4 r + i (their m and sum live in lanes 4 r + i).
      float lsum = ms.l + __shfl_xor(ms.l, 16);
      lsum += __shfl_xor(lsum, 32);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int j = 4 * r + i;
        const float Lj = __shfl(lsum, j);
        const float Mj = __shfl(ms.m, j);
        if (j >= kG) continue;
        const int h = g * kG + j;
        float o[8];
#pragma unroll
        for (int t = 0; t < 8; ++t) o[t] = ms.o[t][i];
        if (whole) {
          store_bf16x8(a.out + b * a.out_row + h * kHeadDim + 8 * dl, o, 1.0f / Lj);
        } else {  // cut sequence: slot 0 if it began before this range (its first), else 1 (its last)
          const int64_t slot = (static_cast<int64_t>(stream) * 2 + (row_lo < lo ? 0 : 1)) * kHeads + h;
          float4* dst = reinterpret_cast<float4*>(a.ws_acc + slot * kHeadDim + 8 * dl);
          dst[0] = make_float4(o[0], o[1], o[2], o[3]);
          dst[1] = make_float4(o[4], o[5], o[6], o[7]);
          if (dl == 0) {
            a.ws_ml[slot * 2 + 0] = Mj;
            a.ws_ml[slot * 2 + 1] = Lj;
          }
        }
      }
      if (x < hi) {  // next non-empty sequence (uniform)
        while (s_off[b + 1] <= x) ++b;
      }
      continue;
    }

    float M[kMfma ? 1 : kG];
    merge_rows<kMfma ? 1 : kG>(st, M);
    // Row r writes query heads g kG + j for j = r, r + 4, ... (every row has all after the merge).
#pragma unroll
    for (int j = 0; j < (kMfma ? 0 : kG); ++j) {
      if ((j & 3) != r) continue;
      const int h = g * kG + j;
      if (whole) {
        store_bf16x8(a.out + b * a.out_row + h * kHeadDim + 8 * dl, st.acc[j], 1.0f / st.l[j]);
      } else {  // cut sequence: slot 0 if it began before this range (its first), else 1 (its last)
        const int64_t slot = (static_cast<int64_t>(stream) * 2 + (row_lo < lo ? 0 : 1)) * kHeads + h;
        float4* dst = reinterpret_cast<float4*>(a.ws_acc + slot * kHeadDim + 8 * dl);
        dst[0] = make_float4(st.acc[j][0], st.acc[j][1], st.acc[j][2], st.acc[j][3]);
        dst[1] = make_float4(st.acc[j][4], st.acc[j][5], st.acc[j][6], st.acc[j][7]);
        if (dl == 0) {
          a.ws_ml[slot * 2 + 0] = M[j];
          a.ws_ml[slot * 2 + 1] = st.l[j];
        }
      }
    }
    if (x < hi) {  // next non-empty sequence (uniform)
      while (s_off[b + 1] <= x) ++b;
    }
  }
}

// ---- Small launches: one workgroup per (sequence, KV head).  Its kSeqWaves wavefronts take
// blocks w, w + kSeqWaves, ... of the sequence with the stream kernel's per-block arithmetic
// (same lane layout, rounding points and lazy rescale), merge their four rows, then merge the
// wavefronts' softmax states through LDS and write the bf16 rows: one launch, nothing in the
// workspace.  A few sequences then spread over many wavefronts instead of a few block ranges
// that a second launch has to merge.
#ifndef MI_DECODE_SEQ_WAVES
#define MI_DECODE_SEQ_WAVES 8
#endif
#ifndef MI_DECODE_SEQ_DEPTH
#define MI_DECODE_SEQ_DEPTH 2
#endif
constexpr int kSeqWaves = MI_DECODE_SEQ_WAVES;
constexpr int kSeqMaxBlocks = 64 * kSeqWaves;  // a lane holds one block id of its wavefront

// kFused: the workgroup first does what mi_qk_norm_rope's decode form does for its heads --
// wavefronts 0 and 1 normalise and rotate query heads 2 g and 2 g + 1 into LDS, wavefront 2 key
// head g, which it writes with value head g into the sequence's new slot -- then attends.  The
// barrier after the pool stores makes them visible to the workgroup's own loads of that block
// (the slot's lines are not in the CU cache before: no other workgroup reads head g of this
// sequence, and the cache starts every launch clean).
template <int kKvHeads, int kG, bool kFused>
__global__ __launch_bounds__(64 * kSeqWaves) void paged_decode_seq_kernel(const DecodeArgs a) {
  constexpr int kRowElems = kKvHeads * kHeadDim;
  constexpr int kBlockElems = kBlockSize * kRowElems;
  constexpr int kSeqDepth = MI_DECODE_SEQ_DEPTH;  // ring: the next kSeqDepth - 1 blocks of the wavefront in flight
  __shared__ float s_acc[kSeqWaves][kG][kHeadDim];
  __shared__ float s_ml[kSeqWaves][kG][2];
  __shared__ __align__(16) uint16_t s_q[kFused ? kG : 1][kHeadDim];
  constexpr bool kMfmaForm = kG >= kSeqMfmaGroup;
  __shared__ __align__(16) uint16_t s_kst[kMfmaForm ? kSeqWaves : 1][kMfmaForm ? kBlockSize * kKStageRow : 8];
  const int b = blockIdx.x;
  const int g = blockIdx.y;
  const int w = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  const int dl = lane & 15;
  const int r = lane >> 4;
  if constexpr (kFused) {
    // Unit u < kG: query head g kG + u, normalised and rotated into LDS; unit kG: key head g,
    // written with value head g into the sequence's new slot.  Wavefront w takes units
    // w, w + kSeqWaves, ...
    for (int u = w; u <= kG; u += kSeqWaves) {  // wave-uniform
      const bool is_q = u < kG;
      const uint16_t* src = is_q ? a.q_raw + b * a.q_raw_row + (g * kG + u) * kHeadDim
                                 : a.k_raw + b * a.k_raw_row + g * kHeadDim;
      float o0, o1;
      norm_rope_head(src, is_q ? a.q_weight : a.k_weight, a.cos + b * kHeadDim, a.sin + b * kHeadDim, a.eps, lane,
                     o0, o1);
      if (is_q) {
        s_q[u][lane] = static_cast<uint16_t>(f32_to_bf16_bits(o0));
        s_q[u][lane + 64] = static_cast<uint16_t>(f32_to_bf16_bits(o1));
      } else {
        const int64_t slot = a.slot_mapping[b * a.slot_stride];
        if (slot >= 0 && slot < a.num_slots) {
          uint16_t* kd = const_cast<uint16_t*>(a.key_pool) + (slot * kKvHeads + g) * kHeadDim;
          uint16_t* vd = const_cast<uint16_t*>(a.value_pool) + (slot * kKvHeads + g) * kHeadDim;
          const uint16_t* vs = a.v_raw + b * a.v_raw_row + g * kHeadDim;
          kd[lane] = static_cast<uint16_t>(f32_to_bf16_bits(o0));
          kd[lane + 64] = static_cast<uint16_t>(f32_to_bf16_bits(o1));
          vd[lane] = vs[lane];
          vd[lane + 64] = vs[lane + 64];
        }
      }
    }
    __syncthreads();
  }
  const int n = static_cast<int>(context_of(a, b));
  const int nblk = blocks_of(n);
  uint16_t* out_b = a.out + b * a.out_row + (g * kG) * kHeadDim;  // query heads g kG .. g kG + kG - 1
  if (nblk == 0) {  // empty context: zero rows (uniform over the workgroup)
    if (threadIdx.x < kG * 16) *reinterpret_cast<uint4*>(out_b + 8 * threadIdx.x) = uint4{0, 0, 0, 0};
    return;
  }
  const float scale = a.scale;
  constexpr bool kMfma = kMfmaForm;  // lane layout and per-block arithmetic as in the stream kernel
  static_assert(kG <= 16, "at most 16 query heads per KV head");
  const int k_off = r * kRowElems + g * kHeadDim + 8 * dl;
  const int v_off = kMfma ? 4 * r * kRowElems + g * kHeadDim + 8 * dl : k_off;
  constexpr int kKStep = 4 * kRowElems;
  constexpr int kVStep = kMfma ? kRowElems : 4 * kRowElems;
  const int cnt = nblk > w ? (nblk - 1 - w) / kSeqWaves + 1 : 0;  // blocks w + kSeqWaves i, i < cnt <= 64

  // Lane i holds the id of block w + kSeqWaves i (ids outside the pool read block 0).
  uint32_t id_lo = 0, id_hi = 0;
  if (lane < cnt) {
    int64_t id = a.block_tables[b * a.bt_stride + w + kSeqWaves * lane];
    if (id < 0 || id >= a.num_blocks) id = 0;
    id_lo = static_cast<uint32_t>(id);
    id_hi = static_cast<uint32_t>(static_cast<uint64_t>(id) >> 32);
  }
  uint4 q[kMfma ? 1 : kG];
  bf16x8 qf[4];
  RowState<kMfma ? 1 : kG> st;
  MfmaState ms;
  if constexpr (kMfma) {  // Q^T fragments: head dl (zero past the group), dims 32 ks + 8 r .. +8
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      if constexpr (kFused)
        qf[ks] = dl < kG ? *reinterpret_cast<const bf16x8*>(&s_q[dl < kG ? dl : 0][32 * ks + 8 * r]) : bf16x8{};
      else
        qf[ks] = dl < kG ? *reinterpret_cast<const bf16x8*>(a.query + b * a.q_row + (g * kG + dl) * a.q_head +
                                                            32 * ks + 8 * r)
                         : bf16x8{};
    }
    ms.m = -INFINITY;
    ms.l = 0.0f;
#pragma unroll
    for (int t = 0; t < 8; ++t) ms.o[t] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  } else {
#pragma unroll
    for (int j = 0; j < kG; ++j) {
      if constexpr (kFused)
        q[j] = *reinterpret_cast<const uint4*>(&s_q[j][8 * dl]);
      else
        q[j] = *reinterpret_cast<const uint4*>(a.query + b * a.q_row + (g * kG + j) * a.q_head + 8 * dl);
    }
    st.init();
  }

  u32x4 kbuf[kSeqDepth][4], vbuf[kSeqDepth][4];
  auto issue = [&](int slot, int i) {  // block w + kSeqWaves i, clamped to the wavefront's last
    i = min(i, cnt - 1);
    const uint32_t blo = __builtin_amdgcn_readlane(id_lo, i);
    const uint32_t bhi = __builtin_amdgcn_readlane(id_hi, i);
    const int64_t base = static_cast<int64_t>((static_cast<uint64_t>(bhi) << 32) | blo) * kBlockElems;
    const uint16_t* kp = a.key_pool + base + k_off;
    const uint16_t* vp = a.value_pool + base + v_off;
#pragma unroll
    for (int t = 0; t < 4; ++t) kbuf[slot][t] = load_vec<kNtLoads>(reinterpret_cast<const u32x4*>(kp + t * kKStep));
#pragma unroll
    for (int t = 0; t < 4; ++t) vbuf[slot][t] = load_vec<kNtLoads>(reinterpret_cast<const u32x4*>(vp + t * kVStep));
  };
  if (cnt > 0) {  // wave-uniform
#pragma unroll
    for (int s = 0; s < kSeqDepth - 1; ++s) issue(s, s);  // ring slot of block i: i % kSeqDepth
    if (kSeqDepth == 1) issue(0, 0);
    // Whole rounds of kSeqDepth blocks, so that the loads stay in straight-line code the compiler
    // can count: indices past cnt re-read the last block and mask all its tokens (block
    // w + kSeqWaves i >= nblk starts at or past the context end).
    for (int i0 = 0; i0 < cnt; i0 += kSeqDepth) {
#pragma unroll
      for (int s = 0; s < kSeqDepth; ++s) {
        const int i = i0 + s;
        if (kSeqDepth > 1) issue((s + kSeqDepth - 1) % kSeqDepth, i + kSeqDepth - 1);
        else if (i > 0) issue(0, i);
        if constexpr (kMfma)
          attend_block_mfma(ms, qf, kbuf[s], vbuf[s], s_kst[w], scale, (w + kSeqWaves * i) * kBlockSize, n, lane);
        else
          attend_block<kG>(st, q, kbuf[s], vbuf[s], scale, (w + kSeqWaves * i) * kBlockSize, n, r);
      }
    }
  }

  // ---- merge the four rows of the wavefront (log-sum-exp), then the wavefronts through LDS
  if constexpr (kMfma) {  // lane: heads 4 r + i, dims 8 dl .. +8; head j's max and sum live in lane j
    float lsum = ms.l + __shfl_xor(ms.l, 16);
    lsum += __shfl_xor(lsum, 32);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int j = 4 * r + i;
      const float Lj = __shfl(lsum, j);
      const float Mj = __shfl(ms.m, j);
      if (j >= kG) continue;
#pragma unroll
      for (int t = 0; t < 8; ++t) s_acc[w][j][8 * dl + t] = ms.o[t][i];
      if (dl == 0) {
        s_ml[w][j][0] = Mj;
        s_ml[w][j][1] = Lj;
      }
    }
  }
  float M[kMfma ? 1 : kG];
  if constexpr (!kMfma) merge_rows<kG>(st, M);
#pragma unroll
  for (int j = 0; j < (kMfma ? 0 : kG); ++j) {  // row r holds heads j = r, r + 4, ... (every row has all after the merge)
    if ((j & 3) != r) continue;
#pragma unroll
    for (int d = 0; d < 8; ++d) s_acc[w][j][8 * dl + d] = st.acc[j][d];
    if (dl == 0) {
      s_ml[w][j][0] = M[j];
      s_ml[w][j][1] = st.l[j];
    }
  }
  __syncthreads();
  if (threadIdx.x < kG * 16) {
    const int h = threadIdx.x >> 4;
    const int dm = threadIdx.x & 15;
    float Mx = -INFINITY;
    for (int v = 0; v < kSeqWaves; ++v) Mx = fmaxf(Mx, s_ml[v][h][0]);
    float L = 0.0f, o[8];
#pragma unroll
    for (int d = 0; d < 8; ++d) o[d] = 0.0f;
    for (int v = 0; v < kSeqWaves; ++v) {
      const float mv = s_ml[v][h][0];
      const float e = mv == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(mv - Mx);
      L += e * s_ml[v][h][1];
#pragma unroll
      for (int d = 0; d < 8; ++d) o[d] += e * s_acc[v][h][8 * dm + d];
    }
    store_bf16x8(out_b + h * kHeadDim + 8 * dm, o, 1.0f / L);
  }
}

// Finishes what the stream kernel left: sequences cut by a range boundary (merge of their
// partials: the cut range's last-sequence slot, then the first-sequence slot of every later
// range up to the one holding the sequence's last block) and empty contexts (zero rows).
// grid: batch; block: heads * 16 lanes rounded up to whole wavefronts, lane (h, dm) < heads * 16
// owns dims [8 dm, 8 dm + 8) of head h.
template <int kHeads>
constexpr int merge_threads() { return (kHeads * 16 + 63) / 64 * 64; }

template <int kHeads>
__global__ __launch_bounds__(merge_threads<kHeads>()) void paged_decode_merge_kernel(const DecodeArgs a) {
  constexpr int kThreads = merge_threads<kHeads>();
  extern __shared__ int s_off[];
  __shared__ int s_wave[kThreads / 64];
  const int total = scan_blocks<kThreads>(a, s_off, s_wave);
  const int b = blockIdx.x;
  if (threadIdx.x >= kHeads * 16) return;
  const int h = threadIdx.x >> 4;
  const int dm = threadIdx.x & 15;
  uint16_t* dst = a.out + b * a.out_row + h * kHeadDim + 8 * dm;
  const int nblk = s_off[b + 1] - s_off[b];
  if (nblk == 0) {
    *reinterpret_cast<uint4*>(dst) = uint4{0, 0, 0, 0};
    return;
  }
  const int first = stream_of(s_off[b], total, a.streams);
  const int last = stream_of(s_off[b + 1] - 1, total, a.streams);
  if (first == last) return;  // written by the stream kernel
  // Partials: the first range's last-sequence slot (1), then the first-sequence slot (0) of each
  // later non-empty range up to `last` (empty ranges -- fewer blocks than ranges -- wrote nothing).
  auto slot_of = [&](int k) -> int64_t { return (static_cast<int64_t>(k) * 2 + (k == first ? 1 : 0)) * kHeads + h; };
  auto empty = [&](int k) {
    return static_cast<int64_t>(k) * total / a.streams >= static_cast<int64_t>(k + 1) * total / a.streams;
  };
  // kMergeUnroll partials per step with independent loads (a serial chain of dependent loads
  // would make a launch of many cut sequences latency-bound).
  constexpr int kMergeUnroll = 4;
  float M = -INFINITY;
  for (int k0 = first; k0 <= last; k0 += kMergeUnroll) {
    float m[kMergeUnroll];
#pragma unroll
    for (int u = 0; u < kMergeUnroll; ++u) {
      const int k = k0 + u;
      m[u] = (k <= last && !empty(k)) ? a.ws_ml[slot_of(k) * 2] : -INFINITY;
    }
#pragma unroll
    for (int u = 0; u < kMergeUnroll; ++u) M = fmaxf(M, m[u]);
  }
  float L = 0.0f, acc[8];
#pragma unroll
  for (int d = 0; d < 8; ++d) acc[d] = 0.0f;
  for (int k0 = first; k0 <= last; k0 += kMergeUnroll) {
    float m[kMergeUnroll], l[kMergeUnroll];
    float4 xv[kMergeUnroll], yv[kMergeUnroll];
#pragma unroll
    for (int u = 0; u < kMergeUnroll; ++u) {
      const int k = k0 + u;
      if (k <= last && !empty(k)) {
        const int64_t slot = slot_of(k);
        m[u] = a.ws_ml[slot * 2];
        l[u] = a.ws_ml[slot * 2 + 1];
        const float4* src = reinterpret_cast<const float4*>(a.ws_acc + slot * kHeadDim + 8 * dm);
        xv[u] = src[0];
        yv[u] = src[1];
      } else {
        m[u] = -INFINITY;
        l[u] = 0.0f;
        xv[u] = yv[u] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
      }
    }
#pragma unroll
    for (int u = 0; u < kMergeUnroll; ++u) {
      const float w = m[u] == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(m[u] - M);
      L += w * l[u];
      acc[0] += w * xv[u].x; acc[1] += w * xv[u].y; acc[2] += w * xv[u].z; acc[3] += w * xv[u].w;
      acc[4] += w * yv[u].x; acc[5] += w * yv[u].y; acc[6] += w * yv[u].z; acc[7] += w * yv[u].w;
    }
  }
  store_bf16x8(dst, acc, 1.0f / L);
}

int head_groups_for(int32_t num_kv_heads) {
  const int waves = num_kv_heads < kMaxWaves ? num_kv_heads : kMaxWaves;
  return num_kv_heads / waves;
}

// Ranges of one launch of `batch` sequences: enough to fill the device (kGroupsPerCu resident
// workgroups per CU), fewer when the launch cannot hold kMinBlocksPerStream blocks per range.
int streams_for(int32_t batch, int32_t max_blocks, int32_t num_kv_heads) {
  const int64_t groups = head_groups_for(num_kv_heads);
  const int64_t resident = static_cast<int64_t>(device_cus()) * kGroupsPerCu / groups;
  const int64_t rows = batch < kMaxBatchPerLaunch ? batch : kMaxBatchPerLaunch;
  const int64_t by_work = (rows * max_blocks + kMinBlocksPerStream - 1) / kMinBlocksPerStream;
  const int64_t s = by_work < resident ? by_work : resident;
  return static_cast<int>(s < 1 ? 1 : s);
}

// The per-sequence kernel serves launches of at most one workgroup per CU with tables it can
// hold; MI_DECODE_PATH=stream or =seq (environment) forces one kernel where both apply.
bool use_seq_path(int32_t batch, int32_t max_blocks, int32_t num_kv_heads) {
  if (max_blocks <= 0 || max_blocks > kSeqMaxBlocks) return false;
  const char* forced = getenv("MI_DECODE_PATH");
  if (forced && strcmp(forced, "stream") == 0) return false;
  if (forced && strcmp(forced, "seq") == 0) return true;
  return static_cast<int64_t>(batch) * num_kv_heads <= device_cus();
}

template <int kKvHeads, int kG, bool kFused>
int32_t launch_decode(const DecodeArgs& a, bool seq_path, hipStream_t s) {
  constexpr int kWaves = kKvHeads < kMaxWaves ? kKvHeads : kMaxWaves;
  constexpr int kHeadGroups = kKvHeads / kWaves;
  constexpr int kHeads = kKvHeads * kG;
  constexpr int kMergeThreads = merge_threads<kHeads>();
  const size_t lds = sizeof(int) * (static_cast<size_t>(a.batch) + 1);
  if (seq_path) {
    if (a.max_blocks > kSeqMaxBlocks) return fail(MI_ERR_UNSUPPORTED, "mi_paged_decode_attention: table too long");
    paged_decode_seq_kernel<kKvHeads, kG, kFused><<<dim3(a.batch, kKvHeads), 64 * kSeqWaves, 0, s>>>(a);
    return check_launch("mi_paged_decode_attention(seq)");
  }
  if constexpr (kFused) return fail(MI_ERR_UNSUPPORTED, "mi_paged_decode_attention: fused form needs the per-sequence kernel");
  if (a.max_blocks > 0) {
    paged_decode_kernel<kKvHeads, kWaves, kG><<<static_cast<uint32_t>(a.streams) * kHeadGroups, 64 * kWaves, lds, s>>>(a);
    int32_t rc = check_launch("mi_paged_decode_attention");
    if (rc != MI_OK) return rc;
  }
  paged_decode_merge_kernel<kHeads><<<a.batch, kMergeThreads, lds, s>>>(a);
  return check_launch("mi_paged_decode_attention(merge)");
}

// GQA groups (query heads per KV head) with compiled kernels: Qwen3 dense models use 2 (0.6B,
// 1.7B), 4 (4B, 8B), 5 (14B) and 8 (32B); 1 is multi-head attention.
bool group_supported(int group) { return group == 1 || group == 2 || group == 4 || group == 5 || group == 8; }

template <int kG, bool kFused>
int32_t launch_for_kv_heads(const DecodeArgs& a, int32_t num_kv_heads, bool seq_path, hipStream_t s) {
  switch (num_kv_heads) {
    case 1: return launch_decode<1, kG, kFused>(a, seq_path, s);
    case 2: return launch_decode<2, kG, kFused>(a, seq_path, s);
    case 4: return launch_decode<4, kG, kFused>(a, seq_path, s);
    default: return launch_decode<8, kG, kFused>(a, seq_path, s);
  }
}

template <bool kFused>
int32_t launch_for_heads(const DecodeArgs& a, int32_t num_heads, int32_t num_kv_heads, bool seq_path, hipStream_t s) {
  switch (num_heads / num_kv_heads) {
    case 1: return launch_for_kv_heads<1, kFused>(a, num_kv_heads, seq_path, s);
    case 2: return launch_for_kv_heads<2, kFused>(a, num_kv_heads, seq_path, s);
    case 4: return launch_for_kv_heads<4, kFused>(a, num_kv_heads, seq_path, s);
    case 5: return launch_for_kv_heads<5, kFused>(a, num_kv_heads, seq_path, s);
    default: return launch_for_kv_heads<8, kFused>(a, num_kv_heads, seq_path, s);
  }
}

// Shape checks shared by the entry points; returns MI_OK or the error it recorded.
int32_t check_heads(const char* what, int32_t num_heads, int32_t num_kv_heads, int32_t head_dim, int32_t block_size) {
  if (head_dim != kHeadDim || block_size != kBlockSize || num_kv_heads <= 0 || num_heads <= 0 ||
      num_heads % num_kv_heads != 0)
    return fail(MI_ERR_UNSUPPORTED,
                "%s: needs head_dim %d, block_size %d, num_heads a multiple of num_kv_heads "
                "(got head_dim %d, block_size %d, heads %d/%d)",
                what, kHeadDim, kBlockSize, head_dim, block_size, num_heads, num_kv_heads);
  if (num_kv_heads != 1 && num_kv_heads != 2 && num_kv_heads != 4 && num_kv_heads != 8)
    return fail(MI_ERR_UNSUPPORTED, "%s: num_kv_heads %d not in {1,2,4,8}", what, num_kv_heads);
  if (!group_supported(num_heads / num_kv_heads))
    return fail(MI_ERR_UNSUPPORTED, "%s: %d query heads per KV head not in {1,2,4,5,8}", what,
                num_heads / num_kv_heads);
  return MI_OK;
}

}  // namespace
}  // namespace mi

extern "C" int64_t mi_paged_decode_workspace_bytes(int32_t batch, int32_t max_blocks, int32_t num_heads,
                                                   int32_t num_kv_heads, int32_t head_dim, int32_t block_size) {
  using namespace mi;
  if (batch <= 0 || max_blocks <= 0 || num_heads <= 0 || num_kv_heads <= 0 || head_dim <= 0 ||
      block_size != kBlockSize || num_heads % num_kv_heads != 0)
    return 0;
  const int64_t streams = streams_for(batch, max_blocks, num_kv_heads);
  return streams * 2 * num_heads * (head_dim + 2) * static_cast<int64_t>(sizeof(float));
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
  if (const int32_t rc = reject_empty_pool("mi_paged_decode_attention", num_blocks, max_blocks > 0)) return rc;
  if (!out || !query || !key_pool || !value_pool || !context_lens || (max_blocks > 0 && !block_tables))
    return fail(MI_ERR_INVALID_ARGUMENT, "mi_paged_decode_attention: null pointer argument");
  if (const int32_t rc = check_heads("mi_paged_decode_attention", num_heads, num_kv_heads, head_dim, block_size))
    return rc;
  if (!aligned16(out) || !aligned16(query) || !aligned16(key_pool) || !aligned16(value_pool) ||
      out_row_stride % 8 != 0 || query_row_stride % 8 != 0 || query_head_stride % 8 != 0)
    return fail(MI_ERR_UNSUPPORTED, "mi_paged_decode_attention: query/out/pools must be 16-byte aligned");
  if (max_blocks > 0 && block_table_stride < max_blocks)
    return fail(MI_ERR_INVALID_ARGUMENT, "mi_paged_decode_attention: block_table_stride < max_blocks");
  if (context_lens_stride <= 0)
    return fail(MI_ERR_INVALID_ARGUMENT, "mi_paged_decode_attention: context_lens_stride must be > 0");
  if (static_cast<int64_t>(kMaxBatchPerLaunch) * max_blocks >= (1ll << 31))
    return fail(MI_ERR_UNSUPPORTED, "mi_paged_decode_attention: max_blocks %d too large", max_blocks);

  const int32_t streams = streams_for(batch, max_blocks, num_kv_heads);
  const int64_t need = mi_paged_decode_workspace_bytes(batch, max_blocks, num_heads, num_kv_heads, head_dim, block_size);
  if (max_blocks > 0 && (!workspace || workspace_bytes < need))
    return fail(MI_ERR_WORKSPACE, "mi_paged_decode_attention: workspace of %lld bytes needed, got %lld",
                static_cast<long long>(need), static_cast<long long>(workspace_bytes));
  if (max_blocks > 0 && !aligned16(workspace))
    return fail(MI_ERR_UNSUPPORTED, "mi_paged_decode_attention: workspace must be 16-byte aligned");
  float* ws_acc = static_cast<float*>(workspace);
  float* ws_ml = ws_acc ? ws_acc + static_cast<int64_t>(streams) * 2 * num_heads * kHeadDim : nullptr;

  hipStream_t s = as_stream(stream);
  const bool seq_path = use_seq_path(batch, max_blocks, num_kv_heads);
  // Sequences go in slices of at most kMaxBatchPerLaunch (the per-workgroup prefix sum lives in
  // LDS); the slices reuse the workspace one after the other on the stream.
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
    a.streams = streams;
    a.scale = scale;
    a.ws_acc = ws_acc;
    a.ws_ml = ws_ml;
    const int32_t rc = launch_for_heads<false>(a, num_heads, num_kv_heads, seq_path, s);
    if (rc != MI_OK) return rc;
  }
  return ok();
}

extern "C" int32_t mi_paged_decode_attention_fused(
    void* out, int64_t out_row_stride, const void* q, int64_t q_row_stride, const void* k, int64_t k_row_stride,
    const void* v, int64_t v_row_stride, const void* q_weight, const void* k_weight, const void* cos, const void* sin,
    float eps, const int64_t* slot_mapping, int64_t slot_stride, void* key_pool, void* value_pool, int64_t num_blocks,
    const int64_t* block_tables, int64_t block_table_stride, int32_t max_blocks, const int64_t* context_lens,
    int64_t context_lens_stride, int32_t batch, int32_t num_heads, int32_t num_kv_heads, int32_t head_dim,
    int32_t block_size, float scale, void* q_scratch, void* workspace, int64_t workspace_bytes, void* stream) {
  using namespace mi;
  if (batch < 0 || max_blocks < 0 || num_blocks < 0)
    return fail(MI_ERR_INVALID_ARGUMENT, "mi_paged_decode_attention_fused: negative size");
  if (batch == 0) return ok();
  if (const int32_t rc = reject_empty_pool("mi_paged_decode_attention_fused", num_blocks, max_blocks > 0)) return rc;
  if (!q || !k || !v || !q_weight || !k_weight || !cos || !sin || !slot_mapping || !q_scratch)
    return fail(MI_ERR_INVALID_ARGUMENT, "mi_paged_decode_attention_fused: null pointer argument");
  if (num_blocks > INT64_MAX / kBlockSize)
    return fail(MI_ERR_INVALID_ARGUMENT, "mi_paged_decode_attention_fused: pool too large");
  if (const int32_t rc = check_heads("mi_paged_decode_attention_fused", num_heads, num_kv_heads, head_dim, block_size))
    return rc;
  if (!use_seq_path(batch, max_blocks, num_kv_heads) || max_blocks == 0) {
    // Large launches: the two-launch form (the append and q rotation, then the stream kernel).
    int32_t rc = mi_qk_norm_rope(q_scratch, nullptr, nullptr, q, q_row_stride, k, k_row_stride, v, v_row_stride,
                                 q_weight, k_weight, cos, sin, batch, num_heads, num_kv_heads, head_dim, eps,
                                 slot_mapping, slot_stride, key_pool, value_pool, num_blocks * block_size, stream);
    if (rc != MI_OK) return rc;
    return mi_paged_decode_attention(out, out_row_stride, q_scratch, static_cast<int64_t>(num_heads) * head_dim,
                                     head_dim, key_pool, value_pool, num_blocks, block_tables, block_table_stride,
                                     max_blocks, context_lens, context_lens_stride, batch, num_heads, num_kv_heads,
                                     head_dim, block_size, scale, workspace, workspace_bytes, stream);
  }
  // One launch: the per-sequence kernel with the prologue.  Shape checks as in the two entry points.
  if (!out || !key_pool || !value_pool || !context_lens || !block_tables)
    return fail(MI_ERR_INVALID_ARGUMENT, "mi_paged_decode_attention_fused: null pointer argument");
  if (!aligned16(out) || !aligned16(key_pool) || !aligned16(value_pool) || out_row_stride % 8 != 0)
    return fail(MI_ERR_UNSUPPORTED, "mi_paged_decode_attention_fused: out/pools must be 16-byte aligned");
  if (block_table_stride < max_blocks || context_lens_stride <= 0 || q_row_stride < num_heads * head_dim ||
      k_row_stride < num_kv_heads * head_dim || v_row_stride < num_kv_heads * head_dim)
    return fail(MI_ERR_INVALID_ARGUMENT, "mi_paged_decode_attention_fused: bad stride");
  DecodeArgs a{};
  a.out = static_cast<uint16_t*>(out);
  a.out_row = out_row_stride;
  a.key_pool = static_cast<const uint16_t*>(key_pool);
  a.value_pool = static_cast<const uint16_t*>(value_pool);
  a.num_blocks = num_blocks;
  a.block_tables = block_tables;
  a.bt_stride = block_table_stride;
  a.context_lens = context_lens;
  a.ctx_stride = context_lens_stride;
  a.batch = batch;
  a.max_blocks = max_blocks;
  a.streams = 1;
  a.scale = scale;
  a.q_raw = static_cast<const uint16_t*>(q);
  a.k_raw = static_cast<const uint16_t*>(k);
  a.v_raw = static_cast<const uint16_t*>(v);
  a.q_raw_row = q_row_stride;
  a.k_raw_row = k_row_stride;
  a.v_raw_row = v_row_stride;
  a.q_weight = static_cast<const uint16_t*>(q_weight);
  a.k_weight = static_cast<const uint16_t*>(k_weight);
  a.cos = static_cast<const uint16_t*>(cos);
  a.sin = static_cast<const uint16_t*>(sin);
  a.slot_mapping = slot_mapping;
  a.slot_stride = slot_stride;
  a.num_slots = num_blocks * kBlockSize;
  a.eps = eps;
  return launch_for_heads<true>(a, num_heads, num_kv_heads, true, as_stream(stream));
}

// ---- The no-allocation variant.  The stream kernel's cut-sequence partials go to `scratch`, a
// fixed device array of this library (each GPU holds its own copy for the life of the process),
// instead of a caller workspace.  No part of it needs clearing: a partial slot is written by its
// range before the merge launch reads it.  Every call on one GPU shares the array, so calls that
// overlap on one GPU (different streams, or threads) race on it.
namespace mi {
namespace {
constexpr int64_t kScratchBytes = MI_PAGED_NOALLOC_SCRATCH_BYTES;  // 4.3 MB used at 16 / 8 heads on 256 CUs
constexpr int kMaxScratchDevices = 64;
}  // namespace
}  // namespace mi

static __device__ __align__(256) unsigned char scratch[mi::kScratchBytes];

namespace mi {
namespace {

// Device address of `scratch` on the current device, looked up once per device with that device
// current (the array's name is only a host-side stand-in for it).
int32_t scratch_on_current_device(void** out) {
  static std::mutex mu;
  static void* ptrs[kMaxScratchDevices] = {nullptr};
  int dev = 0;
  const hipError_t derr = hipGetDevice(&dev);
  if (derr != hipSuccess)
    return fail(MI_ERR_DEVICE, "mi_paged_decode_attention_noalloc: hipGetDevice: %s", hipGetErrorString(derr));
  if (dev < 0 || dev >= kMaxScratchDevices)
    return fail(MI_ERR_UNSUPPORTED, "mi_paged_decode_attention_noalloc: device %d beyond %d", dev, kMaxScratchDevices);
  std::lock_guard<std::mutex> lock(mu);
  if (ptrs[dev] == nullptr) {
    void* p = nullptr;
    const hipError_t err = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (err != hipSuccess || p == nullptr)
      return fail(MI_ERR_DEVICE, "mi_paged_decode_attention_noalloc: hipGetSymbolAddress(scratch): %s",
                  hipGetErrorString(err));
    ptrs[dev] = p;
  }
  *out = ptrs[dev];
  return MI_OK;
}

}  // namespace
}  // namespace mi

extern "C" int32_t mi_paged_decode_attention_noalloc(void* out, int64_t out_row_stride, const void* query,
                                                     int64_t query_row_stride, int64_t query_head_stride,
                                                     const void* key_pool, const void* value_pool, int64_t num_blocks,
                                                     const int64_t* block_tables, int64_t block_table_stride,
                                                     int32_t max_blocks, const int64_t* context_lens,
                                                     int64_t context_lens_stride, int32_t batch, int32_t num_heads,
                                                     int32_t num_kv_heads, int32_t head_dim, int32_t block_size,
                                                     float scale, void* stream) {
  using namespace mi;
  if (batch < 0 || max_blocks < 0 || num_blocks < 0)
    return fail(MI_ERR_INVALID_ARGUMENT, "mi_paged_decode_attention_noalloc: negative size");
  if (batch == 0) return ok();
  if (const int32_t rc = reject_empty_pool("mi_paged_decode_attention_noalloc", num_blocks, max_blocks > 0))
    return rc;
  if (const int32_t rc = check_heads("mi_paged_decode_attention_noalloc", num_heads, num_kv_heads, head_dim,
                                     block_size))
    return rc;
  // The size check comes before any launch, copy or scratch lookup (it only queries the current
  // device and its CU count): a launch that needs more than the fixed array is rejected before
  // any work reaches the GPU.
  const int64_t need =
      mi_paged_decode_workspace_bytes(batch, max_blocks, num_heads, num_kv_heads, head_dim, block_size);
  if (need > kScratchBytes)
    return fail(MI_ERR_WORKSPACE,
                "mi_paged_decode_attention_noalloc: this launch needs %lld bytes of scratch, the fixed array "
                "holds %lld (use mi_paged_decode_attention with a workspace)",
                static_cast<long long>(need), static_cast<long long>(kScratchBytes));
  void* ws = nullptr;
  if (need > 0) {
    if (const int32_t rc = scratch_on_current_device(&ws)) return rc;
  }
  return mi_paged_decode_attention(out, out_row_stride, query, query_row_stride, query_head_stride, key_pool,
                                   value_pool, num_blocks, block_tables, block_table_stride, max_blocks, context_lens,
                                   context_lens_stride, batch, num_heads, num_kv_heads, head_dim, block_size, scale,
                                   ws, need > 0 ? kScratchBytes : 0, stream);
}
