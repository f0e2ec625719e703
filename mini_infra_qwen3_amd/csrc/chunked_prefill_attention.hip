// Kernel 4: chunked-prefill attention on MFMA, history read straight from the paged pool.
//
// Behaviour of a chunked-prefill layer of the reference: the history gather of
// PagedKVCachePool.gather_blocks (src/mini_infra/worker/paged_kv_cache.py:54-72), the concat of
// history and chunk in Qwen3Attention.forward (src/mini_infra/model/qwen3.py:325-330), the visibility
// mask of PagedRunner.run_prefill_chunk_step (src/mini_infra/worker/paged_runner.py:83-89) with the
// causal mask of Qwen3Model._prepare_position_ids_and_allowed_mask (qwen3.py:477-484), and
// Qwen3Attention._attend (qwen3.py:219-255) -- as one flash-style kernel.
//
// Row b of the batch: chunk of padded length L whose last len_b positions are real (left
// padding), logical start start_b, history = the first nh = min(start_b, 16 * max_history_blocks)
// pool slots of its block table.  Query i (i >= L - len_b) sees every history slot k < nh and
// chunk keys j with L - len_b <= j <= i.  Rows i < L - len_b (padding) get a zero output.
//
// Tiling for gfx950 (v_mfma_f32_16x16x32_bf16, 64-lane wavefronts):
//  * workgroup = (row b, query-head pair p of KV head g, 128-query tile), 8 wavefronts (one
//    workgroup per CU at two waves per SIMD): wave w serves query head G g + 2 p + (w >> 2) of the
//    GQA group of G heads on KV head g and queries [32 (w & 3), +32) of the tile, so the two
//    heads share every K/V tile staged in LDS.  A group of G heads takes ceil(G / 2) pairs; when G
//    is odd, the second half of its last pair repeats the group's last head and writes nothing.
//  * KV tiles of 64 keys: history tiles first (pool blocks through the block table -- the
//    gather is fused, nothing is materialised), then chunk tiles up to the causal limit.
//    K is staged row-major (288-byte rows), V transposed (V^T) in double-buffered LDS; the loads
//    of the next two tiles are in flight in registers while the current one is multiplied.
//  * S^T = K Q^T: A = K rows from LDS, B = Q^T from registers (loaded once), C lane layout =
//    (query = lane % 16, keys 4 (lane / 16) + i).  Each query's softmax state lives in the
//    lanes of its column; the row max needs two cross-lane steps, the row sum is deferred.
//  * O^T = V^T P^T: the probabilities of a 32-key step are already in the B-operand lanes if
//    the MFMA's k index is read as key 16 (k' / 4) + 4 (lane / 16) + k' % 4; V^T rows in LDS
//    hold the keys in that order, so the A operand is one 16-byte read.
//  * Softmax and accumulation are fp32 with lazy rescaling of the running max as in the decode
//    kernel.  Scores keep the reference's bf16 rounding points (bf16 product, then bf16 product
//    with the scale), one packed bf16 convert per rounding: for N(0,1) inputs those roundings
//    move logits by ~1e-2, so dropping them would leave the 2e-2 parity band.
//  * Measured on MI355X, MFMA and VALU work of the same SIMD mostly add up rather than overlap,
//    so the time per tile is about MFMA + VALU: the score roundings, exponentials and converts
//    are the VALU share.
#include <algorithm>
#include <initializer_list>

#include "mi_common.h"

namespace mi {
namespace {

constexpr int kHeadDim = 128;
constexpr int kBlockSize = 16;
constexpr int kGroup = 2;  // query heads per workgroup (a pair of one GQA group)
#ifndef MI_PREFILL_WAVES_PER_HEAD
#define MI_PREFILL_WAVES_PER_HEAD 4
#endif
constexpr int kWavesPerHead = MI_PREFILL_WAVES_PER_HEAD;
#ifndef MI_PREFILL_NT
#define MI_PREFILL_NT 2
#endif
constexpr int kNt = MI_PREFILL_NT;                        // 16-query MFMA column tiles per wave
constexpr int kQPerWave = 16 * kNt;
constexpr int kQTile = kQPerWave * kWavesPerHead;         // queries per head per workgroup
constexpr int kWavesPerSimd = kNt == 1 ? 4 : 2;           // occupancy the register budget is set for
#ifndef MI_PREFILL_AHEAD
#define MI_PREFILL_AHEAD 2
#endif
constexpr int kAhead = MI_PREFILL_AHEAD;                  // K/V tiles in flight in registers (1 or 2)
static_assert(kAhead == 1 || kAhead == 2, "one or two tiles ahead");
constexpr int kKTile = 64;                 // keys per KV tile
#ifndef MI_PREFILL_K_PAD
#define MI_PREFILL_K_PAD 16
#endif
#ifndef MI_PREFILL_V_PAD
#define MI_PREFILL_V_PAD 16
#endif
constexpr int kKStride = kHeadDim + MI_PREFILL_K_PAD;  // LDS row of K (elements): 288 B
constexpr int kVStride = kKTile + MI_PREFILL_V_PAD;    // LDS row of V^T (elements): 160 B, 16-byte aligned
constexpr int kThreads = 64 * kGroup * kWavesPerHead;    // one workgroup per CU at 4 waves per head
constexpr int kKeysPerPass = kThreads / 16;               // K rows one pass of 16-byte pieces covers
constexpr int kKPieces = kKTile / kKeysPerPass;           // K pieces per thread and tile
constexpr int kVPieces = kKTile / (2 * kKeysPerPass);     // V key pairs per thread and tile
static_assert(kKPieces * kKeysPerPass == kKTile && kVPieces * 2 * kKeysPerPass == kKTile, "tile cover");
constexpr int kMaxHistoryBlocks = 16384;   // history table staged in LDS: 64 KiB at most (256k tokens)
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
  uint16_t* key_pool;
  uint16_t* value_pool;
  int64_t num_blocks;
  const int64_t* history_blocks;
  int64_t history_stride;
  int32_t max_history_blocks;
  const int64_t* start_lens;
  const int64_t* chunk_lens;
  int64_t lens_stride;
  int32_t padded_len;
  int32_t group;   // query heads per KV head (G)
  int32_t pairs;   // workgroups per KV head: ceil(G / 2)
  float scale;
  int32_t tiles;   // query tiles per row: ceil(padded_len / kQTile)
  int32_t batch;   // rows
  int32_t groups;  // workgroups of these rows: tiles x num_kv_heads x pairs x batch
  // Decode rows (a mixed step's single new tokens, padded_len 1): start_lens holds each row's
  // context length including its token, so the history is the context minus one and a row with
  // context 0 is padding; the token's K/V row is appended to pool slot slot_mapping[b] (skipped
  // when outside the pool) by the workgroup of the first head pair of each KV head.
  int32_t decode_rows;
  const int64_t* slot_mapping;
  int64_t slot_stride;
};

typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));

// bf16 rounding of one float as an fp32 value in one instruction: the packed convert with a zero
// low half leaves bf16(x) in the high half and zeros below, which is exactly bf16(x) as fp32.
__device__ __forceinline__ float round_bf16_hi(float x) {
  return __builtin_bit_cast(float, __builtin_convertvector((f32x2){0.0f, x}, bf16x2));
}

// The reference's scores: bf16(bf16(q . k) * scale) (src/mini_infra/model/qwen3.py:243), in place.
__device__ __forceinline__ void reference_scores(f32x4& v, float scale) {
#pragma unroll
  for (int i = 0; i < 4; ++i) v[i] = round_bf16_hi(round_bf16_hi(v[i]) * scale);
}

// Column (element) of key `key` in V^T row `dim`: rows of 32 dims are rotated by 8 keys (4 dwords)
// per group, so that the transposing stores -- each thread writes dims 8 x .. 8 x + 7 of two keys,
// x = lane % 16 -- spread over all banks (32 or 64 banks of 4 bytes) instead of 8 of them, while
// the PV operand reads (8 consecutive keys of one dim) stay contiguous and conflict-free.
__device__ __forceinline__ int vcol(int dim, int key) { return (key + 8 * (dim >> 5)) & (kKTile - 1); }
// Position of key k of a tile in its V^T row (before the vcol rotation): the 8 keys one lane group
// feeds to a PV MFMA (16 (k' / 4) + 4 (lane / 16) + k' % 4 within each 32-key half) sit next to
// each other, so the A operand is one 16-byte read; key pairs (2 j, 2 j + 1) stay adjacent.
__device__ __forceinline__ int vpos(int key) {
  const int k = key & 31;
  return (key & 32) + 8 * ((k & 15) >> 2) + 4 * (k >> 4) + (k & 3);
}

__device__ __forceinline__ uint32_t perm(uint32_t hi_src, uint32_t lo_src, uint32_t sel) {
  return __builtin_amdgcn_perm(hi_src, lo_src, sel);
}

// One launch serves up to two sets of rows (a mixed step's chunk rows and its decode rows): the
// first a0.groups workgroups take a0, the rest a1.
template <int kKvHeads>
__global__ __launch_bounds__(kThreads, kWavesPerSimd) void chunked_prefill_kernel(const PrefillArgs a0,
                                                                                   const PrefillArgs a1) {
  __shared__ __align__(16) uint16_t sK[2][kKTile * kKStride];
  __shared__ __align__(16) uint16_t sV[2][kHeadDim * kVStride];
  extern __shared__ int s_hblk[];  // [ceil(nh / 16)] history block ids of this row (dynamic LDS)

  const bool second = static_cast<int>(blockIdx.x) >= a0.groups;  // uniform
  const PrefillArgs a = second ? a1 : a0;

  // Workgroup -> (row b, head pair hp, query tile qt).  Consecutive workgroup ids go round-robin to
  // the 8 XCDs, each with its own L2; so that the query tiles of one (row, head) -- which stream
  // the same K/V tiles -- share an L2, id L runs on XCD L % 8 and takes the (L / 8)-th tile of that
  // XCD's (row, head pair) units in order.  Shapes whose pair count is not a multiple of 8 keep the
  // plain mapping.  Within a pair the heaviest (latest) query tiles start first.
  int b, hp, qt;
  {
    const int tiles = a.tiles;
    const int per_row = kKvHeads * a.pairs;
    const int pairs = per_row * a.batch;
    const int lin = static_cast<int>(blockIdx.x) - (second ? a0.groups : 0);
    int pair, rank;
    if (pairs % 8 == 0) {
      const int slot = lin >> 3;
      pair = (slot / tiles) * 8 + (lin & 7);
      rank = slot % tiles;
    } else {
      pair = lin / tiles;
      rank = lin % tiles;
    }
    hp = pair % per_row;
    b = pair / per_row;
    qt = tiles - 1 - rank;
  }
  const int q0 = qt * kQTile;
  const int L = a.padded_len;
  int64_t len64, start64;
  if (a.decode_rows) {
    const int64_t ctx = a.start_lens[b * a.lens_stride];
    len64 = ctx > 0 ? 1 : 0;
    start64 = ctx > 0 ? ctx - 1 : 0;
  } else {
    len64 = a.chunk_lens[b * a.lens_stride];
    start64 = a.start_lens[b * a.lens_stride];
  }
  len64 = len64 < 0 ? 0 : (len64 > L ? L : len64);
  const int pad = L - static_cast<int>(len64);
  start64 = start64 < 0 ? 0 : start64;
  const int64_t hist_cap = static_cast<int64_t>(a.max_history_blocks) * kBlockSize;
  const int nh = static_cast<int>(start64 < hist_cap ? start64 : hist_cap);

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave index, uniform: keeps edge-tile branches real
  const int hh = w / kWavesPerHead;
  const int qs = w % kWavesPerHead;
  const int g = hp / a.pairs;                    // KV head
  const int j0 = (hp - g * a.pairs) * kGroup;    // first head of the pair within the group
  const bool head_live = j0 + hh < a.group;      // wave-uniform: false for the spare half of an odd group
  const int h = g * a.group + min(j0 + hh, a.group - 1);
  const int ql = lane & 15;
  const int gq = lane >> 4;

  if (a.decode_rows && j0 == 0 && tid < 32 && len64 > 0) {  // append the token's K and V rows of KV head g
    const int64_t slot = a.slot_mapping[b * a.slot_stride];
    if (slot >= 0 && slot < a.num_blocks * kBlockSize) {
      const int piece = (tid & 15) * 8;
      const uint16_t* src = tid < 16 ? a.key + b * a.k_row + g * a.k_head : a.value + b * a.v_row + g * a.v_head;
      uint16_t* dst = (tid < 16 ? a.key_pool : a.value_pool) + (slot * kKvHeads + g) * kHeadDim;
      *reinterpret_cast<uint4*>(dst + piece) = *reinterpret_cast<const uint4*>(src + piece);
    }
  }

  uint16_t* out_b = a.out + b * a.out_row;
  if (q0 + kQTile <= pad) {  // the whole tile is padding: zero rows
    for (int c = tid; c < kQTile * kGroup * (kHeadDim / 8); c += kThreads) {
      const int qi = q0 + c / (kGroup * (kHeadDim / 8));
      const int rem = c % (kGroup * (kHeadDim / 8));
      const int jj = j0 + rem / (kHeadDim / 8);
      const int head = g * a.group + jj;
      if (qi < L && jj < a.group)
        *reinterpret_cast<uint4*>(out_b + qi * a.out_tok + head * kHeadDim + (rem % (kHeadDim / 8)) * 8) =
            uint4{0, 0, 0, 0};
    }
    return;
  }

  // ---- Q^T fragments (B operand): query column n = ql of n-tile nt, dims 32 ks + 8 gq .. +8
  bf16x8 qf[kNt][4];
  const int qw0 = q0 + kQPerWave * qs;  // first query of this wave
#pragma unroll
  for (int nt = 0; nt < kNt; ++nt) {
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

  // ---- tile loader.  Thread tid owns K pieces (key kKeysPerPass kk + tid / 16, dims 8 (tid % 16)
  // .. +8), kk < kKPieces, and V key pairs (keys 2 kKeysPerPass kk + 2 (tid / 16) + {0, 1}, same
  // dims), kk < kVPieces.  In a history tile each piece lies in pool block (its first key) / 16 of
  // the tile -- uniform across a wavefront, whose 64 lanes span 4 consecutive keys (or pairs) of
  // one block -- read from LDS where the workgroup staged its history table once.  Every load
  // reads valid memory: block indices are clamped to the last history block and chunk positions
  // to L - 1; keys past the context are masked later.
  const int tkey = tid >> 4;
  const int tdim = (tid & 15) * 8;
  const int nhb = (nh + kBlockSize - 1) / kBlockSize;
  for (int i = tid; i < nhb; i += kThreads) {
    const int64_t x = a.history_blocks[b * a.history_stride + i];
    s_hblk[i] = (x < 0 || x >= a.num_blocks) ? 0 : static_cast<int>(x);
  }
  constexpr int64_t kBlkElems = static_cast<int64_t>(kBlockSize) * kKvHeads * kHeadDim;
  // Per-lane parts of the load addresses (elements, 32-bit): the uniform parts -- the pool block
  // of a history piece, the first chunk row of a pass -- are added as one scalar base per load.
  const uint32_t k_hist_off = static_cast<uint32_t>(((tkey % kBlockSize) * kKvHeads + g) * kHeadDim + tdim);
  const int voff = (2 * tkey) % kBlockSize;
  const uint32_t v_hist_off0 = static_cast<uint32_t>((voff * kKvHeads + g) * kHeadDim + tdim);
  const uint32_t v_hist_off1 = v_hist_off0 + kKvHeads * kHeadDim;
  const uint16_t* k_rows = a.key + b * a.k_row + g * a.k_head;
  const uint16_t* v_rows = a.value + b * a.v_row + g * a.v_head;
  const uint32_t k_tok = static_cast<uint32_t>(a.k_tok);  // < 2^24, checked by the entry point
  const uint32_t v_tok = static_cast<uint32_t>(a.v_tok);

#define MI_HIST_BLOCK(T, KEY) \
  __builtin_amdgcn_readfirstlane(s_hblk[min((T) * (kKTile / kBlockSize) + (KEY) / kBlockSize, max(nhb - 1, 0))])
  // Loads of tile t, branch-free: each piece is a scalar base (pool block, or the chunk row of the
  // pass clamped to L - 1) plus a 32-bit lane offset, selected on the uniform history/chunk test,
  // so the compiler can count them and wait for exactly the pieces a store needs.  Chunk rows past
  // L - 1 read row L - 1 (their keys are masked).
  auto load_tile = [&](const int t, u32x4 (&kr)[kKPieces], u32x4 (&vr)[kVPieces][2]) {
    const bool hist = t < n_hist_tiles;
    const int key0 = (c_lo + t - n_hist_tiles) * kKTile;
#pragma unroll
    for (int kk = 0; kk < kKPieces; ++kk) {
      const int row = kKeysPerPass * kk;
      const int kc = min(key0 + row, L - 1);
      const uint32_t chunk_off = __umul24(static_cast<uint32_t>(min(tkey, L - 1 - kc)), k_tok) + tdim;
      const uint16_t* base = hist ? a.key_pool + static_cast<int64_t>(MI_HIST_BLOCK(t, row + tkey)) * kBlkElems
                                  : k_rows + static_cast<int64_t>(kc) * a.k_tok;
      const uint32_t off = hist ? k_hist_off : chunk_off;
      kr[kk] = *reinterpret_cast<const u32x4*>(reinterpret_cast<const char*>(base) + 2u * off);
    }
#pragma unroll
    for (int kk = 0; kk < kVPieces; ++kk) {
      const int row = 2 * kKeysPerPass * kk;
      const int vc = min(key0 + row, L - 1);
      const uint16_t* base = hist ? a.value_pool + static_cast<int64_t>(MI_HIST_BLOCK(t, row + 2 * tkey)) * kBlkElems
                                  : v_rows + static_cast<int64_t>(vc) * a.v_tok;
#pragma unroll
      for (int e = 0; e < 2; ++e) {
        const uint32_t chunk_off = __umul24(static_cast<uint32_t>(min(2 * tkey + e, L - 1 - vc)), v_tok) + tdim;
        const uint32_t off = hist ? (e ? v_hist_off1 : v_hist_off0) : chunk_off;
        vr[kk][e] = *reinterpret_cast<const u32x4*>(reinterpret_cast<const char*>(base) + 2u * off);
      }
    }
  };

#define MI_STORE_TILE(BUF, KR, VR)                                                                                 \
  do {                                                                                                         \
    const int buf_ = (BUF);                                                                                    \
    _Pragma("unroll") for (int kk = 0; kk < kKPieces; ++kk)                                                    \
        *reinterpret_cast<u32x4*>(&sK[buf_][(kKeysPerPass * kk + tkey) * kKStride + tdim]) = KR[kk];         \
    _Pragma("unroll") for (int kk = 0; kk < kVPieces; ++kk) {                                                  \
      const int key = 2 * kKeysPerPass * kk + 2 * tkey;                                                        \
      const uint32_t x[4] = {VR[kk][0][0], VR[kk][0][1], VR[kk][0][2], VR[kk][0][3]};                  \
      const uint32_t y[4] = {VR[kk][1][0], VR[kk][1][1], VR[kk][1][2], VR[kk][1][3]};                  \
      _Pragma("unroll") for (int d2 = 0; d2 < 4; ++d2) {                                                       \
        *reinterpret_cast<uint32_t*>(&sV[buf_][(tdim + 2 * d2) * kVStride + vcol(tdim, vpos(key))]) =          \
            perm(y[d2], x[d2], 0x05040100u);                                                                   \
        *reinterpret_cast<uint32_t*>(&sV[buf_][(tdim + 2 * d2 + 1) * kVStride + vcol(tdim, vpos(key))]) =      \
            perm(y[d2], x[d2], 0x07060302u);                                                                   \
      }                                                                                                        \
    }                                                                                                          \
  } while (0)

  // oacc[0..7]: O^T dims 16 dt + 4 gq + i; oacc[8]: the softmax row sums.  Tile 8 multiplies P^T by
  // a constant A with ones in rows 0, 4, 8, 12: its rows 0, 4, 8, 12 -- element 0 of every lane group
  // -- accumulate sum_k bf16(p_k) on the matrix cores instead of 32 VALU adds per tile, and the
  // lazy rescale of oacc covers them.
  f32x4 oacc[9][kNt];
#pragma unroll
  for (int dt = 0; dt < 9; ++dt)
#pragma unroll
    for (int nt = 0; nt < kNt; ++nt) oacc[dt][nt] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  const __bf16 one_or_zero = (ql & 3) == 0 ? static_cast<__bf16>(1.0f) : static_cast<__bf16>(0.0f);
  const bf16x8 ones_frag = {one_or_zero, one_or_zero, one_or_zero, one_or_zero,
                            one_or_zero, one_or_zero, one_or_zero, one_or_zero};
  float m_run[kNt];
#pragma unroll
  for (int nt = 0; nt < kNt; ++nt) m_run[nt] = -INFINITY;
  const float scale = a.scale;

  // With kAhead = 2, two register sets carry the K/V pieces of the next two tiles: tile t + 2 is
  // fetched while tile t is computed, and tile t + 1 (fetched one iteration earlier) goes to LDS
  // at its end.  With kAhead = 1 one set fetches tile t + 1 and stores it at the end of tile t.
  u32x4 kregA[kKPieces], vregA[kVPieces][2], kregB[kKPieces], vregB[kVPieces][2];
  __syncthreads();  // s_hblk ready
  load_tile(0, kregA, vregA);
  MI_STORE_TILE(0, kregA, vregA);
  if constexpr (kAhead == 2) load_tile(min(1, n_tiles - 1), kregA, vregA);
  __syncthreads();

  // kl / vl: registers tile t + 2 is fetched into; ks / vs: registers holding tile t + 1.
  auto tile_step = [&](const int t, u32x4 (&kl)[kKPieces], u32x4 (&vl)[kVPieces][2], u32x4 (&ks_)[kKPieces],
                       u32x4 (&vs_)[kVPieces][2]) {
    const int buf = t & 1;
    load_tile(min(t + kAhead, n_tiles - 1), kl, vl);  // past the end: re-reads the last tile

    // ---- S^T = K Q^T for 64 keys x 32 queries
    f32x4 sacc[4][kNt];
#pragma unroll
    for (int mt = 0; mt < 4; ++mt)
#pragma unroll
      for (int nt = 0; nt < kNt; ++nt) sacc[mt][nt] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
#pragma unroll
      for (int mt = 0; mt < 4; ++mt) {
        const bf16x8 kf = *reinterpret_cast<const bf16x8*>(&sK[buf][(mt * 16 + ql) * kKStride + ks * 32 + gq * 8]);
#pragma unroll
        for (int nt = 0; nt < kNt; ++nt)
          sacc[mt][nt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kf, qf[nt][ks], sacc[mt][nt], 0, 0, 0);
      }
    }

    // ---- scores, masks (uniform branch: only edge tiles need them)
    const bool is_hist = t < n_hist_tiles;
    const int key0 = is_hist ? t * kKTile : (c_lo + t - n_hist_tiles) * kKTile;
    bool need_mask;
    if (is_hist) {
      need_mask = key0 + kKTile > nh || qw0 < pad || qw0 + kQPerWave - 1 >= L;
    } else {
      need_mask = key0 + kKTile - 1 > qw0 || key0 < pad || qw0 < pad || qw0 + kQPerWave - 1 >= L;
    }
    // Scores rounded like the reference; log2(e) is applied inside the exp2 FMA below.
#pragma unroll
    for (int mt = 0; mt < 4; ++mt)
#pragma unroll
      for (int nt = 0; nt < kNt; ++nt) reference_scores(sacc[mt][nt], scale);
    if (__builtin_expect(__builtin_amdgcn_readfirstlane(static_cast<int>(need_mask)) != 0, 0)) {
      // Bitwise (not short-circuit) conditions keep the edge-tile path free of branches.
#pragma unroll
      for (int nt = 0; nt < kNt; ++nt) {
        const int qi = qw0 + 16 * nt + ql;
        const bool row_ok = (qi >= pad) & (qi < L);
        const int lo = is_hist ? 0 : pad;        // visible key range [lo, hi] of this query
        const int hi = is_hist ? nh - 1 : qi;
#pragma unroll
        for (int mt = 0; mt < 4; ++mt)
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const int kpos = key0 + mt * 16 + 4 * gq + i;
            const bool vis = row_ok & (kpos >= lo) & (kpos <= hi);
            sacc[mt][nt][i] = vis ? sacc[mt][nt][i] : -INFINITY;
          }
      }
    }

    // ---- online softmax per query column (lanes ql, ql+16, ql+32, ql+48 hold its 64 keys)
    // Lazy rescale: m_run (shared by the four lanes of a query column) only has to bound every
    // score to within kRescaleSlack, so each lane tests its own 16 scores and the cross-lane
    // column max is taken only on the rare tiles that raise m_run.
    constexpr float to_log2 = kLog2e;
    float mx[kNt];
#pragma unroll
    for (int nt = 0; nt < kNt; ++nt) {
      float v = -INFINITY;
#pragma unroll
      for (int mt = 0; mt < 4; ++mt)
#pragma unroll
        for (int i = 0; i < 4; ++i) v = fmaxf(v, sacc[mt][nt][i]);
      mx[nt] = v * to_log2;
    }
    bool grow = false;
#pragma unroll
    for (int nt = 0; nt < kNt; ++nt) grow = grow || mx[nt] > m_run[nt] + kRescaleSlack;
    if (__builtin_amdgcn_ballot_w64(grow) != 0) {
#pragma unroll
      for (int nt = 0; nt < kNt; ++nt) {
        mx[nt] = fmaxf(mx[nt], __shfl_xor(mx[nt], 16));
        mx[nt] = fmaxf(mx[nt], __shfl_xor(mx[nt], 32));
        const float mn = fmaxf(m_run[nt], mx[nt]);
        const float alpha = mn == -INFINITY ? 1.0f : __builtin_amdgcn_exp2f(m_run[nt] - mn);
        m_run[nt] = mn;
#pragma unroll
        for (int dt = 0; dt < 9; ++dt) oacc[dt][nt] *= alpha;
      }
    }
    bf16x8 pf[kNt][2];  // [nt][ks2]
#pragma unroll
    for (int nt = 0; nt < kNt; ++nt) {
      const float ref = m_run[nt] == -INFINITY ? 0.0f : m_run[nt];
#pragma unroll
      for (int mt = 0; mt < 4; ++mt)
#pragma unroll
        for (int i = 0; i < 4; ++i) sacc[mt][nt][i] = __builtin_amdgcn_exp2f(__builtin_fmaf(sacc[mt][nt][i], to_log2, -ref));
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
        const uint16_t* vrow = &sV[buf][(dt * 16 + ql) * kVStride];
        const bf16x8 vf = *reinterpret_cast<const bf16x8*>(vrow + vcol(dt * 16, 32 * ks2 + 8 * gq));
#pragma unroll
        for (int nt = 0; nt < kNt; ++nt)
          oacc[dt][nt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(vf, pf[nt][ks2], oacc[dt][nt], 0, 0, 0);
      }
#pragma unroll
      for (int nt = 0; nt < kNt; ++nt)
        oacc[8][nt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ones_frag, pf[nt][ks2], oacc[8][nt], 0, 0, 0);
    }

    MI_STORE_TILE(buf ^ 1, ks_, vs_);  // past the end: a buffer no later tile reads
    __syncthreads();
  };
  if constexpr (kAhead == 2) {
    for (int t = 0; t < n_tiles; t += 2) {
      tile_step(t, kregB, vregB, kregA, vregA);
      if (t + 1 < n_tiles) tile_step(t + 1, kregA, vregA, kregB, vregB);
    }
  } else {
    for (int t = 0; t < n_tiles; ++t) tile_step(t, kregA, vregA, kregA, vregA);
  }

  // ---- normalise and write: lane holds query qw0 + 16 nt + ql, dims 16 dt + 4 gq + i
#pragma unroll
  for (int nt = 0; nt < kNt; ++nt) {
    const float lt = oacc[8][nt][0];
    const float inv = lt > 0.0f ? 1.0f / lt : 0.0f;
    const int qi = qw0 + 16 * nt + ql;
    if (qi >= L || !head_live) continue;
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

namespace mi {
namespace {

// Checks shared by the entry points (sizes, head shape, strides, alignment).
int32_t check_common(const char* name, int32_t num_heads, int32_t num_kv_heads, int32_t head_dim, int32_t block_size,
                     int64_t num_blocks, std::initializer_list<int64_t> strides, std::initializer_list<const void*> tensors) {
  if (head_dim != kHeadDim || block_size != kBlockSize || num_kv_heads <= 0 || num_heads <= 0 ||
      num_heads % num_kv_heads != 0)
    return fail(MI_ERR_UNSUPPORTED,
                "%s: needs head_dim %d, block_size %d, num_heads a multiple of num_kv_heads (got head_dim %d, "
                "block_size %d, heads %d/%d)",
                name, kHeadDim, kBlockSize, head_dim, block_size, num_heads, num_kv_heads);
  if (num_kv_heads != 1 && num_kv_heads != 2 && num_kv_heads != 4 && num_kv_heads != 8)
    return fail(MI_ERR_UNSUPPORTED, "%s: num_kv_heads %d not in {1,2,4,8}", name, num_kv_heads);
  for (int64_t st : strides)
    if (st % 8 != 0) return fail(MI_ERR_UNSUPPORTED, "%s: strides must be multiples of 8", name);
  for (const void* t : tensors)
    if (t && !aligned16(t)) return fail(MI_ERR_UNSUPPORTED, "%s: tensors must be 16-byte aligned", name);
  if (num_blocks > 0x7fffffff) return fail(MI_ERR_UNSUPPORTED, "%s: pool too large", name);
  return MI_OK;
}

// Fills the row-independent fields; the caller sets the pointers and strides of its rows.
PrefillArgs rows_args(int32_t batch, int32_t padded_len, int32_t num_heads, int32_t num_kv_heads, float scale) {
  PrefillArgs a{};
  a.batch = batch;
  a.padded_len = padded_len;
  a.group = num_heads / num_kv_heads;
  a.pairs = (a.group + kGroup - 1) / kGroup;
  a.scale = scale;
  a.tiles = (padded_len + kQTile - 1) / kQTile;
  const int64_t groups = static_cast<int64_t>(a.tiles) * num_kv_heads * a.pairs * batch;
  a.groups = groups > 0x3fffffff ? -1 : static_cast<int32_t>(groups);
  return a;
}

int32_t launch_rows(const char* name, const PrefillArgs& a0, const PrefillArgs& a1, int32_t num_kv_heads,
                    int32_t max_history_blocks, void* stream) {
  if (a0.groups < 0 || a1.groups < 0 || static_cast<int64_t>(a0.groups) + a1.groups > 0x3fffffff)
    return fail(MI_ERR_UNSUPPORTED, "%s: too many workgroups", name);
  if (max_history_blocks > kMaxHistoryBlocks)
    return fail(MI_ERR_UNSUPPORTED, "%s: history of %d blocks exceeds %d", name, max_history_blocks, kMaxHistoryBlocks);
  const int groups = a0.groups + a1.groups;
  if (groups == 0) return ok();
  const size_t lds = sizeof(int) * static_cast<size_t>(max_history_blocks > 0 ? max_history_blocks : 1);
  hipStream_t s = as_stream(stream);
  switch (num_kv_heads) {
    case 1: chunked_prefill_kernel<1><<<groups, kThreads, lds, s>>>(a0, a1); break;
    case 2: chunked_prefill_kernel<2><<<groups, kThreads, lds, s>>>(a0, a1); break;
    case 4: chunked_prefill_kernel<4><<<groups, kThreads, lds, s>>>(a0, a1); break;
    default: chunked_prefill_kernel<8><<<groups, kThreads, lds, s>>>(a0, a1); break;
  }
  return check_launch(name);
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
  const char* name = "mi_chunked_prefill_attention";
  if (batch < 0 || padded_len < 0 || max_history_blocks < 0 || num_blocks < 0)
    return fail(MI_ERR_INVALID_ARGUMENT, "%s: negative size", name);
  if (batch == 0 || padded_len == 0) return ok();
  if (!out || !query || !key || !value || !start_lens || !chunk_lens ||
      (max_history_blocks > 0 && (!history_blocks || !key_pool || !value_pool)))
    return fail(MI_ERR_INVALID_ARGUMENT, "%s: null pointer argument", name);
  int32_t rc = check_common(name, num_heads, num_kv_heads, head_dim, block_size, num_blocks,
                            {out_row_stride, out_tok_stride, query_row_stride, query_head_stride, query_tok_stride,
                             key_row_stride, key_head_stride, key_tok_stride, value_row_stride, value_head_stride,
                             value_tok_stride},
                            {out, query, key, value, max_history_blocks > 0 ? key_pool : nullptr,
                             max_history_blocks > 0 ? value_pool : nullptr});
  if (rc != MI_OK) return rc;
  if (max_history_blocks > 0 && history_stride < max_history_blocks)
    return fail(MI_ERR_INVALID_ARGUMENT, "%s: history_stride < max_history_blocks", name);
  if (lens_stride <= 0) return fail(MI_ERR_INVALID_ARGUMENT, "%s: lens_stride must be > 0", name);
  if (key_tok_stride < 0 || key_tok_stride >= (1 << 24) || value_tok_stride < 0 || value_tok_stride >= (1 << 24))
    return fail(MI_ERR_UNSUPPORTED, "%s: key/value token strides must be in [0, 2^24)", name);
  if (batch > 65535) return fail(MI_ERR_UNSUPPORTED, "%s: batch > 65535", name);

  PrefillArgs a = rows_args(batch, padded_len, num_heads, num_kv_heads, scale);
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
  a.key_pool = static_cast<uint16_t*>(const_cast<void*>(key_pool));
  a.value_pool = static_cast<uint16_t*>(const_cast<void*>(value_pool));
  a.num_blocks = num_blocks;
  a.history_blocks = history_blocks;
  a.history_stride = history_stride;
  a.max_history_blocks = max_history_blocks;
  a.start_lens = start_lens;
  a.chunk_lens = chunk_lens;
  a.lens_stride = lens_stride;
  return launch_rows(name, a, PrefillArgs{}, num_kv_heads, max_history_blocks, stream);
}

extern "C" int32_t mi_mixed_paged_attention(
    void* out, int64_t out_tok_stride, const void* query, int64_t query_tok_stride, int64_t query_head_stride,
    const void* key, int64_t key_tok_stride, int64_t key_head_stride, const void* value, int64_t value_tok_stride,
    int64_t value_head_stride, void* key_pool, void* value_pool, int64_t num_blocks, int32_t prefill_rows,
    int32_t prefill_width, const int64_t* history_blocks, int64_t history_stride, int32_t max_history_blocks,
    const int64_t* start_lens, const int64_t* chunk_lens, int64_t lens_stride, int32_t decode_rows,
    const int64_t* block_tables, int64_t block_table_stride, int32_t max_blocks, const int64_t* context_lens,
    int64_t context_lens_stride, const int64_t* slot_mapping, int64_t slot_stride, int32_t num_heads,
    int32_t num_kv_heads, int32_t head_dim, int32_t block_size, float scale, void* stream) {
  using namespace mi;
  const char* name = "mi_mixed_paged_attention";
  if (prefill_rows < 0 || prefill_width < 0 || decode_rows < 0 || max_history_blocks < 0 || max_blocks < 0 ||
      num_blocks < 0)
    return fail(MI_ERR_INVALID_ARGUMENT, "%s: negative size", name);
  const bool chunks = prefill_rows > 0 && prefill_width > 0;
  if (!chunks && decode_rows == 0) return ok();
  if (!out || !query || !key || !value || (chunks && (!start_lens || !chunk_lens)) ||
      (chunks && max_history_blocks > 0 && !history_blocks) ||
      (decode_rows > 0 && (!context_lens || !slot_mapping || (max_blocks > 0 && !block_tables))) ||
      ((decode_rows > 0 || max_history_blocks > 0) && (!key_pool || !value_pool)))
    return fail(MI_ERR_INVALID_ARGUMENT, "%s: null pointer argument", name);
  const bool pools = decode_rows > 0 || max_history_blocks > 0;
  int32_t rc = check_common(name, num_heads, num_kv_heads, head_dim, block_size, num_blocks,
                            {out_tok_stride, query_tok_stride, query_head_stride, key_tok_stride, key_head_stride,
                             value_tok_stride, value_head_stride},
                            {out, query, key, value, pools ? key_pool : nullptr, pools ? value_pool : nullptr});
  if (rc != MI_OK) return rc;
  if (chunks && max_history_blocks > 0 && history_stride < max_history_blocks)
    return fail(MI_ERR_INVALID_ARGUMENT, "%s: history_stride < max_history_blocks", name);
  if (decode_rows > 0 && max_blocks > 0 && block_table_stride < max_blocks)
    return fail(MI_ERR_INVALID_ARGUMENT, "%s: block_table_stride < max_blocks", name);
  if ((chunks && lens_stride <= 0) || (decode_rows > 0 && (context_lens_stride <= 0 || slot_stride <= 0)))
    return fail(MI_ERR_INVALID_ARGUMENT, "%s: lens, context_lens and slot strides must be > 0", name);
  if (key_tok_stride < 0 || key_tok_stride >= (1 << 24) || value_tok_stride < 0 || value_tok_stride >= (1 << 24))
    return fail(MI_ERR_UNSUPPORTED, "%s: key/value token strides must be in [0, 2^24)", name);
  if (prefill_rows > 65535 || decode_rows > 65535) return fail(MI_ERR_UNSUPPORTED, "%s: more than 65535 rows", name);

  // Chunk rows: tokens [0, P L), row b at token b L.  Decode rows: tokens [P L, P L + D), one each.
  const int64_t n = chunks ? static_cast<int64_t>(prefill_rows) * prefill_width : 0;
  auto fill = [&](PrefillArgs& a, int64_t tok0, int64_t rows_tokens) {
    a.out = static_cast<uint16_t*>(out) + tok0 * out_tok_stride;
    a.out_row = rows_tokens * out_tok_stride;
    a.out_tok = out_tok_stride;
    a.query = static_cast<const uint16_t*>(query) + tok0 * query_tok_stride;
    a.q_row = rows_tokens * query_tok_stride;
    a.q_head = query_head_stride;
    a.q_tok = query_tok_stride;
    a.key = static_cast<const uint16_t*>(key) + tok0 * key_tok_stride;
    a.k_row = rows_tokens * key_tok_stride;
    a.k_head = key_head_stride;
    a.k_tok = key_tok_stride;
    a.value = static_cast<const uint16_t*>(value) + tok0 * value_tok_stride;
    a.v_row = rows_tokens * value_tok_stride;
    a.v_head = value_head_stride;
    a.v_tok = value_tok_stride;
    a.key_pool = static_cast<uint16_t*>(key_pool);
    a.value_pool = static_cast<uint16_t*>(value_pool);
    a.num_blocks = num_blocks;
  };
  PrefillArgs a0{}, a1{};
  if (chunks) {
    a0 = rows_args(prefill_rows, prefill_width, num_heads, num_kv_heads, scale);
    fill(a0, 0, prefill_width);
    a0.history_blocks = history_blocks;
    a0.history_stride = history_stride;
    a0.max_history_blocks = max_history_blocks;
    a0.start_lens = start_lens;
    a0.chunk_lens = chunk_lens;
    a0.lens_stride = lens_stride;
  }
  if (decode_rows > 0) {
    a1 = rows_args(decode_rows, 1, num_heads, num_kv_heads, scale);
    fill(a1, n, 1);
    a1.history_blocks = block_tables;
    a1.history_stride = block_table_stride;
    a1.max_history_blocks = max_blocks;
    a1.start_lens = context_lens;
    a1.chunk_lens = context_lens;
    a1.lens_stride = context_lens_stride;
    a1.decode_rows = 1;
    a1.slot_mapping = slot_mapping;
    a1.slot_stride = slot_stride;
  }
  return launch_rows(name, a0, a1, num_kv_heads,
                     std::max(chunks ? max_history_blocks : 0, decode_rows > 0 ? max_blocks : 0), stream);
}
