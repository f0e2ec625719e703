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
//  * Dispatch order: the query tiles of one (row, head pair) stay on one XCD (shared L2), and each
//    XCD's queue runs in rounds of as many whole pairs as its CUs hold, heaviest query tiles first
//    inside a round, so the causal chunk's light and heavy tiles pair up on every CU.
//  * KV tiles of 64 keys: history tiles first (pool blocks through the block table -- the
//    gather is fused, nothing is materialised), then chunk tiles up to the causal limit.
//    K and V tiles go from memory straight into double-buffered LDS (global_load_lds_dwordx4, no
//    registers on the way), row-major with 256-byte rows whose 16-byte chunks are XOR-swizzled by
//    the row; tile t + 1 is in flight while tile t is multiplied.
//  * S^T = K Q^T: A = K rows from LDS, B = Q^T from registers (loaded once), C lane layout =
//    (query = lane % 16, keys 4 (lane / 16) + i).  Each query's softmax state lives in the
//    lanes of its column; the row max needs two cross-lane steps, the row sum is deferred.
//  * O^T = V^T P^T: the probabilities of a 32-key step are already in the B-operand lanes if
//    the MFMA's k index is read as key 16 (k' / 4) + 4 (lane / 16) + k' % 4.  The A operand (V^T)
//    comes from the row-major V tile by two transposing reads (ds_read_b64_tr_b16), 4 keys each.
//  * Softmax and accumulation are fp32 with lazy rescaling of the running max as in the decode
//    kernel.  Scores keep the reference's bf16 rounding points (bf16 product, then bf16 product
//    with the scale), one packed bf16 convert per rounding: for N(0,1) inputs those roundings
//    move logits by ~1e-2, so dropping them would leave the 2e-2 parity band.
//  * The two waves of a SIMD run in step (one workgroup barrier per tile), so per tile the
//    matrix work, the score roundings, exponentials and converts, and the LDS operand latency
//    largely add up.
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
constexpr int kKTile = 64;                 // keys per KV tile
constexpr int kThreads = 64 * kGroup * kWavesPerHead;    // one workgroup per CU at 4 waves per head
constexpr int kSpans = kKTile / 4;                       // 1 KiB LDS spans (4 rows of 256 B) per K or V tile
static_assert(kSpans % (kThreads / 64) == 0, "every wave moves the same number of spans");
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
  int32_t round_pairs;  // (row, head pair) units per dispatch round of one workgroup queue
  // Decode rows (a mixed step's single new tokens, padded_len 1): start_lens holds each row's
  // context length including its token, so the history is the context minus one and a row with
  // context 0 is padding; the token's K/V row is appended to pool slot slot_mapping[b] (skipped
  // when outside the pool) by the workgroup of the first head pair of each KV head.
  int32_t decode_rows;
  const int64_t* slot_mapping;
  int64_t slot_stride;
  // Ragged chunk rows (a mixed step's chunks packed back to back): when set, the len_b real tokens
  // of row b are flat tokens row_first[b] .. row_first[b] + len_b - 1 of query / key / value / out
  // (the token strides apply, the row strides are unused; row_first[b] is clamped to
  // [0, row_tokens - len_b]), and padding positions are neither read nor written.
  const int64_t* row_first;
  int64_t row_tokens;
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

// One 16-byte-per-lane load straight into LDS: lane i writes bytes [16 i, 16 i + 16) of the
// 1 KiB span at LDS address lds (wave-uniform, passed in M0; one wait state between the M0 write
// and the load).  Issued by inline assembly: the compiler's own form ties every later LDS read to
// the completion of all such loads (it cannot tell the two tile buffers apart), which would wait
// for tile t + 1 before reading tile t.  The compiler does not see these loads, so the kernel waits
// for them itself (vmcnt(0) before each tile barrier).  The LDS address goes in through an M0
// operand constraint, so the compiler writes M0 itself and knows its value across the asm.
__device__ __forceinline__ void dma16(const void* gptr, uint32_t lds) {
  asm volatile("s_nop 0\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(gptr), "{m0}"(lds) : "memory");
}

// One launch serves up to two sets of rows (a mixed step's chunk rows and its decode rows): the
// first a0.groups workgroups take a0, the rest a1.
template <int kKvHeads>
__global__ __launch_bounds__(kThreads, kWavesPerSimd) void chunked_prefill_kernel(const PrefillArgs a0,
                                                                                   const PrefillArgs a1) {
  // K and V tiles row-major, 256-byte rows, 16-byte chunk c of row r stored at chunk c ^ (r % 16).
  __shared__ __align__(1024) uint16_t sK[2][kKTile * kHeadDim];
  __shared__ __align__(1024) uint16_t sV[2][kKTile * kHeadDim];
  extern __shared__ int s_hblk[];  // [ceil(nh / 16)] history block ids of this row (dynamic LDS)

  const bool second = static_cast<int>(blockIdx.x) >= a0.groups;  // uniform
  const PrefillArgs a = second ? a1 : a0;

  // Workgroup -> (row b, head pair hp, query tile qt).  Consecutive workgroup ids go round-robin to
  // the kXcds XCDs, each with its own L2, and each XCD starts its ids in order on whichever CU
  // frees first.  When the pair count is a multiple of kXcds, id L runs on XCD L % kXcds and takes
  // place L / kXcds in the queue of that XCD's own pairs, so the query tiles of one (row, head
  // pair) -- which stream the same K/V tiles -- share an L2; otherwise one queue holds every pair.
  // A queue is cut into rounds of round_pairs pairs (as many as its CUs hold with all their query
  // tiles at once), and inside a round the tiles go heaviest (latest) first, pair by pair: the CUs
  // that finish a round's light tiles first take the next round's heavy ones, so every CU ends up
  // with about the same number of key tiles under the causal mask.
  int b, hp, qt;
  {
    const int tiles = a.tiles;
    const int per_row = kKvHeads * a.pairs;
    const int pairs = per_row * a.batch;
    const int lin = static_cast<int>(blockIdx.x) - (second ? a0.groups : 0);
    const bool by_xcd = pairs % kXcds == 0;
    const int units = by_xcd ? pairs / kXcds : pairs;  // pairs in this queue
    const int slot = by_xcd ? lin / kXcds : lin;       // place in this queue
    const int round_idx = slot / (a.round_pairs * tiles);
    const int within = slot - round_idx * a.round_pairs * tiles;
    const int round_size = min(a.round_pairs, units - round_idx * a.round_pairs);
    const int rank = within / round_size;
    const int unit = round_idx * a.round_pairs + (within - rank * round_size);
    const int pair = by_xcd ? unit * kXcds + lin % kXcds : unit;
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
  // Element offset of padded position rpad of row b (its first stored token): position i >= rpad
  // of a tensor with row / token strides (r, t) is at base + (i - rpad) t.
  const bool ragged = a.row_first != nullptr;  // uniform
  if (ragged && len64 == 0) return;             // an empty ragged row stores nothing
  int64_t first = 0;
  if (ragged) {
    first = a.row_first[b];
    first = first < 0 ? 0 : (first > a.row_tokens - len64 ? a.row_tokens - len64 : first);
  }
  const int rpad = ragged ? pad : 0;
  const int64_t q_base = ragged ? first * a.q_tok : b * a.q_row;
  const int64_t k_base = ragged ? first * a.k_tok : b * a.k_row;
  const int64_t v_base = ragged ? first * a.v_tok : b * a.v_row;
  const int64_t o_base = ragged ? first * a.out_tok : b * a.out_row;
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

  uint16_t* out_b = a.out + o_base;  // padded position rpad
  if (q0 + kQTile <= pad) {  // the whole tile is padding: zero rows (a ragged row stores none)
    if (ragged) return;
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
      if (qi < L && qi >= rpad)
        v = *reinterpret_cast<const uint4*>(a.query + q_base + h * a.q_head + (qi - rpad) * a.q_tok + ks * 32 + gq * 8);
      qf[nt][ks] = __builtin_bit_cast(bf16x8, v);
    }
  }

  const int n_hist_tiles = (nh + kKTile - 1) / kKTile;
  const int c_lo = pad / kKTile;
  const int last_q = min(q0 + kQTile, L) - 1;
  const int c_hi = last_q / kKTile;
  const int n_tiles = n_hist_tiles + (c_hi - c_lo + 1);

  // ---- tile loads straight into LDS (global_load_lds_dwordx4: lane i of an instruction writes
  // bytes [16 i, 16 i + 16) of a 1 KiB LDS span).  A tile is kSpans such spans of 4 rows for K and
  // as many for V; wave w moves spans [kSpansPerWave w, kSpansPerWave (w + 1)) of each.  Lane i of
  // span m fetches row 4 m + i / 16, global chunk (i % 16) ^ (row % 16), so that the chunk lands at
  // its swizzled place: the 16 lanes of an MFMA operand read (16 rows, one logical chunk) then hit
  // 16 different chunk positions, i.e. all banks.  In a history tile a wave's spans lie in one pool
  // block, whose id comes from the history table the workgroup staged in LDS; the id for tile t + 1
  // is read while tile t - 1 is computed, so no tile waits for that read.  Chunk rows past L - 1
  // read row L - 1, and a ragged row's padding rows its first stored row (their keys are masked).
  const int nhb = (nh + kBlockSize - 1) / kBlockSize;
  for (int i = tid; i < nhb; i += kThreads) {
    const int64_t x = a.history_blocks[b * a.history_stride + i];
    s_hblk[i] = (x < 0 || x >= a.num_blocks) ? 0 : static_cast<int>(x);
  }
  constexpr int64_t kBlkElems = static_cast<int64_t>(kBlockSize) * kKvHeads * kHeadDim;
  constexpr int kSpansPerWave = kSpans / (kThreads / 64);
  const int drow = lane >> 4;
  const int dchunk = lane & 15;
  const uint16_t* k_rows = a.key + k_base + g * a.k_head;  // padded position rpad
  const uint16_t* v_rows = a.value + v_base + g * a.v_head;
  const uint32_t k_tok = static_cast<uint32_t>(a.k_tok);  // < 2^24, checked by the entry point
  const uint32_t v_tok = static_cast<uint32_t>(a.v_tok);
  typedef __attribute__((address_space(3))) void* lds_ptr_t;
  static_assert(kBlockSize % (4 * kSpansPerWave) == 0, "a wave's spans of a tile must lie in one pool block");
  const int wave_blk = 4 * kSpansPerWave * w / kBlockSize;  // pool block of this wave's rows within a tile
  const auto hist_slot = [&](const int t) { return min(t * (kKTile / kBlockSize) + wave_blk, max(nhb - 1, 0)); };
  // LDS byte addresses of this wave's first K and V span in buffer 0 (buffer 1 follows at + kTileBytes).
  constexpr uint32_t kTileBytes = kKTile * kHeadDim * sizeof(uint16_t);
  const uint32_t k_lds0 = static_cast<uint32_t>(reinterpret_cast<uintptr_t>((lds_ptr_t)(&sK[0][kSpansPerWave * w * 512])));
  const uint32_t v_lds0 = static_cast<uint32_t>(reinterpret_cast<uintptr_t>((lds_ptr_t)(&sV[0][kSpansPerWave * w * 512])));

  // hblk: this wave's history block id for tile t (unused for chunk tiles).
  auto dma_tile = [&](const int t, const int buf, const int hblk) {
    const bool hist = t < n_hist_tiles;
    const int key0 = (c_lo + t - n_hist_tiles) * kKTile;
#pragma unroll
    for (int i = 0; i < kSpansPerWave; ++i) {
      const int m = kSpansPerWave * w + i;
      const int r = 4 * m + drow;
      const uint32_t c8 = static_cast<uint32_t>((dchunk ^ (r & 15)) * 8);
      const uint16_t* ksrc;
      const uint16_t* vsrc;
      if (hist) {
        const int64_t blk = __builtin_amdgcn_readfirstlane(hblk);
        const uint32_t off = static_cast<uint32_t>(((r & 15) * kKvHeads + g) * kHeadDim) + c8;
        ksrc = a.key_pool + blk * kBlkElems + off;
        vsrc = a.value_pool + blk * kBlkElems + off;
      } else {
        const uint32_t kc = static_cast<uint32_t>(min(max(key0 + r, rpad), L - 1) - rpad);
        ksrc = k_rows + (__umul24(kc, k_tok) + c8);
        vsrc = v_rows + (__umul24(kc, v_tok) + c8);
      }
      dma16(ksrc, __builtin_amdgcn_readfirstlane(k_lds0 + buf * kTileBytes + i * 1024));
      dma16(vsrc, __builtin_amdgcn_readfirstlane(v_lds0 + buf * kTileBytes + i * 1024));
    }
  };
  // Per-lane LDS byte offsets of the MFMA operands.  K (A of S^T = K Q^T): row 16 mt + ql, global
  // chunk 4 ks + gq.  V (A of O^T = V^T P^T, by transposing 8-byte reads): lane L of a 16-lane group
  // addresses row k0 + L / 4, dims 16 dt + 4 (L % 4) .. + 3, and receives dim 16 dt + L of rows
  // k0 .. k0 + 3; k0 = 32 ks2 + 4 gq, then + 16, gives the 8 keys in the MFMA's k order.
  uint32_t k_off[4];
#pragma unroll
  for (int ks = 0; ks < 4; ++ks) k_off[ks] = ql * 256 + (((4 * ks + gq) ^ ql) & 15) * 16;
  const int vr = 4 * gq + (ql >> 2);
  uint32_t v_off[8];
#pragma unroll
  for (int dt = 0; dt < 8; ++dt) v_off[dt] = vr * 256 + (((2 * dt + ((ql >> 1) & 1)) ^ vr) & 15) * 16 + (ql & 1) * 8;

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

  // Tile t + 1 moves into the other buffer while tile t is computed; each wave waits for its own
  // loads before the tile barrier, after which every wave's part is in place.
  __syncthreads();  // s_hblk ready
  dma_tile(0, 0, s_hblk[hist_slot(0)]);
  int hblk_next = s_hblk[hist_slot(1)];
  // s_waitcnt vmcnt(0) (expcnt and lgkmcnt unconstrained) as a real instruction, so that the
  // compiler also counts the Q fragment loads as complete and waits for nothing inside the loop.
  __builtin_amdgcn_s_waitcnt(0x0F70);
  __syncthreads();

  auto tile_step = [&](const int t, const int buf) {
    if (t + 1 < n_tiles) dma_tile(t + 1, buf ^ 1, hblk_next);
    hblk_next = s_hblk[hist_slot(t + 2)];
    const char* sKb = reinterpret_cast<const char*>(sK[buf]);
    const char* sVb = reinterpret_cast<const char*>(sV[buf]);

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
        const bf16x8 kf = *reinterpret_cast<const bf16x8*>(sKb + mt * 4096 + k_off[ks]);
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
        typedef short s16x4 __attribute__((ext_vector_type(4)));
        typedef __attribute__((address_space(3))) s16x4* lds_s16x4;
        const s16x4 v0 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4)(sVb + 32 * ks2 * 256 + v_off[dt]));
        const s16x4 v1 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4)(sVb + (32 * ks2 + 16) * 256 + v_off[dt]));
        const bf16x8 vf = __builtin_bit_cast(bf16x8, __builtin_shufflevector(v0, v1, 0, 1, 2, 3, 4, 5, 6, 7));
#pragma unroll
        for (int nt = 0; nt < kNt; ++nt)
          oacc[dt][nt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(vf, pf[nt][ks2], oacc[dt][nt], 0, 0, 0);
      }
#pragma unroll
      for (int nt = 0; nt < kNt; ++nt)
        oacc[8][nt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ones_frag, pf[nt][ks2], oacc[8][nt], 0, 0, 0);
    }

    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
  };
  for (int t = 0; t < n_tiles; t += 2) {
    tile_step(t, 0);
    if (t + 1 < n_tiles) tile_step(t + 1, 1);
  }

  // ---- normalise and write: lane holds query qw0 + 16 nt + ql, dims 16 dt + 4 gq + i
#pragma unroll
  for (int nt = 0; nt < kNt; ++nt) {
    const float lt = oacc[8][nt][0];
    const float inv = lt > 0.0f ? 1.0f / lt : 0.0f;
    const int qi = qw0 + 16 * nt + ql;
    if (qi >= L || qi < rpad || !head_live) continue;
    uint16_t* orow = out_b + (qi - rpad) * a.out_tok + h * kHeadDim + 4 * gq;
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
  const int64_t pairs = static_cast<int64_t>(num_kv_heads) * a.pairs * batch;
  const int64_t groups = a.tiles * pairs;
  a.groups = groups > 0x3fffffff ? -1 : static_cast<int32_t>(groups);
  // Dispatch rounds: the queue of one XCD (or of the whole device when the pairs do not split
  // evenly over the XCDs) holds its CUs' worth of whole pairs per round.
  const bool by_xcd = pairs % kXcds == 0;
  const int64_t units = by_xcd ? pairs / kXcds : pairs;
  const int64_t cus = by_xcd ? device_cus() / kXcds : device_cus();
  const int64_t per_round = std::min(a.tiles > 0 ? cus / a.tiles : int64_t{1}, units);
  a.round_pairs = static_cast<int32_t>(std::max(per_round, int64_t{1}));
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

// One workgroup per token t of [0, row_tokens): every thread checks its share of the rows, and the
// workgroup writes a zero row unless one of them covers t.
constexpr int kZeroThreads = 256;
__global__ __launch_bounds__(kZeroThreads) void zero_uncovered_kernel(uint16_t* out, int64_t out_tok, int32_t row_elems,
                                                                       const int64_t* first, const int64_t* lens,
                                                                       int64_t lens_stride, int32_t rows, int32_t width,
                                                                       int64_t row_tokens, int32_t vec) {
  const int64_t t = blockIdx.x;
  int covered = 0;
  for (int b = threadIdx.x; b < rows; b += kZeroThreads) {
    int64_t len = lens[b * lens_stride];
    len = len < 0 ? 0 : (len > width ? width : len);
    int64_t f = first[b];
    f = f < 0 ? 0 : (f > row_tokens - len ? row_tokens - len : f);
    covered |= t >= f && t < f + len;
  }
  if (__syncthreads_or(covered)) return;
  uint16_t* row = out + t * out_tok;
  if (vec) {
    for (int i = threadIdx.x; i < row_elems / 8; i += kZeroThreads) reinterpret_cast<uint4*>(row)[i] = uint4{0, 0, 0, 0};
  } else {
    for (int i = threadIdx.x; i < row_elems; i += kZeroThreads) row[i] = 0;
  }
}

}  // namespace

int32_t zero_uncovered_tokens(const char* what, void* out, int64_t out_tok_stride, int32_t row_elems,
                              const int64_t* first, const int64_t* lens, int64_t lens_stride, int32_t rows,
                              int32_t width, int64_t row_tokens, void* stream) {
  if (row_tokens <= 0) return MI_OK;
  if (row_tokens > 0x7fffffff) return fail(MI_ERR_UNSUPPORTED, "%s: more than 2^31 - 1 chunk tokens", what);
  const int32_t vec = aligned16(out) && out_tok_stride % 8 == 0 && row_elems % 8 == 0;
  zero_uncovered_kernel<<<static_cast<unsigned>(row_tokens), kZeroThreads, 0, as_stream(stream)>>>(
      static_cast<uint16_t*>(out), out_tok_stride, row_elems, first, lens, lens_stride, rows, width, row_tokens, vec);
  return check_launch(what);
}

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
  if (const int32_t rc = reject_empty_pool(name, num_blocks, max_history_blocks > 0)) return rc;
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
    int32_t prefill_width, int64_t chunk_tokens, const int64_t* chunk_first, const int64_t* history_blocks,
    int64_t history_stride, int32_t max_history_blocks, const int64_t* start_lens, const int64_t* chunk_lens,
    int64_t lens_stride, int32_t decode_rows, const int64_t* block_tables, int64_t block_table_stride,
    int32_t max_blocks, const int64_t* context_lens, int64_t context_lens_stride, const int64_t* slot_mapping,
    int64_t slot_stride, int32_t num_heads, int32_t num_kv_heads, int32_t head_dim, int32_t block_size, float scale,
    void* stream) {
  using namespace mi;
  const char* name = "mi_mixed_paged_attention";
  if (prefill_rows < 0 || prefill_width < 0 || decode_rows < 0 || max_history_blocks < 0 || max_blocks < 0 ||
      num_blocks < 0 || (chunk_first && chunk_tokens < 0))
    return fail(MI_ERR_INVALID_ARGUMENT, "%s: negative size", name);
  const bool chunks = prefill_rows > 0 && prefill_width > 0;
  const bool ragged = chunk_first && chunk_tokens > 0;  // writes a zero row for every uncovered token
  if (!chunks && decode_rows == 0 && !ragged) return ok();
  if (const int32_t rc = reject_empty_pool(name, num_blocks, (chunks && max_history_blocks > 0) ||
                                                                 (decode_rows > 0 && max_blocks > 0)))
    return rc;
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

  // Chunk rows: tokens [0, P L), row b at token b L, or with chunk_first the ragged rows of tokens
  // [0, chunk_tokens).  Decode rows: the D tokens after them, one each.
  const int64_t n = chunk_first ? chunk_tokens : (chunks ? static_cast<int64_t>(prefill_rows) * prefill_width : 0);
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
    a0.row_first = chunk_first;
    a0.row_tokens = chunk_tokens;
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
  if (ragged) {
    rc = zero_uncovered_tokens(name, out, out_tok_stride, num_heads * head_dim, chunk_first, chunk_lens, lens_stride,
                               chunks ? prefill_rows : 0, prefill_width, chunk_tokens, stream);
    if (rc != MI_OK) return rc;
  }
  return launch_rows(name, a0, a1, num_kv_heads,
                     std::max(chunks ? max_history_blocks : 0, decode_rows > 0 ? max_blocks : 0), stream);
}
