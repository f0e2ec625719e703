// Kernel 2: block-table gather of whole physical blocks.
//
// Behaviour of PagedKVCachePool.gather_blocks (src/mini_infra/worker/paged_kv_cache.py:54-72):
// per layer `key_pool[block_ids]` materialised as `[batch, nb, block_size, H, D]`, for K and V of
// every layer in one launch.  A block of one layer is contiguous in the pool (32 KiB for
// 16 x 8 x 128 bf16) and contiguous in the output, so eight workgroups of 256 lanes stream one
// block, a contiguous 4 KiB eighth each, with 16-byte pieces: lane i moves bytes [16 i, 16 i + 16)
// of the eighth, one piece per lane.
//
// XCD runs.  Workgroups are dealt round-robin to the 8 XCDs, so in launch order the eight parts of
// one block would be read by eight XCDs.  The kernel maps blockIdx so that each XCD takes kXcdRun
// consecutive parts (sixteen whole blocks at 128).
//
// Measured on MI355X (the history gather of 4 prompts x 16384 tokens in 2048-token chunks, 28
// layers, 20 timed launches, three repetitions in one process; read + write copy ceiling of the
// same process 6.58-6.66 TB/s, copy from 32 KiB units at scattered places 6.31-6.38):
//   form (lanes x pieces in flight, parts per block, XCD run)   fragmented tables   near-sequential
//   256 x 1, 8 parts, runs of 128                               6.52-6.56 TB/s      6.79-6.81
//   256 x 1, 8 parts, runs of 32 / 64                           6.50-6.55 / 6.46-6.48   6.61-6.66 / 6.73-6.76
//   128 x 2, 8 parts, no runs (the earlier form)                6.16-6.37           6.54-6.62
//   128 x 2, 8 parts, runs of 32 / 64 / 128                     6.32-6.45 / 6.44-6.47 / 6.43-6.51   6.63-6.68
//   128 x 2 and 128 x 1, 16 parts, runs of 64                   6.47-6.57           6.58-6.65
// Runs of 8 or 16 parts are slower than none (5.74-6.13 TB/s).  Without runs, earlier: four 8 KiB
// workgroups of 256 lanes x 2 6.25-6.31 TB/s, sixteen 2 KiB workgroups of 128 x 1 6.00-6.01, one
// 32 KiB workgroup per block 5.68-6.01.
#include "mi_common.h"

namespace mi {
namespace {

#ifndef MI_GATHER_UNROLL
#define MI_GATHER_UNROLL 1
#endif
#ifndef MI_GATHER_NT
#define MI_GATHER_NT 1
#endif

#ifndef MI_GATHER_THREADS
#define MI_GATHER_THREADS 256
#endif
#ifndef MI_GATHER_SPLIT
#define MI_GATHER_SPLIT 8
#endif
constexpr int kSplit = MI_GATHER_SPLIT;  // workgroups per block: each copies a contiguous 1 / kSplit
constexpr int kThreads = MI_GATHER_THREADS;
constexpr int kUnroll = MI_GATHER_UNROLL;
constexpr bool kNt = MI_GATHER_NT != 0;  // non-temporal pool loads and output stores
#ifndef MI_GATHER_XCD_RUN
#define MI_GATHER_XCD_RUN 128
#endif
constexpr int kXcdRun = MI_GATHER_XCD_RUN;  // consecutive parts per XCD run (0: round-robin order)

struct GatherArgs {
  const char* key_pool[kMaxLayersPerLaunch];
  const char* value_pool[kMaxLayersPerLaunch];
  char* key_out[kMaxLayersPerLaunch];
  char* value_out[kMaxLayersPerLaunch];
  const int64_t* block_ids;
  int64_t block_id_stride;
  int64_t num_blocks;
  int64_t block_bytes;
  uint32_t nb;            // gathered blocks per row
  uint32_t pieces;        // block_bytes / sizeof(V)
  uint32_t parts;         // workgroups along x: rows * nb * kSplit
};

// grid: x = (row * nb + j) * kSplit + part (part of one gathered block), y = layer, z = 0 for K / 1
// for V.
template <typename V>
__global__ __launch_bounds__(kThreads) void gather_blocks_kernel(const GatherArgs a) {
  uint32_t x = blockIdx.x;
  if (kXcdRun > 0) {
    // Workgroups go round-robin to the XCDs: within each super-run of kXcds * kXcdRun parts, the
    // workgroups on XCD i take parts [i kXcdRun, (i + 1) kXcdRun) in order; the tail keeps identity.
    constexpr uint32_t kSuper = static_cast<uint32_t>(kXcds) * kXcdRun;
    if (x < a.parts / kSuper * kSuper) {
      const uint32_t base = x / kSuper * kSuper, r = x - base;
      x = base + (r % kXcds) * kXcdRun + r / kXcds;
    }
  }
  const uint32_t flat = x / kSplit;
  const uint32_t part = x - flat * kSplit;
  const uint32_t row = flat / a.nb;
  const uint32_t j = flat - row * a.nb;
  const int layer = blockIdx.y;
  const bool is_value = blockIdx.z != 0;
  const int64_t bid = a.block_ids[static_cast<int64_t>(row) * a.block_id_stride + j];
  const bool valid = bid >= 0 && bid < a.num_blocks;
  const V* src = reinterpret_cast<const V*>((is_value ? a.value_pool[layer] : a.key_pool[layer]) +
                                            (valid ? bid : 0) * a.block_bytes);
  V* dst = reinterpret_cast<V*>((is_value ? a.value_out[layer] : a.key_out[layer]) +
                                static_cast<int64_t>(flat) * a.block_bytes);

  const uint32_t per_part = (a.pieces + kSplit - 1) / kSplit;
  const uint32_t p0 = part * per_part;
  const uint32_t p1 = min(a.pieces, p0 + per_part);
  for (uint32_t base = p0; base < p1; base += kThreads * kUnroll) {
    V val[kUnroll];
#pragma unroll
    for (int k = 0; k < kUnroll; ++k) {
      const uint32_t p = base + k * kThreads + threadIdx.x;
      if (p < p1) val[k] = load_vec<kNt>(src + p);
    }
#pragma unroll
    for (int k = 0; k < kUnroll; ++k) {
      const uint32_t p = base + k * kThreads + threadIdx.x;
      if (p < p1) store_stream<kNt>(dst + p, val[k]);
    }
  }
}

}  // namespace
}  // namespace mi

extern "C" int32_t mi_gather_blocks(const void* const* key_pools, const void* const* value_pools, int64_t num_blocks,
                                    const int64_t* block_ids, int64_t block_id_stride, int32_t batch,
                                    int32_t num_gathered_blocks, void* const* key_out, void* const* value_out,
                                    int32_t num_layers, int64_t block_bytes, void* stream) {
  using namespace mi;
  if (batch < 0 || num_gathered_blocks < 0 || num_layers < 0 || num_blocks < 0 || block_bytes < 0)
    return fail(MI_ERR_INVALID_ARGUMENT, "mi_gather_blocks: negative size");
  if (batch == 0 || num_gathered_blocks == 0 || num_layers == 0 || block_bytes == 0) return ok();
  if (const int32_t rc = reject_empty_pool("mi_gather_blocks", num_blocks, true)) return rc;
  if (!key_pools || !value_pools || !key_out || !value_out || !block_ids)
    return fail(MI_ERR_INVALID_ARGUMENT, "mi_gather_blocks: null pointer argument");
  if (block_id_stride < num_gathered_blocks)
    return fail(MI_ERR_INVALID_ARGUMENT, "mi_gather_blocks: block_id_stride %lld < num_gathered_blocks %d",
                static_cast<long long>(block_id_stride), num_gathered_blocks);
  if (static_cast<int64_t>(batch) * num_gathered_blocks * kSplit > 0x7fffffff)
    return fail(MI_ERR_UNSUPPORTED, "mi_gather_blocks: too many blocks in one call");

  GatherArgs a{};
  a.block_ids = block_ids;
  a.block_id_stride = block_id_stride;
  a.num_blocks = num_blocks;
  a.block_bytes = block_bytes;
  a.nb = static_cast<uint32_t>(num_gathered_blocks);

  bool wide = block_bytes % 16 == 0;
  for (int l = 0; l < num_layers && wide; ++l)
    wide = aligned16(key_pools[l]) && aligned16(value_pools[l]) && aligned16(key_out[l]) && aligned16(value_out[l]);
  const int64_t piece = wide ? 16 : (block_bytes % 4 == 0 ? 4 : 2);
  if (block_bytes % piece != 0 || block_bytes / piece > 0x7fffffff)
    return fail(MI_ERR_UNSUPPORTED, "mi_gather_blocks: block of %lld bytes not supported",
                static_cast<long long>(block_bytes));
  a.pieces = static_cast<uint32_t>(block_bytes / piece);

  hipStream_t s = as_stream(stream);
  for (int l0 = 0; l0 < num_layers; l0 += kMaxLayersPerLaunch) {
    const int nl = num_layers - l0 < kMaxLayersPerLaunch ? num_layers - l0 : kMaxLayersPerLaunch;
    for (int l = 0; l < nl; ++l) {
      if (!key_pools[l0 + l] || !value_pools[l0 + l] || !key_out[l0 + l] || !value_out[l0 + l])
        return fail(MI_ERR_INVALID_ARGUMENT, "mi_gather_blocks: null pointer for layer %d", l0 + l);
      a.key_pool[l] = static_cast<const char*>(key_pools[l0 + l]);
      a.value_pool[l] = static_cast<const char*>(value_pools[l0 + l]);
      a.key_out[l] = static_cast<char*>(key_out[l0 + l]);
      a.value_out[l] = static_cast<char*>(value_out[l0 + l]);
    }
    a.parts = static_cast<uint32_t>(batch) * num_gathered_blocks * kSplit;
    dim3 grid(a.parts, nl, 2);
    if (piece == 16)
      gather_blocks_kernel<u32x4><<<grid, kThreads, 0, s>>>(a);
    else if (piece == 4)
      gather_blocks_kernel<uint32_t><<<grid, kThreads, 0, s>>>(a);
    else
      gather_blocks_kernel<uint16_t><<<grid, kThreads, 0, s>>>(a);
    int32_t rc = check_launch("mi_gather_blocks");
    if (rc != MI_OK) return rc;
  }
  return ok();
}
