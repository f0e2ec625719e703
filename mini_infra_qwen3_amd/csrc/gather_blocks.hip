// Kernel 2: block-table gather of whole physical blocks.
//
// Behaviour of PagedKVCachePool.gather_blocks (src/mini_infra/worker/paged_kv_cache.py:54-72):
// per layer `key_pool[block_ids]` materialised as `[batch, nb, block_size, H, D]`, for K and V of
// every layer in one launch.  A block of one layer is contiguous in the pool (32 KiB for
// 16 x 8 x 128 bf16) and contiguous in the output, so eight workgroups of 128 lanes stream one
// block, a contiguous 4 KiB eighth each, with 16-byte pieces: lane i moves bytes [16 i, 16 i + 16)
// of each 2 KiB stripe, both stripes in flight, loads issued before the stores.  Measured on
// MI355X (the history gather of 4 prompts x 16384 tokens in 2048-token chunks, three repetitions in one process, against the read + write
// copy ceiling of the same process, 6.44-6.54 TB/s): 6.47-6.53 TB/s (99-100%), against 6.25-6.31
// for four 8 KiB workgroups of 256 lanes x 2, 6.29-6.34 for eight of 256 lanes x 1, 6.25-6.31 for
// four of 512 x 1, 6.00-6.01 for sixteen 2 KiB workgroups of 128 x 1; earlier, 5.68-6.01 for one
// 32 KiB workgroup per block (512 lanes x 2) and 5.49-5.69 for 256 lanes x 8.
#include "mi_common.h"

namespace mi {
namespace {

#ifndef MI_GATHER_UNROLL
#define MI_GATHER_UNROLL 2
#endif
#ifndef MI_GATHER_NT
#define MI_GATHER_NT 1
#endif

#ifndef MI_GATHER_THREADS
#define MI_GATHER_THREADS 128
#endif
#ifndef MI_GATHER_SPLIT
#define MI_GATHER_SPLIT 8
#endif
constexpr int kSplit = MI_GATHER_SPLIT;  // workgroups per block: each copies a contiguous 1 / kSplit
constexpr int kThreads = MI_GATHER_THREADS;
constexpr int kUnroll = MI_GATHER_UNROLL;
constexpr bool kNt = MI_GATHER_NT != 0;  // non-temporal pool loads and output stores

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
};

// grid: x = (row * nb + j) * kSplit + part (part of one gathered block), y = layer, z = 0 for K / 1
// for V.
template <typename V>
__global__ __launch_bounds__(kThreads) void gather_blocks_kernel(const GatherArgs a) {
  const uint32_t flat = blockIdx.x / kSplit;
  const uint32_t part = blockIdx.x - flat * kSplit;
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
    dim3 grid(static_cast<uint32_t>(batch) * num_gathered_blocks * kSplit, nl, 2);
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
