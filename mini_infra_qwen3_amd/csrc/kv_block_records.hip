// KV block records: the wire / swap format of whole physical blocks.
//
// The reference plans a "swap" preemption mode that moves a victim's physical KV blocks to a CPU
// host swap pool over PCIe and back on resume (src/mini_infra/core/types.py:110-114,
// src/mini_infra/core/scheduler.py:312-313); its pool keeps each layer's K and V as
// [num_blocks, block_size, H, D] (src/mini_infra/worker/paged_kv_cache.py:23-52), so one block's
// data is 2 x num_layers pieces scattered over the pool.
//
// A record is one physical block, every layer, contiguous:
//   record[layer][0 = K, 1 = V][block_size][H][D]      (record_bytes = 2 * num_layers * block_bytes)
// n records are n * record_bytes contiguous bytes, so a swap is one DMA copy and a file is a
// header plus the records.  mi_pack_blocks gathers blocks into records and mi_unpack_blocks
// scatters records into (other) blocks; both are bit-exact copies.
//
// grid (one dimension): x = ((record * layers + layer) * 2 + K / V) * kSplit + part, so consecutive
// workgroups walk a record's bytes in order.  kSplit workgroups share one block_bytes piece (32 KiB
// for 16 x 8 x 128 bf16), a contiguous 1 / kSplit each, with 16-byte loads issued before the
// stores.  Measured on 2048 random blocks of the 28-layer pool (2 x 3.76 GB per launch), three
// repetitions in one process: 8 workgroups of 256 lanes x 1 piece 6.14-6.22 TB/s pack, 5.69-5.70
// unpack; 8 x 128 x 2 6.03-6.08 / 5.60-5.63; 4 x 256 x 2 5.84-5.87 / 5.51-5.54; with the
// (record; layer; K / V) grid instead, one 1024 x 2 workgroup per piece 5.39-5.42 / 5.28-5.29 and
// 8 x 256 x 1 5.44-5.45 / 5.41-5.43.  Non-temporal accesses measured faster than plain ones.
#include "mi_common.h"

namespace mi {
namespace {

#ifndef MI_RECORDS_THREADS
#define MI_RECORDS_THREADS 256
#endif
#ifndef MI_RECORDS_UNROLL
#define MI_RECORDS_UNROLL 1
#endif
#ifndef MI_RECORDS_NT_LOAD
#define MI_RECORDS_NT_LOAD 1
#endif
#ifndef MI_RECORDS_NT_STORE
#define MI_RECORDS_NT_STORE 1
#endif
#ifndef MI_RECORDS_SPLIT
#define MI_RECORDS_SPLIT 8
#endif

constexpr int kThreads = MI_RECORDS_THREADS;
constexpr int kUnroll = MI_RECORDS_UNROLL;
constexpr int kSplit = MI_RECORDS_SPLIT;  // workgroups per block piece, each a contiguous 1 / kSplit
constexpr bool kNtLoad = MI_RECORDS_NT_LOAD != 0;    // non-temporal loads of the source
constexpr bool kNtStore = MI_RECORDS_NT_STORE != 0;  // non-temporal stores of the destination
#ifndef MI_RECORDS_XCD_RUN_PACK
#define MI_RECORDS_XCD_RUN_PACK 64
#endif
#ifndef MI_RECORDS_XCD_RUN_UNPACK
#define MI_RECORDS_XCD_RUN_UNPACK 0
#endif
// Consecutive workgroups per XCD run (0: round-robin launch order): within each super-run of
// kXcds * run workgroups, those on XCD i take [i run, (i + 1) run) in order.  Measured on MI355X
// (2048 records of the Qwen3-0.6B pool, two repetitions): pack 6.27-6.33 TB/s without runs,
// 6.23-6.28 at 16, 6.43 at 32, 6.41-6.46 at 64, 6.42-6.43 at 128 and 256; unpack 5.79 without,
// 5.52-5.76 with runs of 16-256.
constexpr int kXcdRunPack = MI_RECORDS_XCD_RUN_PACK;
constexpr int kXcdRunUnpack = MI_RECORDS_XCD_RUN_UNPACK;

struct RecordArgs {
  char* pool[2][kMaxLayersPerLaunch];  // [0] = key pools, [1] = value pools of this launch's layers
  char* records;
  const int64_t* block_ids;
  int64_t num_blocks;
  int64_t block_bytes;
  int64_t record_bytes;
  int32_t layer0;   // first layer of this launch
  int32_t layers;   // layers of this launch
  uint32_t pieces;  // block_bytes / sizeof(V)
  uint32_t groups;  // workgroups of this launch
};

// kPack: block -> record (an out-of-range block id reads the null block 0, as every read does).
// !kPack: record -> block (an out-of-range block id is skipped, as every write is).
template <typename V, bool kPack>
__global__ __launch_bounds__(kThreads) void kv_records_kernel(const RecordArgs a) {
  constexpr int kXcdRun = kPack ? kXcdRunPack : kXcdRunUnpack;
  uint32_t x = blockIdx.x;
  if (kXcdRun > 0) {
    constexpr uint32_t kSuper = static_cast<uint32_t>(kXcds) * kXcdRun;
    if (x < a.groups / kSuper * kSuper) {
      const uint32_t base = x / kSuper * kSuper, r = x - base;
      x = base + (r % kXcds) * kXcdRun + r / kXcds;
    }
  }
  const uint32_t part = x % kSplit;
  const uint32_t piece_id = x / kSplit;
  const int kv = piece_id & 1;
  const int layer = (piece_id >> 1) % a.layers;
  const int64_t i = (piece_id >> 1) / a.layers;
  const int64_t bid = a.block_ids[i];
  const bool valid = bid >= 0 && bid < a.num_blocks;
  if (!kPack && !valid) return;
  V* block = reinterpret_cast<V*>(a.pool[kv][layer] + (valid ? bid : 0) * a.block_bytes);
  V* rec = reinterpret_cast<V*>(a.records + i * a.record_bytes + (2 * (a.layer0 + layer) + kv) * a.block_bytes);
  const V* src = kPack ? block : rec;
  V* dst = kPack ? rec : block;
  const uint32_t per_part = (a.pieces + kSplit - 1) / kSplit;
  const uint32_t p0 = part * per_part;
  const uint32_t p1 = min(a.pieces, p0 + per_part);
  for (uint32_t base = p0; base < p1; base += kThreads * kUnroll) {
    V val[kUnroll];
#pragma unroll
    for (int k = 0; k < kUnroll; ++k) {
      const uint32_t p = base + k * kThreads + threadIdx.x;
      if (p < p1) val[k] = load_vec<kNtLoad>(src + p);
    }
#pragma unroll
    for (int k = 0; k < kUnroll; ++k) {
      const uint32_t p = base + k * kThreads + threadIdx.x;
      if (p < p1) store_stream<kNtStore>(dst + p, val[k]);
    }
  }
}

template <bool kPack>
int32_t launch_records(const char* what, void* records, const void* const* key_pools,
                       const void* const* value_pools, int64_t num_blocks, const int64_t* block_ids,
                       int64_t num_records, int32_t num_layers, int64_t block_bytes, void* stream) {
  if (num_records < 0 || num_layers < 0 || num_blocks < 0 || block_bytes < 0)
    return fail(MI_ERR_INVALID_ARGUMENT, "%s: negative size", what);
  if (num_records == 0 || num_layers == 0 || block_bytes == 0) return ok();
  if (const int32_t rc = reject_empty_pool(what, num_blocks, kPack)) return rc;
  if (!records || !key_pools || !value_pools || !block_ids)
    return fail(MI_ERR_INVALID_ARGUMENT, "%s: null pointer argument", what);
  if (num_records * kSplit * 2 * kMaxLayersPerLaunch > 0x7fffffff)
    return fail(MI_ERR_UNSUPPORTED, "%s: too many records in one call", what);
  const int64_t record_bytes = 2 * static_cast<int64_t>(num_layers) * block_bytes;

  bool wide = block_bytes % 16 == 0 && aligned16(records);
  for (int l = 0; l < num_layers && wide; ++l) wide = aligned16(key_pools[l]) && aligned16(value_pools[l]);
  const int64_t piece = wide ? 16 : (block_bytes % 4 == 0 ? 4 : 2);
  if (block_bytes % piece != 0 || block_bytes / piece > 0x7fffffff)
    return fail(MI_ERR_UNSUPPORTED, "%s: block of %lld bytes not supported", what,
                static_cast<long long>(block_bytes));

  RecordArgs a{};
  a.records = static_cast<char*>(records);
  a.block_ids = block_ids;
  a.num_blocks = num_blocks;
  a.block_bytes = block_bytes;
  a.record_bytes = record_bytes;
  a.pieces = static_cast<uint32_t>(block_bytes / piece);
  hipStream_t s = as_stream(stream);
  for (int l0 = 0; l0 < num_layers; l0 += kMaxLayersPerLaunch) {
    const int nl = num_layers - l0 < kMaxLayersPerLaunch ? num_layers - l0 : kMaxLayersPerLaunch;
    for (int l = 0; l < nl; ++l) {
      if (!key_pools[l0 + l] || !value_pools[l0 + l])
        return fail(MI_ERR_INVALID_ARGUMENT, "%s: null pointer for layer %d", what, l0 + l);
      a.pool[0][l] = const_cast<char*>(static_cast<const char*>(key_pools[l0 + l]));
      a.pool[1][l] = const_cast<char*>(static_cast<const char*>(value_pools[l0 + l]));
    }
    a.layer0 = l0;
    a.layers = nl;
    a.groups = static_cast<uint32_t>(num_records * nl * 2 * kSplit);
    const dim3 grid(a.groups, 1, 1);
    if (piece == 16)
      kv_records_kernel<u32x4, kPack><<<grid, kThreads, 0, s>>>(a);
    else if (piece == 4)
      kv_records_kernel<uint32_t, kPack><<<grid, kThreads, 0, s>>>(a);
    else
      kv_records_kernel<uint16_t, kPack><<<grid, kThreads, 0, s>>>(a);
    const int32_t rc = check_launch(what);
    if (rc != MI_OK) return rc;
  }
  return ok();
}

}  // namespace
}  // namespace mi

extern "C" int32_t mi_pack_blocks(void* records, const void* const* key_pools, const void* const* value_pools,
                                  int64_t num_blocks, const int64_t* block_ids, int64_t num_records,
                                  int32_t num_layers, int64_t block_bytes, void* stream) {
  return mi::launch_records<true>("mi_pack_blocks", records, key_pools, value_pools, num_blocks, block_ids,
                                  num_records, num_layers, block_bytes, stream);
}

extern "C" int32_t mi_unpack_blocks(void* const* key_pools, void* const* value_pools, int64_t num_blocks,
                                    const void* records, const int64_t* block_ids, int64_t num_records,
                                    int32_t num_layers, int64_t block_bytes, void* stream) {
  return mi::launch_records<false>("mi_unpack_blocks", const_cast<void*>(records),
                                   const_cast<const void* const*>(key_pools),
                                   const_cast<const void* const*>(value_pools), num_blocks, block_ids, num_records,
                                   num_layers, block_bytes, stream);
}
