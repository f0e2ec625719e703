// HBM calibration kernels: what plain streaming traffic reaches on this device, the ceiling the
// data-plane kernels' rates are read against (bench.py --only copy).  Not part of the paged-KV
// C ABI: a separate library, libmi_calib.so.
//
// Traffic shapes over 16-byte non-temporal accesses, each workgroup streaming one contiguous span of
// `span` bytes with `kInFlight` pieces per lane in flight: copy (read + write), read (loads folded
// into one word per workgroup), write (stores only), and copies whose destination or source 32 KiB
// units lie at scattered places (the write pattern of the scatter, the read pattern of the gather).
// A variant is (lanes per workgroup, pieces in flight, span, store form); bench.py sweeps them and
// keeps the best of each shape.  Store forms: the non-temporal store, or the same store at device
// scope as well (nt sc1: the line goes out to memory instead of staying dirty in the XCD's L2),
// the form the gather and the KV record copies use.
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

template <bool kStream>
__device__ __forceinline__ void put(u32x4* p, const u32x4& v) {
  if constexpr (kStream) {
    // s_nop 1: the wait states a >8-byte store needs before a VALU write of its data VGPRs, which
    // the compiler cannot insert after an asm store.
    asm volatile("global_store_dwordx4 %0, %1, off nt sc1\n\ts_nop 1" ::"v"(p), "v"(v) : "memory");
  } else {
    __builtin_nontemporal_store(v, p);
  }
}

struct Variant {
  int threads;
  int in_flight;
  int64_t span;  // bytes per workgroup
  bool stream;   // device-scope non-temporal stores (nt sc1) instead of non-temporal ones
};

constexpr Variant kVariants[] = {
    {64, 2, 2 << 10, false},     {64, 4, 4 << 10, false},     {64, 8, 8 << 10, false},
    {128, 1, 2 << 10, false},    {128, 2, 4 << 10, false},    {128, 4, 8 << 10, false},
    {128, 2, 8 << 10, false},    {256, 1, 4 << 10, false},    {256, 2, 8 << 10, false},
    {512, 1, 8 << 10, false},    {256, 4, 16 << 10, false},   {512, 2, 16 << 10, false},
    {512, 2, 32 << 10, false},   {256, 4, 64 << 10, false},   {512, 4, 64 << 10, false},
    {512, 8, 128 << 10, false},  {1024, 4, 128 << 10, false}, {256, 8, 256 << 10, false},
    {512, 8, 256 << 10, false},  {1024, 8, 512 << 10, false},
    {64, 2, 2 << 10, true},      {128, 1, 2 << 10, true},     {128, 2, 4 << 10, true},
    {256, 1, 4 << 10, true},     {256, 2, 8 << 10, true},     {512, 1, 8 << 10, true},
    {512, 2, 16 << 10, true},
};
constexpr int kNumVariants = sizeof(kVariants) / sizeof(kVariants[0]);

// permute 0: span i of the source to span i of the destination.  1 and 2 move whole 32 KiB units
// (a pool block of one layer's K or V: 2^unit_shift spans): unit u goes to destination unit
// (u * 0x9E3779B1) mod n (1: destination blocks at scattered places, the scatter's writes) or comes
// from that source unit (2: the gather's reads), the spans inside a unit in order.  With n a power
// of two (checked by the host) the odd multiplier makes it a permutation, and every span is whole.
template <int kInFlight, bool kStream>
__global__ void copy_kernel(u32x4* __restrict__ dst, const u32x4* __restrict__ src, int64_t pieces,
                            int64_t span_pieces, int32_t permute, int64_t unit_mask, int32_t unit_shift) {
  const int64_t span = blockIdx.x;
  const int64_t moved = ((((span >> unit_shift) * 0x9E3779B1LL) & unit_mask) << unit_shift) |
                        (span & ((int64_t{1} << unit_shift) - 1));
  const int64_t src_base = (permute == 2 ? moved : span) * span_pieces;
  const int64_t dst_base = (permute == 1 ? moved : span) * span_pieces;
  const int64_t n = min(span_pieces, pieces - span * span_pieces);
  const int64_t step = static_cast<int64_t>(blockDim.x) * kInFlight;
  for (int64_t q0 = threadIdx.x; q0 < n; q0 += step) {
    u32x4 v[kInFlight];
#pragma unroll
    for (int k = 0; k < kInFlight; ++k) {
      const int64_t q = q0 + static_cast<int64_t>(k) * blockDim.x;
      if (q < n) v[k] = __builtin_nontemporal_load(src + src_base + q);
    }
#pragma unroll
    for (int k = 0; k < kInFlight; ++k) {
      const int64_t q = q0 + static_cast<int64_t>(k) * blockDim.x;
      if (q < n) put<kStream>(dst + dst_base + q, v[k]);
    }
  }
}

template <int kInFlight>
__global__ void read_kernel(const u32x4* __restrict__ src, uint32_t* __restrict__ sink, int64_t pieces,
                            int64_t span_pieces) {
  const int64_t base = static_cast<int64_t>(blockIdx.x) * span_pieces;
  const int64_t end = min(base + span_pieces, pieces);
  const int64_t step = static_cast<int64_t>(blockDim.x) * kInFlight;
  uint32_t acc = 0;
  for (int64_t p0 = base + threadIdx.x; p0 < end; p0 += step) {
    u32x4 v[kInFlight];
#pragma unroll
    for (int k = 0; k < kInFlight; ++k) {
      const int64_t p = p0 + static_cast<int64_t>(k) * blockDim.x;
      v[k] = p < end ? __builtin_nontemporal_load(src + p) : u32x4{0u, 0u, 0u, 0u};
    }
#pragma unroll
    for (int k = 0; k < kInFlight; ++k) acc ^= v[k][0] ^ v[k][1] ^ v[k][2] ^ v[k][3];
  }
  // One word per workgroup keeps the loads live: lane 0 always stores, and every other lane's store
  // depends on its own value, so no lane's loads are dead code.
  if (threadIdx.x == 0 || acc == 0x9e3779b9u) sink[blockIdx.x] = acc;
}

template <int kInFlight, bool kStream>
__global__ void write_kernel(u32x4* __restrict__ dst, int64_t pieces, int64_t span_pieces) {
  const int64_t base = static_cast<int64_t>(blockIdx.x) * span_pieces;
  const int64_t end = min(base + span_pieces, pieces);
  const int64_t step = static_cast<int64_t>(blockDim.x) * kInFlight;
  const u32x4 v = {static_cast<uint32_t>(blockIdx.x), 1u, 2u, 3u};
  for (int64_t p0 = base + threadIdx.x; p0 < end; p0 += step) {
#pragma unroll
    for (int k = 0; k < kInFlight; ++k) {
      const int64_t p = p0 + static_cast<int64_t>(k) * blockDim.x;
      if (p < end) put<kStream>(dst + p, v);
    }
  }
}

int check_args(int64_t bytes, int32_t variant) {
  if (bytes <= 0 || bytes % 16 != 0 || variant < 0 || variant >= kNumVariants) return -1;
  return 0;
}

}  // namespace

extern "C" int32_t calib_num_variants(void) { return kNumVariants; }

extern "C" int32_t calib_variant(int32_t variant, int32_t* threads, int32_t* in_flight, int64_t* span,
                                 int32_t* stream_stores) {
  if (variant < 0 || variant >= kNumVariants) return -1;
  *threads = kVariants[variant].threads;
  *in_flight = kVariants[variant].in_flight;
  *span = kVariants[variant].span;
  *stream_stores = kVariants[variant].stream ? 1 : 0;
  return 0;
}

// Workgroups a launch of `bytes` takes (the read kernel's sink needs one word each).
extern "C" int64_t calib_groups(int64_t bytes, int32_t variant) {
  if (check_args(bytes, variant)) return -1;
  return (bytes + kVariants[variant].span - 1) / kVariants[variant].span;
}

// shape: 0 = copy (dst <- src), 1 = read (src, sink of calib_groups words), 2 = write (dst),
// 3 = copy to destination 32 KiB units at scattered places, 4 = copy from source 32 KiB units at
// scattered places (3 and 4 need spans of at most 32 KiB and a power-of-two number of whole units).
extern "C" int32_t calib_stream(int32_t shape, void* dst, const void* src, void* sink, int64_t bytes,
                                int32_t variant, void* stream) {
  if (check_args(bytes, variant) || shape < 0 || shape > 4) return -1;
  if ((shape != 1 && !dst) || (shape != 2 && !src) || (shape == 1 && !sink)) return -1;
  const bool copies = shape == 0 || shape >= 3;
  if ((reinterpret_cast<uintptr_t>(dst) | reinterpret_cast<uintptr_t>(src)) & 15u) return -1;
  const Variant v = kVariants[variant];
  const int64_t pieces = bytes / 16, span_pieces = v.span / 16;
  const int64_t groups = (pieces + span_pieces - 1) / span_pieces;
  if (groups > 0x7fffffff) return -1;
  constexpr int64_t kUnitBytes = 32 << 10;
  int32_t unit_shift = 0;
  int64_t unit_mask = 0;
  if (shape >= 3) {
    if (v.span > kUnitBytes || kUnitBytes % v.span != 0 || bytes % kUnitBytes != 0) return -1;
    const int64_t units = bytes / kUnitBytes;
    if ((units & (units - 1)) != 0) return -1;
    while ((int64_t{1} << unit_shift) * v.span < kUnitBytes) ++unit_shift;
    unit_mask = units - 1;
  }
  const int32_t permute = shape == 3 ? 1 : (shape == 4 ? 2 : 0);
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  const dim3 grid(static_cast<uint32_t>(groups));
  u32x4* d = static_cast<u32x4*>(dst);
  const u32x4* r = static_cast<const u32x4*>(src);
  uint32_t* k = static_cast<uint32_t*>(sink);
#define CALIB_LAUNCH(N)                                                                                 \
  if (copies && v.stream)                                                                         \
    copy_kernel<N, true><<<grid, v.threads, 0, s>>>(d, r, pieces, span_pieces, permute, unit_mask, unit_shift);  \
  else if (copies)                                                                                \
    copy_kernel<N, false><<<grid, v.threads, 0, s>>>(d, r, pieces, span_pieces, permute, unit_mask, unit_shift); \
  else if (shape == 1) read_kernel<N><<<grid, v.threads, 0, s>>>(r, k, pieces, span_pieces);             \
  else if (v.stream) write_kernel<N, true><<<grid, v.threads, 0, s>>>(d, pieces, span_pieces);           \
  else write_kernel<N, false><<<grid, v.threads, 0, s>>>(d, pieces, span_pieces);
  switch (v.in_flight) {
    case 1: CALIB_LAUNCH(1) break;
    case 2: CALIB_LAUNCH(2) break;
    case 4: CALIB_LAUNCH(4) break;
    default: CALIB_LAUNCH(8) break;
  }
#undef CALIB_LAUNCH
  return hipGetLastError() == hipSuccess ? 0 : -4;
}
