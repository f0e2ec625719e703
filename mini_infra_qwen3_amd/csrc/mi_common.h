// Shared helpers for the paged-KV data plane kernels (gfx950 / CDNA4).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/mi_paged.h"

namespace mi {

// ---------------------------------------------------------------- errors ---
// Records a printf-style message for mi_last_error() on this thread and
// returns `code`, so call sites can write `return fail(MI_ERR_..., "...")`.
int32_t fail(int32_t code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
// Clears the thread's last error and returns MI_OK.
int32_t ok();
// Checks hipGetLastError() after a launch; MI_ERR_DEVICE with the HIP message.
int32_t check_launch(const char* what);

// Zeroes the out rows of the tokens of [0, row_tokens) that no ragged chunk row of a mixed step
// covers (row b covers tokens first[b] .. first[b] + len_b - 1, with len_b = lens[b lens_stride]
// clamped to [0, width] and first[b] to [0, row_tokens - len_b], as the attention kernels clamp
// them); row_elems bf16 values per token, token stride out_tok_stride.  One launch on `stream`.
int32_t zero_uncovered_tokens(const char* what, void* out, int64_t out_tok_stride, int32_t row_elems,
                              const int64_t* first, const int64_t* lens, int64_t lens_stride, int32_t rows,
                              int32_t width, int64_t row_tokens, void* stream);

// 16-byte vector used by the streaming copies (a native vector type, so the
// non-temporal builtins accept it).
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// Loads / stores of data touched once per launch (pool rows, copies), optionally with the
// non-temporal hint so the stream does not displace reused lines in L2 and the Infinity
// Cache.  Each kernel picks kNt from its own tunable.
template <bool kNt, typename T>
__device__ __forceinline__ T load_vec(const T* p) {
  if constexpr (kNt) {
    return __builtin_nontemporal_load(p);
  } else {
    return *p;
  }
}
template <bool kNt, typename T>
__device__ __forceinline__ void store_vec(T* p, const T& v) {
  if constexpr (kNt) {
    __builtin_nontemporal_store(v, p);
  } else {
    *p = v;
  }
}

// 16-byte store of data this launch writes once and never reads back: non-temporal and at device
// scope (sc1), so the line goes out to memory rather than staying dirty in the XCD's L2.  On MI355X
// a 2 GiB copy streams 6.69-6.71 TB/s with these stores against 6.48-6.50 with non-temporal ones;
// the gather and the KV record copies gain 2-3%, while the scatter's 2 KiB rows at random slots
// lose 2% and keep store_vec.  Other vector types take store_vec.
// A VMEM store of more than 8 bytes needs a wait state before a VALU instruction may overwrite its
// data VGPRs.  The compiler inserts it after the stores it emits, but it cannot see into this asm,
// so the asm carries its own (s_nop 1: two wait states); without it, register reuse right after the
// store can send the new values.
template <bool kNt, typename T>
__device__ __forceinline__ void store_stream(T* p, const T& v) {
  if constexpr (kNt && __is_same(T, u32x4)) {
    asm volatile("global_store_dwordx4 %0, %1, off nt sc1\n\ts_nop 1" ::"v"(p), "v"(v) : "memory");
  } else {
    store_vec<kNt>(p, v);
  }
}

inline hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

// An out-of-range block id reads the null block 0, which an empty pool does not have: a call that
// would read any block of a pool with no blocks is an invalid argument, rejected before launch.
inline int32_t reject_empty_pool(const char* what, int64_t num_blocks, bool reads_blocks) {
  if (num_blocks == 0 && reads_blocks)
    return fail(MI_ERR_INVALID_ARGUMENT, "%s: the pool has no blocks to read", what);
  return MI_OK;
}

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// Compute units of the current device (256 on MI355X), read once per device; 256 when the
// attribute cannot be read.
inline int device_cus() {
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

// Workgroups are handed out round-robin to this many XCDs (accelerator complex dies), each with
// its own L2: consecutive workgroup ids land on different XCDs.
constexpr int kXcds = 8;

// At most this many layers go into one launch (pointer tables travel in the
// kernel argument segment); callers with more layers are split into chunks.
constexpr int kMaxLayersPerLaunch = 32;

// ---------------------------------------------------------------- bf16 -----
// bf16 -> fp32 is exact: the bf16 bits are the high half of the fp32 word.
__device__ __forceinline__ float bf16_lo(uint32_t pair) { return __uint_as_float(pair << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t pair) { return __uint_as_float(pair & 0xffff0000u); }

// fp32 -> bf16 with round-to-nearest-even (NaN kept quiet): add 0x7fff plus the
// lowest kept bit, then truncate -- the standard bit-level RNE construction.
__device__ __forceinline__ uint32_t f32_to_bf16_bits(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (u >> 16) | 0x40u;
  u += 0x7fffu + ((u >> 16) & 1u);
  return u >> 16;
}
__device__ __forceinline__ float round_bf16(float f) { return __uint_as_float(f32_to_bf16_bits(f) << 16); }
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  return f32_to_bf16_bits(lo) | (f32_to_bf16_bits(hi) << 16);
}
__device__ __forceinline__ float bf16_bits_to_f32(uint16_t b) { return __uint_as_float(static_cast<uint32_t>(b) << 16); }

// Cross-lane steps without LDS permutes: a 16-lane DPP butterfly within each row (xor 1, xor 2,
// 8-lane mirror, 16-lane mirror; on the two halves of a double), then v_permlane16_swap /
// v_permlane32_swap across rows (a swap returns the lane's own value and its partner's, so their
// sum is x + x[lane ^ 16] or x + x[lane ^ 32] in every lane).  Every lane of the wavefront must be
// active.  The sums met here are exact (or, for the remainders of the exact kernels' split sums,
// far below what the roundings see), so the order gives the bits of any other.
template <int kCtrl>
__device__ __forceinline__ double dpp_f64(double x) {
  const uint64_t u = __double_as_longlong(x);
  const uint32_t lo = static_cast<uint32_t>(
      __builtin_amdgcn_update_dpp(0, static_cast<int>(static_cast<uint32_t>(u)), kCtrl, 0xf, 0xf, false));
  const uint32_t hi = static_cast<uint32_t>(
      __builtin_amdgcn_update_dpp(0, static_cast<int>(static_cast<uint32_t>(u >> 32)), kCtrl, 0xf, 0xf, false));
  return __longlong_as_double(static_cast<long long>((static_cast<uint64_t>(hi) << 32) | lo));
}
template <int kCtrl>
__device__ __forceinline__ float dpp_f32(float x) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), kCtrl, 0xf, 0xf, false));
}
__device__ __forceinline__ double join_f64(uint32_t hi, uint32_t lo) {
  return __longlong_as_double(static_cast<long long>((static_cast<uint64_t>(hi) << 32) | lo));
}
__device__ __forceinline__ double dpp_sum16_f64(double x) {
  x += dpp_f64<0xB1>(x);   // quad_perm [1,0,3,2]
  x += dpp_f64<0x4E>(x);   // quad_perm [2,3,0,1]
  x += dpp_f64<0x141>(x);  // row_half_mirror
  x += dpp_f64<0x140>(x);  // row_mirror
  return x;
}
__device__ __forceinline__ double xsum16_f64(double x) {  // x + x[lane ^ 16]
  const uint64_t u = __double_as_longlong(x);
  const auto lo = __builtin_amdgcn_permlane16_swap(static_cast<uint32_t>(u), static_cast<uint32_t>(u), false, false);
  const auto hi =
      __builtin_amdgcn_permlane16_swap(static_cast<uint32_t>(u >> 32), static_cast<uint32_t>(u >> 32), false, false);
  return join_f64(hi[0], lo[0]) + join_f64(hi[1], lo[1]);
}
__device__ __forceinline__ double xsum32_f64(double x) {  // x + x[lane ^ 32]
  const uint64_t u = __double_as_longlong(x);
  const auto lo = __builtin_amdgcn_permlane32_swap(static_cast<uint32_t>(u), static_cast<uint32_t>(u), false, false);
  const auto hi =
      __builtin_amdgcn_permlane32_swap(static_cast<uint32_t>(u >> 32), static_cast<uint32_t>(u >> 32), false, false);
  return join_f64(hi[0], lo[0]) + join_f64(hi[1], lo[1]);
}
__device__ __forceinline__ float xmax16(float x) {
  const auto p = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(p[0]), __uint_as_float(p[1]));
}
__device__ __forceinline__ float xmax32(float x) {
  const auto p = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(p[0]), __uint_as_float(p[1]));
}

// ------------------------------------------------------- RMSNorm, exact ---
// The reference's RMSNorm (src/mini_infra/model/qwen3.py:67-78) is
//   h = x.float(); y = w * (h * rsqrt(h.pow(2).mean(-1) + eps)).to(bf16)
// whose fp32 mean depends on the order ATen sums the squares in.  Here the sum is exact (the
// square of a bf16 value has at most 16 significant bits, so fp64 adds them without loss unless
// the terms span more than 2^37), and so is the reciprocal square root:
//   var = fp32(sum(h^2) / N),  t = fp32(var + eps),  r = fp32(1 / sqrt_f64(t))
// (sqrt and division correctly rounded in fp64, then one rounding to fp32) -- a result that does
// not depend on the reduction order or the device, which torch's on-device chain also gives
// whenever its fp32 sum rounds the same way.
__device__ __forceinline__ double wave_sum64_f64(double v) { return xsum32_f64(xsum16_f64(dpp_sum16_f64(v))); }

// r = fp32(1 / sqrt(fp32(fp32(sum_sq / n) + eps))), the division by n in fp64.
__device__ __forceinline__ float rms_inv(double sum_sq, double n, float eps) {
  const float var = static_cast<float>(sum_sq / n);
  const float t = var + eps;
  return static_cast<float>(1.0 / sqrt(static_cast<double>(t)));
}

// ------------------------------------------------------- q/k norm + RoPE ---
// Per-head RMSNorm + RoPE of one 128-wide q or k head by one wavefront, with the reference's bf16
// rounding points (src/mini_infra/model/qwen3.py:67-78 on the head, then _apply_rotary_embedding
// :111-145): n = bf16(x * r) with r the exact reciprocal RMS above, y = bf16(w * n),
// out = bf16(bf16(y * cos) + bf16(rotate_half(y) * sin)).  Lane l owns elements l and l + 64, the
// pair rotate_half couples, so the rotation is lane-local; o0 / o1 are elements l / l + 64 (exact
// bf16 values held in fp32).
__device__ __forceinline__ void norm_rope_head(const uint16_t* src, const uint16_t* weight, const uint16_t* cos,
                                               const uint16_t* sin, float eps, int lane, float& o0, float& o1) {
  const float x0 = bf16_bits_to_f32(src[lane]), x1 = bf16_bits_to_f32(src[lane + 64]);
  const double sq = static_cast<double>(x0) * x0 + static_cast<double>(x1) * x1;
  const float r = rms_inv(wave_sum64_f64(sq), 128.0, eps);
  const float y0 = round_bf16(bf16_bits_to_f32(weight[lane]) * round_bf16(x0 * r));
  const float y1 = round_bf16(bf16_bits_to_f32(weight[lane + 64]) * round_bf16(x1 * r));
  // element l:      y*cos - y[l+64]*sin ; element l+64: y*cos + y[l]*sin  (rotate_half = cat(-y2, y1))
  o0 = round_bf16(round_bf16(y0 * bf16_bits_to_f32(cos[lane])) + round_bf16(-y1 * bf16_bits_to_f32(sin[lane])));
  o1 = round_bf16(round_bf16(y1 * bf16_bits_to_f32(cos[lane + 64])) + round_bf16(y0 * bf16_bits_to_f32(sin[lane + 64])));
}

}  // namespace mi
