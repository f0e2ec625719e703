// Greedy sampling: the index of the largest logit of each row.
//
// The reference samples with torch.argmax over the last position's logits
// (src/mini_infra/worker/sampler.py:9-23); over Qwen3's 151,936-entry vocabulary that is one
// generic two-value ATen reduction per decode step.  This kernel gives the same answer in one
// pass over each row:
//   * ties go to the smallest index (the first occurrence);
//   * -0 and +0 compare equal;
//   * a NaN counts as larger than every number, and the first NaN of a row wins;
//   * a row of -inf returns index 0.
//
// One workgroup of 1024 lanes per row.  Each lane walks its 16-byte pieces (8 bf16 logits) in
// increasing index order, so a strict "greater than" keeps the first occurrence, and the lanes'
// winners are combined as 64-bit keys (ordered value << 32 | ~index) under an unsigned max.
// The row is read once (304 KB for the vocabulary above); a decode batch of B rows is B
// workgroups.

#include "mi_common.h"

namespace mi {
namespace {

constexpr int kArgmaxThreads = 1024;  // 16 wavefronts
constexpr int kArgmaxUnroll = 4;      // 16-byte pieces in flight per lane

struct ArgmaxArgs {
  int64_t* out;
  const uint16_t* logits;
  int64_t rows;
  int64_t row_stride;  // elements
  int32_t cols;
};

// Lane-local running winner.  best starts at -inf with idx at the lane's first index, so a lane
// whose values are all -inf reports its first one.  take = !(v <= best) && best is not NaN:
// a number greater than best, or the first NaN; nothing replaces a NaN.
struct Winner {
  float best;
  int32_t idx;
  __device__ __forceinline__ void see(float v, int32_t i) {
    const bool take = !(v <= best) && best == best;
    best = take ? v : best;
    idx = take ? i : idx;
  }
};

// Unsigned key that orders like the float comparison above: NaN above +inf, -0 equal to +0.
// Lanes that saw no element return 0, below every real key.
__device__ __forceinline__ uint64_t winner_key(const Winner& w, bool valid) {
  const uint32_t bits = __float_as_uint(w.best);
  uint32_t key;
  if (w.best != w.best) {
    key = 0xffffffffu;
  } else if ((bits << 1) == 0) {
    key = 0x80000000u;
  } else {
    key = (bits & 0x80000000u) ? ~bits : (bits | 0x80000000u);
  }
  const uint64_t packed = (static_cast<uint64_t>(key) << 32) | (0xffffffffu - static_cast<uint32_t>(w.idx));
  return valid ? packed : 0;
}

__device__ __forceinline__ uint64_t key_max(uint64_t a, uint64_t b) { return a > b ? a : b; }

template <bool kVec>
__global__ __launch_bounds__(kArgmaxThreads) void argmax_rows_kernel(const ArgmaxArgs a) {
  const int64_t row = blockIdx.x;
  const uint16_t* src = a.logits + row * a.row_stride;
  const int tid = threadIdx.x;
  Winner w{-__builtin_inff(), 0};
  bool valid;
  if constexpr (kVec) {
    const int pieces = a.cols >> 3;
    const u32x4* vsrc = reinterpret_cast<const u32x4*>(src);
    valid = tid < pieces;
    w.idx = 8 * tid;
    for (int p0 = tid; p0 < pieces; p0 += kArgmaxUnroll * kArgmaxThreads) {
      u32x4 v[kArgmaxUnroll];
#pragma unroll
      for (int j = 0; j < kArgmaxUnroll; ++j) {
        const int p = p0 + j * kArgmaxThreads;
        // -inf pairs past the end are never taken.
        v[j] = p < pieces ? vsrc[p] : u32x4{0xff80ff80u, 0xff80ff80u, 0xff80ff80u, 0xff80ff80u};
      }
#pragma unroll
      for (int j = 0; j < kArgmaxUnroll; ++j) {
        const int base = 8 * (p0 + j * kArgmaxThreads);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          w.see(bf16_lo(v[j][e]), base + 2 * e);
          w.see(bf16_hi(v[j][e]), base + 2 * e + 1);
        }
      }
    }
    // The cols % 8 tail: its indices exceed every piece's, so each lane still sees them last.
    const int t = 8 * pieces + tid;
    if (tid < (a.cols & 7)) {
      if (!valid) w.idx = t;
      valid = true;
      w.see(__uint_as_float(static_cast<uint32_t>(src[t]) << 16), t);
    }
  } else {
    valid = tid < a.cols;
    w.idx = tid;
    for (int i = tid; i < a.cols; i += kArgmaxThreads) w.see(__uint_as_float(static_cast<uint32_t>(src[i]) << 16), i);
  }

  uint64_t key = winner_key(w, valid);
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) key = key_max(key, __shfl_xor(key, m, 64));
  __shared__ uint64_t s_key[kArgmaxThreads / 64];
  if ((tid & 63) == 0) s_key[tid >> 6] = key;
  __syncthreads();
  if (tid < 64) {
    key = tid < kArgmaxThreads / 64 ? s_key[tid] : 0;
#pragma unroll
    for (int m = 8; m >= 1; m >>= 1) key = key_max(key, __shfl_xor(key, m, 64));
    if (tid == 0) a.out[row] = static_cast<int64_t>(0xffffffffu - static_cast<uint32_t>(key));
  }
}

}  // namespace
}  // namespace mi

extern "C" int32_t mi_argmax_rows(int64_t* out, const void* logits, int64_t rows, int32_t cols, int64_t row_stride,
                                  void* stream) {
  using namespace mi;
  if (rows < 0 || cols <= 0 || row_stride < cols) return fail(MI_ERR_INVALID_ARGUMENT, "mi_argmax_rows: bad size");
  if (rows == 0) return ok();
  if (!out || !logits) return fail(MI_ERR_INVALID_ARGUMENT, "mi_argmax_rows: null pointer argument");
  if (rows > 0x7fffffff) return fail(MI_ERR_UNSUPPORTED, "mi_argmax_rows: too many rows");
  ArgmaxArgs a{out, static_cast<const uint16_t*>(logits), rows, row_stride, cols};
  const dim3 grid(static_cast<uint32_t>(rows));
  if (aligned16(logits) && row_stride % 8 == 0)
    argmax_rows_kernel<true><<<grid, kArgmaxThreads, 0, as_stream(stream)>>>(a);
  else
    argmax_rows_kernel<false><<<grid, kArgmaxThreads, 0, as_stream(stream)>>>(a);
  return check_launch("mi_argmax_rows");
}
