// Shared helpers of the r2splat HIP library (gfx950, wave64).
//
// Host side: status codes, the per-thread error message, launch checking and
// a bump allocator that carves caller-provided workspace.  Device side:
// wave-level primitives used by the binning sort, the compaction scan and
// the reductions.
#pragma once

#include <type_traits>

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "r2splat_hip.h"

namespace r2s {

// ---------------------------------------------------------------- host ----

void set_error(const char *fmt, ...) __attribute__((format(printf, 1, 2)));
void clear_error();

// Returns R2S_OK, or R2S_EHIP with the message set, after a launch sequence.
int check_launch(const char *what);

inline hipStream_t as_stream(r2s_stream_t s) { return reinterpret_cast<hipStream_t>(s); }

#define R2S_REQUIRE(cond, ...)            \
  do {                                    \
    if (!(cond)) {                        \
      ::r2s::set_error(__VA_ARGS__);      \
      return R2S_EINVAL;                  \
    }                                     \
  } while (0)

#define R2S_RETURN_IF(...)                \
  do {                                    \
    int _st = (__VA_ARGS__);              \
    if (_st != R2S_OK) return _st;        \
  } while (0)

constexpr int64_t kInt32Max = 2147483647LL;

inline int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }
inline size_t align_up(size_t v, size_t a) { return (v + a - 1) / a * a; }

// Carves 256-byte aligned sub-buffers out of a caller-provided workspace.
// `base == nullptr` measures only (used by the *_workspace_bytes queries).
struct Carver {
  char *base;
  size_t used = 0;
  explicit Carver(void *b) : base(static_cast<char *>(b)) {}
  template <typename T>
  T *take(int64_t count) {
    size_t off = align_up(used, 256);
    used = off + static_cast<size_t>(count > 0 ? count : 0) * sizeof(T);
    return base ? reinterpret_cast<T *>(base + off) : nullptr;
  }
};

// Block-id swizzle so that consecutive logical tiles land on the same XCD.
// Hardware dispatches workgroup b to XCD (b % 8); logical id L is mapped to
// a contiguous range per XCD.  A bijection on [0, n).
__device__ __forceinline__ uint32_t xcd_swizzle(uint32_t b, uint32_t n) {
  constexpr uint32_t kXcd = 8;
  const uint32_t q = n / kXcd, r = n % kXcd;
  const uint32_t x = b % kXcd, k = b / kXcd;
  return (x < r) ? x * (q + 1) + k : r * (q + 1) + (x - r) * q + k;
}

// ------------------------------------------------------------- device ----

__device__ __forceinline__ uint32_t lane_id() { return __lane_id(); }

// Mask of lanes strictly below the calling lane.
__device__ __forceinline__ uint64_t lanemask_lt() {
  const uint32_t l = __lane_id();
  return (l == 0) ? 0ull : ((~0ull) >> (64u - l));
}

// Number of set bits of `mask` below the calling lane (v_mbcnt pair).
__device__ __forceinline__ uint32_t mbcnt(uint64_t mask) {
  uint32_t lo = __builtin_amdgcn_mbcnt_lo(static_cast<uint32_t>(mask), 0u);
  return __builtin_amdgcn_mbcnt_hi(static_cast<uint32_t>(mask >> 32), lo);
}

__device__ __forceinline__ uint64_t ballot(bool p) { return __ballot(p); }

// Index of the calling wave in its workgroup, as a wave-uniform (scalar) value.
__device__ __forceinline__ uint32_t wave_index() {
  return static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6)));
}

// Value of `v` in lane `src` (src must be wave-uniform).
__device__ __forceinline__ uint32_t readlane_u32(uint32_t v, uint32_t src) {
  return static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(v), static_cast<int>(src)));
}
__device__ __forceinline__ int64_t readlane_i64(int64_t v, uint32_t src) {
  uint32_t lo = readlane_u32(static_cast<uint32_t>(v), src);
  uint32_t hi = readlane_u32(static_cast<uint32_t>(static_cast<uint64_t>(v) >> 32), src);
  return static_cast<int64_t>((static_cast<uint64_t>(hi) << 32) | lo);
}

// One DPP lane move of a 32- or 64-bit value (the halves moved
// separately): lanes the move does not write (no source lane in the row, or
// a row outside kRowMask) read `fill`.
template <int kCtrl, int kRowMask, typename T>
__device__ __forceinline__ T dpp_take(T v, T fill = T(0)) {
  static_assert(sizeof(T) == 4 || sizeof(T) == 8, "32- or 64-bit values");
  if constexpr (sizeof(T) == 4) {
    const int x = __builtin_bit_cast(int, v), f = __builtin_bit_cast(int, fill);
    return __builtin_bit_cast(T, __builtin_amdgcn_update_dpp(f, x, kCtrl, kRowMask, 0xf, false));
  } else {
    const uint64_t u = __builtin_bit_cast(uint64_t, v), uf = __builtin_bit_cast(uint64_t, fill);
    const int lo = __builtin_amdgcn_update_dpp(static_cast<int>(static_cast<uint32_t>(uf)),
                                               static_cast<int>(static_cast<uint32_t>(u)), kCtrl,
                                               kRowMask, 0xf, false);
    const int hi = __builtin_amdgcn_update_dpp(static_cast<int>(static_cast<uint32_t>(uf >> 32)),
                                               static_cast<int>(static_cast<uint32_t>(u >> 32)),
                                               kCtrl, kRowMask, 0xf, false);
    return __builtin_bit_cast(T, (static_cast<uint64_t>(static_cast<uint32_t>(hi)) << 32) |
                                     static_cast<uint32_t>(lo));
  }
}

// Wave64 inclusive prefix sum of an integer, all lanes active: DPP row
// shifts by 1, 2, 4, 8 within each row of 16 lanes (Hillis-Steele), then the
// broadcasts of lane 15 into rows 1 and 3 and of lane 31 into rows 2 and 3.
// VALU only: no LDS round trip per step.
template <typename T>
__device__ __forceinline__ T wave_inclusive_scan(T v) {
  static_assert(std::is_integral<T>::value, "integer sums (the order is not the lane order)");
  v += dpp_take<0x111, 0xf>(v);  // row_shr:1
  v += dpp_take<0x112, 0xf>(v);  // row_shr:2
  v += dpp_take<0x114, 0xf>(v);  // row_shr:4
  v += dpp_take<0x118, 0xf>(v);  // row_shr:8
  v += dpp_take<0x142, 0xa>(v);  // row_bcast:15
  v += dpp_take<0x143, 0xc>(v);  // row_bcast:31
  return v;
}

template <typename T>
__device__ __forceinline__ T wave_sum(T v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}

// Hardware float atomics (no CAS loop; built with -munsafe-fp-atomics).
// Transpose of a 64 x 64 bit matrix held one row per lane (bit j of lane
// i's word is M[i][j]): returns column `lane` (bit i is M[i][lane]).  Six
// butterfly stages swap blocks of 32, 16, ..., 1 bits between lanes i and
// i ^ s, two lane shuffles and a few logic operations each.
__device__ __forceinline__ uint64_t transpose_bits64(uint64_t row, uint32_t lane) {
  constexpr uint64_t kKeep[6] = {0x00000000FFFFFFFFull, 0x0000FFFF0000FFFFull,
                                 0x00FF00FF00FF00FFull, 0x0F0F0F0F0F0F0F0Full,
                                 0x3333333333333333ull, 0x5555555555555555ull};
#pragma unroll
  for (int k = 0; k < 6; ++k) {
    const int s = 32 >> k;
    const uint64_t m = kKeep[k];
    const uint32_t lo = static_cast<uint32_t>(__shfl_xor(static_cast<int>(row), s));
    const uint32_t hi = static_cast<uint32_t>(__shfl_xor(static_cast<int>(row >> 32), s));
    const uint64_t other = (static_cast<uint64_t>(hi) << 32) | lo;
    row = (lane & static_cast<uint32_t>(s)) ? (((other >> s) & m) | (row & ~m))
                                            : ((row & m) | ((other & m) << s));
  }
  return row;
}

// N records of type Rec staged in LDS word-major: word w of record i at
// words[w][i].  Lanes that touch one word of consecutive records hit
// consecutive banks; a record-major array whose record size is a multiple
// of 64 bytes would put a whole wave on two of the 32 banks.
template <typename Rec, int N>
struct WordMajor {
  static constexpr int kWords = static_cast<int>((sizeof(Rec) + 3) / 4);
  uint32_t words[kWords][N];
  __device__ __forceinline__ void store(int i, const Rec &r) {
    uint32_t t[kWords];
    __builtin_memcpy(t, &r, sizeof(Rec));
#pragma unroll
    for (int w = 0; w < kWords; ++w) words[w][i] = t[w];
  }
  __device__ __forceinline__ Rec load(int i) const {
    uint32_t t[kWords];
#pragma unroll
    for (int w = 0; w < kWords; ++w) t[w] = words[w][i];
    Rec r;
    __builtin_memcpy(&r, t, sizeof(Rec));
    return r;
  }
};

__device__ __forceinline__ void atomic_add(float *p, float v) { unsafeAtomicAdd(p, v); }
__device__ __forceinline__ void atomic_add(double *p, double v) { unsafeAtomicAdd(p, v); }

// Segments of a wave: runs of equal `seg` over consecutive lanes.
// suffix_sum(x) returns the sum of x over the caller's segment from the
// caller onwards, so the first lane of a segment receives its total.
struct WaveSegments {
  uint32_t same;  // bit s set: lane + 2^s is in the caller's segment
  __device__ __forceinline__ explicit WaveSegments(int32_t seg) : same(0) {
    const uint32_t lane = lane_id();
#pragma unroll
    for (int s = 0; s < 6; ++s) {
      const int32_t sy = __shfl_down(seg, 1 << s, 64);
      if (lane + (1u << s) < 64u && sy == seg) same |= 1u << s;
    }
  }
  template <typename T>
  __device__ __forceinline__ T suffix_sum(T x) const {
#pragma unroll
    for (int s = 0; s < 6; ++s) {
      const T y = __shfl_down(x, 1 << s, 64);
      if ((same >> s) & 1u) x += y;
    }
    return x;
  }
};

}  // namespace r2s
