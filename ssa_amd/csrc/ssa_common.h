// Shared device helpers and host-side status plumbing for libssa_hip.
//
// Arithmetic contract (identical to the CPU oracle, bit for bit):
//   * inputs are widened exactly to fp32; every dot product is one fmaf chain
//     in ascending index order from +0.0f;
//   * division and sqrt are IEEE correctly rounded (the library is built with
//     -fhip-fp32-correctly-rounded-divide-sqrt, -ffp-contract=off and no
//     denormal flushing);
//   * selections order by the 64-bit composite key
//     (ordered_bits(score) << 32) | (0xFFFFFFFF - index): larger is better,
//     so ties on score go to the lowest index.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "ssa_hip.h"

namespace ssa {

// ------------------------------------------------------------------ device

__device__ __forceinline__ float bf16_bits_to_f32(uint16_t u) {
  return __uint_as_float(static_cast<uint32_t>(u) << 16);
}

// fp32 -> bf16 bits, round to nearest even; NaN stays a (quiet) NaN.  Both
// results are computed and one is selected: no branch, so no exec-mask
// sequence per value.
__device__ __forceinline__ uint16_t f32_to_bf16_rne(float f) {
  const uint32_t u = __float_as_uint(f);
  const uint32_t rounded = (u + 0x7FFFu + ((u >> 16) & 1u)) >> 16;
  const bool nan = (u & 0x7FFFFFFFu) > 0x7F800000u;
  return static_cast<uint16_t>(nan ? ((u >> 16) | 0x40u) : rounded);
}

// a / b for 0 <= a < 2^32 and 0 < b < 2^32.  Row, head and query indices are
// below 2^31 (the launchers check), and the 32-bit unsigned division takes a
// small fraction of the instructions of the 64-bit sequence (about 130 scalar
// instructions per division, once per row in the one-row-per-wave kernels).
__device__ __forceinline__ int64_t udiv32(int64_t a, int64_t b) {
  return static_cast<int64_t>(static_cast<uint32_t>(a) / static_cast<uint32_t>(b));
}

// x of lane src for a wave-uniform src (a loop counter, a ballot's first bit):
// v_readlane, a scalar result with no LDS round trip, where __shfl's
// ds_bpermute waits on the LDS.  The lane's register is read whatever the
// exec mask, so x must have been computed by that lane.
__device__ __forceinline__ int lane_value(int x, int src) { return __builtin_amdgcn_readlane(x, src); }
__device__ __forceinline__ float lane_value(float x, int src) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x), src));
}

// Element loaders: T is the storage type (float or uint16_t holding bf16 bits).
__device__ __forceinline__ float ld(const float* p) { return *p; }
__device__ __forceinline__ float ld(const uint16_t* p) { return bf16_bits_to_f32(*p); }

// Monotone map float -> uint32; -0.0 folds into +0.0.
__device__ __forceinline__ uint32_t score_key(float s) {
  uint32_t u = __float_as_uint(s);
  if (u == 0x80000000u) u = 0u;
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

__device__ __forceinline__ uint64_t composite_key(float s, uint32_t idx) {
  return (static_cast<uint64_t>(score_key(s)) << 32) | static_cast<uint64_t>(0xFFFFFFFFu - idx);
}

__device__ __forceinline__ uint32_t key_index(uint64_t key) {
  return 0xFFFFFFFFu - static_cast<uint32_t>(key & 0xFFFFFFFFull);
}

// Inclusive prefix sum over the 64 lanes of a wave (all lanes active), in six
// DPP adds: row_shr 1, 2, 4 (banks 1-3), 8 (banks 2-3) scan each 16-lane row,
// then row_bcast 15 and 31 carry the row totals into the rows above.  A lane
// whose DPP source does not exist adds the `old` operand, 0.  (A shuffle
// ladder costs an LDS round trip and its address arithmetic per step.)
__device__ __forceinline__ int wave_incl_scan(int x) {
  int v = x;
  v += __builtin_amdgcn_update_dpp(0, v, 0x111, 0xF, 0xF, false);
  v += __builtin_amdgcn_update_dpp(0, v, 0x112, 0xF, 0xF, false);
  v += __builtin_amdgcn_update_dpp(0, v, 0x114, 0xF, 0xE, false);
  v += __builtin_amdgcn_update_dpp(0, v, 0x118, 0xF, 0xC, false);
  v += __builtin_amdgcn_update_dpp(0, v, 0x142, 0xA, 0xF, false);
  v += __builtin_amdgcn_update_dpp(0, v, 0x143, 0xC, 0xF, false);
  return v;
}

// fp32 fused multiply-add, single rounding (v_fma_f32).
__device__ __forceinline__ float fma_rn(float a, float b, float c) { return __builtin_fmaf(a, b, c); }

// The GPU hands workgroups to its 8 XCDs (each with its own L2) round-robin:
// workgroup w runs on XCD w mod 8.  xcd_block maps the launched workgroup w of
// a grid of 8 * per workgroups to the logical block (w mod 8) * per + w / 8, so
// that XCD x runs the contiguous logical blocks [x * per, (x + 1) * per) and
// its L2 holds their shared data (the rows of one KV head, say) instead of a
// slice of everything.  Logical blocks at or past the real count are idle.
constexpr int kXcds = 8;
__host__ __device__ inline int64_t xcd_per(int64_t nblocks) { return (nblocks + kXcds - 1) / kXcds; }
__device__ __forceinline__ int64_t xcd_block(int64_t w, int64_t per) { return (w % kXcds) * per + w / kXcds; }

// Block-strided loop over elements [0, count) (thread `tid` of NT takes tid,
// tid + NT, ...) that issues U independent loads before it uses any of them.
// A loop whose body loads one element and then uses it waits out a whole
// memory round trip per iteration; in the small grids of decoding those
// round trips are most of a kernel's time.  Whole batches load without
// bounds tests (a guarded load sits in a branch of its own, behind a wait
// for the loads before it); only the last, partial batch tests each element.
template <int U, int NT, typename Load, typename Use>
__device__ __forceinline__ void strided_batches(int64_t count, int tid, Load load, Use use) {
  using V = decltype(load(int64_t(0)));
  int64_t e0 = 0;
  for (; e0 + static_cast<int64_t>(U) * NT <= count; e0 += static_cast<int64_t>(U) * NT) {
    V v[U];
#pragma unroll
    for (int j = 0; j < U; ++j) v[j] = load(e0 + static_cast<int64_t>(j) * NT + tid);
#pragma unroll
    for (int j = 0; j < U; ++j) use(e0 + static_cast<int64_t>(j) * NT + tid, v[j]);
  }
  for (int64_t e = e0 + tid; e < count; e += NT) use(e, load(e));
}

// ------------------------------------------------------------------ host

// Records a human-readable detail for the last failing call on this thread.
int fail(int status, const char* fmt, ...);

// Maps a pending HIP launch error to SSA_ERR_HIP (and records its text).
int check_launch(const char* what);

inline hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

// Makes `bytes` of dynamic LDS available to `kernel` on the current device, or
// fails with SSA_ERR_UNSUPPORTED when the device cannot provide it.
int reserve_lds(const void* kernel, size_t bytes, const char* what);

__host__ __device__ inline int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }

__host__ __device__ inline size_t align_up(size_t x, size_t a) { return (x + a - 1) / a * a; }

}  // namespace ssa
