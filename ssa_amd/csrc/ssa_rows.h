// Gathers of whole bf16 rows (K / V rows picked by index) into LDS, shared by
// the attention kernel and the candidate screen of stage (c).
//
// A wave-wide buffer_load_dwordx4 ... lds moves 1 KB: lane l's 16 bytes land
// at the load's LDS base + 16*l.  Loads that move whole rows (4 rows of 256 B
// at d = 128) are the shape the texture path moves fastest; a load touching
// 16 rows x 64 B moves bytes about 3x slower from L2.
#pragma once

#include "ssa_common.h"

namespace ssa {
namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float floatx4_t __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) bf16x8_t* lds_bf16x8_ptr;
typedef __attribute__((address_space(3))) void* lds_void_ptr;

constexpr int kMfChunk = 32;  // keys gathered per chunk

// Raw buffer descriptor word 3 for gfx9-family loads (32-bit data format),
// and a byte offset past any buffer this kernel builds (an out-of-range buffer
// load returns zeros, also into LDS).
constexpr int kBufferWord3 = 0x00020000;
constexpr uint32_t kOobOffset = 0x7FFFFFF0u;

template <int D>
struct MfShape {
  static constexpr int KB = D / 32;           // 32-dim blocks of Q.K
  static constexpr int NT = D / 16;           // 16-feature tiles of P.V
  static constexpr int ROW = 2 * D;           // bytes per staged row
  static constexpr int SEGS = D / 8;          // 16-byte segments per row
  static constexpr int KPI = 64 / SEGS;       // rows per wave-wide load (KPI * ROW = 1 KB)
  static constexpr int NLD = kMfChunk / KPI;  // loads per chunk, each for K and V
  static constexpr int RPL = 256 / ROW;       // rows per 256-byte bank line
  static constexpr int SWZ_PERIOD = (D == 128) ? 4 : 2;  // mf_swz of load r repeats with this period
  static_assert(D == 64 || D == 128, "row gathers: d = 64 or 128");
};

// LDS slot of segment s of chunk row `key` is s ^ mf_swz(key).  With u = key /
// RPL (rows of one bank line share u), swz = 2*(u mod SEGS/2) + (u / (SEGS/2)
// mod 2): the 16 rows of a K fragment read (one segment each) hit 16 distinct
// 16-byte bank groups, and the four rows of a transposing V read (two adjacent
// segments each) hit four distinct 32-byte groups.
template <int D>
__device__ __forceinline__ int mf_swz(int key) {
  using S = MfShape<D>;
  const int u = key / S::RPL;
  return ((u & (S::SEGS / 2 - 1)) << 1) | ((u / (S::SEGS / 2)) & 1);
}

// Byte offset within its row of the segment lane `lane` fetches in load r of a
// chunk (slot lane % SEGS of chunk row KPI*r + lane / SEGS); periodic in r.
template <int D>
__device__ __forceinline__ void row_seg16(int lane, uint32_t (&seg16)[MfShape<D>::SWZ_PERIOD]) {
  using S = MfShape<D>;
#pragma unroll
  for (int r = 0; r < S::SWZ_PERIOD; ++r)
    seg16[r] = static_cast<uint32_t>(((lane % S::SEGS) ^ mf_swz<D>(S::KPI * r + lane / S::SEGS)) << 4);
}

// One chunk of rows of one tensor into LDS at `l` (load r at l + r KB).
// jsafe (lanes < kMfChunk): the row index per chunk slot, negative for a slot
// that must read as zeros; sn2: the row stride in bytes.
template <int D>
__device__ __forceinline__ void row_issue(__amdgpu_buffer_rsrc_t rs, unsigned char* l, int jsafe, int lane,
                                          uint32_t sn2, const uint32_t (&seg16)[MfShape<D>::SWZ_PERIOD]) {
  using S = MfShape<D>;
  int jr[S::NLD];
#pragma unroll
  for (int r = 0; r < S::NLD; ++r) jr[r] = __shfl(jsafe, S::KPI * r + lane / S::SEGS);
#pragma unroll
  for (int r = 0; r < S::NLD; ++r) {
    const uint32_t o = jr[r] >= 0 ? __umul24(static_cast<uint32_t>(jr[r]), sn2) + seg16[r % S::SWZ_PERIOD]
                                  : kOobOffset;
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (lds_void_ptr)(l + r * 1024), 16, static_cast<int>(o), 0, 0, 0);
  }
}

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef short v4i16_t __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) v4i16_t* lds_v4i16_ptr;

__device__ __forceinline__ uint32_t pack_bf16x2(float a, float b) {
  const bf16x2_t v = {static_cast<__bf16>(a), static_cast<__bf16>(b)};
  return __builtin_bit_cast(uint32_t, v);
}
// lane p of each 16-lane row reads lane p - 8 (lanes p < 8 read 0: bound_ctrl,
// so no zeroed old value is needed and the compiler may fold the move into
// the instruction that uses it)
__device__ __forceinline__ uint32_t dpp_from_minus8(uint32_t x) {
  return __builtin_amdgcn_update_dpp(0u, x, 0x118, 0xF, 0xF, true);
}
// lane p of each 16-lane row reads lane p + 8 (lanes p >= 8 read 0)
__device__ __forceinline__ float dpp_from_plus8(float x) {
  return __uint_as_float(__builtin_amdgcn_update_dpp(0u, __float_as_uint(x), 0x108, 0xF, 0xF, true));
}

// NaN-propagating maximum (v_maximum3_f32 on gfx950): unlike fmaxf it needs no
// canonicalizing v_max of a matrix-core result first.
__device__ __forceinline__ float max_nan(float a, float b) { return __builtin_elementwise_maximum(a, b); }

// Combine each lane's value with those of lanes l ^ 16, l ^ 32 and l ^ 48
// (the four 16-lane rows): v_permlane16_swap / v_permlane32_swap exchange
// whole rows in registers, so no LDS round trip (as a shuffle would take).
// Each swap leaves lane l with its own value and its partner's, in some
// order; op is symmetric.
template <class Op>
__device__ __forceinline__ float rows4_reduce(float x, Op op) {
  const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  x = op(__uint_as_float(a[0]), __uint_as_float(a[1]));
  const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return op(__uint_as_float(b[0]), __uint_as_float(b[1]));
}

// op over all 64 lanes, the result in every lane, with no LDS round trip:
// DPP quad_perm [1,0,3,2] and [2,3,0,1] within each quad, row_half_mirror
// (lane i of 8 reads 7 - i: the other quad) and row_mirror (lane i of 16
// reads 15 - i: the other half), then rows4_reduce across the rows.  op is
// symmetric and associative (min, max).
template <class Op>
__device__ __forceinline__ float wave_allreduce(float x, Op op) {
  x = op(x, __uint_as_float(__builtin_amdgcn_update_dpp(0u, __float_as_uint(x), 0xB1, 0xF, 0xF, true)));
  x = op(x, __uint_as_float(__builtin_amdgcn_update_dpp(0u, __float_as_uint(x), 0x4E, 0xF, 0xF, true)));
  x = op(x, __uint_as_float(__builtin_amdgcn_update_dpp(0u, __float_as_uint(x), 0x141, 0xF, 0xF, true)));
  x = op(x, __uint_as_float(__builtin_amdgcn_update_dpp(0u, __float_as_uint(x), 0x140, 0xF, 0xF, true)));
  return rows4_reduce(x, op);
}

// V^T (or K^T) fragment of 16-feature tile t from a chunk's rows in LDS at `l`
// (the A operand of O^T += V^T P^T): within each 16-lane group, lane p receives
// element p mod 4 from the rows addressed by lanes p / 4 + 4e, which matches
// the key order of a P^T operand built from the S^T layout (lane (q4, c16):
// keys 16t' + 4 q4 + e).
template <int D>
__device__ __forceinline__ bf16x8_t rows_transposed(const unsigned char* l, int t, int q4, int c16) {
  using S = MfShape<D>;
  const int vkey = 4 * q4 + (c16 >> 2);
  const int off = vkey * S::ROW + (((2 * t + ((c16 & 3) >> 1)) ^ mf_swz<D>(vkey)) << 4) + (c16 & 1) * 8;
  const v4i16_t a0 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4i16_ptr)(l + off));
  const v4i16_t a1 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4i16_ptr)(l + off + 16 * S::ROW));
  return __builtin_bit_cast(bf16x8_t, make_uint4(__builtin_bit_cast(uint2, a0).x, __builtin_bit_cast(uint2, a0).y,
                                                 __builtin_bit_cast(uint2, a1).x, __builtin_bit_cast(uint2, a1).y));
}

// s_waitcnt encodings (gfx9): vmcnt(0) alone, lgkmcnt(0) alone; vmcnt(N) for
// N < 16 is kWaitVmBase | N.
constexpr int kWaitVm0 = 0x0F70;
constexpr int kWaitVmBase = 0x0F70;
constexpr int kWaitLgkm0 = 0xC07F;

// Which chunks (kMfChunk index slots each) of a row hold a key to attend.  A
// row gathers its chunks one after the other, each chunk's loads flying while
// the one before computes; a chunk with nothing to attend (below a dense
// prefix, past the causal cut, filler) would still cost one index load's
// latency with nothing else in flight.  build() loads the indices of the first
// 16 chunks all at once, two chunks per load (lanes 32..63 take the odd one),
// and sets bit u of `live` when a slot of chunk u passes ok(); chunks from 16
// on count as live (a second batch would put a second load latency in front of
// every row, which rows without filler, the common case at top_k 1024, never
// repay).  The 16 chunks' indices stay in registers for get().
struct LiveChunks {
  static constexpr int kPairs = 8;  // chunk pairs per batch of loads
  uint64_t live;
  int n;   // chunks of the row
  int nm;  // chunks the mask covers
  int first[kPairs];

  // raw(u, l): index entry of slot l of chunk u, as loaded (any value where
  // key() drops the slot); key(u, l, entry): its key, negative when none
  // (checks and flags happen here, after all loads of a batch are out);
  // ok(key): the slot is attended
  template <class Raw, class Key, class Ok>
  __device__ __forceinline__ void build(int nch, int lane, Raw raw, Key key, Ok ok) {
    n = nch;
    nm = nch < 2 * kPairs ? nch : 2 * kPairs;
    live = 0;
    uint64_t rv[kPairs];
#pragma unroll
    for (int e = 0; e < kPairs; ++e) {
      const int u = 2 * e + (lane >> 5);
      rv[e] = u < nm ? raw(u, lane & 31) : 0;
    }
#pragma unroll
    for (int e = 0; e < kPairs; ++e) {
      const int u = 2 * e + (lane >> 5);
      first[e] = u < nm ? key(u, lane & 31, rv[e]) : -1;
    }
#pragma unroll
    for (int e = 0; e < kPairs; ++e) {
      const uint64_t b = __ballot(ok(first[e]));
      live |= (static_cast<uint64_t>(static_cast<uint32_t>(b) != 0u) << (2 * e)) |
              (static_cast<uint64_t>((b >> 32) != 0u) << (2 * e + 1));
    }
  }
  // no mask: every chunk counts as live (rows without a dense prefix, whose
  // chunks all hold selected keys)
  __device__ __forceinline__ void all_live(int nch) {
    n = nch;
    nm = 0;
    live = 0;
  }
  // the first chunk after u to process, n when none is left
  __device__ __forceinline__ int next(int u) const {
    const int v = u + 1;
    if (v >= nm) return v < n ? v : n;
    const uint64_t m = live & (~0ull << v);
    if (m) return __builtin_ctzll(m);
    return nm < n ? nm : n;
  }
  // indices of chunk u in lanes < kMfChunk (-1 in the others): from the
  // registers for the chunks the mask covers, else load(u)
  template <class Load>
  __device__ __forceinline__ int get(int u, int lane, Load load) const {
    if (u >= nm) return load(u);
    int x = first[0];
#pragma unroll
    for (int e = 1; e < kPairs; ++e) x = (u >> 1) == e ? first[e] : x;
    const int y = __shfl_xor(x, 32);
    return lane < kMfChunk ? ((u & 1) ? y : x) : -1;
  }
};

}  // namespace
}  // namespace ssa
