// Stage (a): routing vectors and codebook top-codes.
//
// Replaces ssa/router.py:102-141 (projection, GQA mean, F.normalize, codebook
// einsum / temperature, topk).  All arithmetic is exact-order fp32 so that the
// selected codes are bit-identical with the CPU oracle.
#include <algorithm>
#include <type_traits>

#include "ssa_common.h"
#include "ssa_internal.h"

namespace ssa {
namespace {

constexpr int kRouteThreads = 256;
constexpr int kRouteRowsPerThread = 4;

// One thread owns one routing coordinate s for kRouteRowsPerThread rows:
//   out[b][h][i][s] = normalize_s( (sum_gg chain_t x[b][i][h*g+gg][t] * w[s][t]) / g )
// W and a tile of x rows (one GQA head at a time) are staged in LDS as fp32.
template <typename T>
__global__ __launch_bounds__(kRouteThreads) void route_vectors_kernel(
    const T* __restrict__ x, int64_t n, int h_in, int group, int d, int64_t sb, int64_t sn,
    int64_t sh, const float* __restrict__ w, int d_s, int dsp, float* __restrict__ out) {
  extern __shared__ __align__(16) float smem[];
  const int dpad = d + 4;
  const int rows_per_pass = kRouteThreads / dsp;
  const int rb = rows_per_pass * kRouteRowsPerThread;
  float* Ws = smem;                // [d_s][dpad]
  float* Xs = Ws + d_s * dpad;     // [rb][dpad]
  float* red = Xs + rb * dpad;     // [rb][d_s]

  const int h_out = h_in / group;
  const int64_t tiles = (n + rb - 1) / rb;
  const int64_t bh = udiv32(blockIdx.x, tiles);
  const int64_t i0 = (blockIdx.x - bh * tiles) * rb;
  const int64_t b = udiv32(bh, h_out);
  const int h = static_cast<int>(bh - b * h_out);
  const int tid = threadIdx.x;

  for (int e = tid; e < d_s * d; e += kRouteThreads) Ws[(e / d) * dpad + (e % d)] = w[e];

  const int r = tid / dsp;
  const int s = tid % dsp;
  const bool lane_ok = (r < rows_per_pass) && (s < d_s);
  float sum[kRouteRowsPerThread];
#pragma unroll
  for (int u = 0; u < kRouteRowsPerThread; ++u) sum[u] = 0.0f;

  for (int gg = 0; gg < group; ++gg) {
    __syncthreads();
    const T* xh = x + b * sb + static_cast<int64_t>(h * group + gg) * sh;
    for (int e = tid; e < rb * d; e += kRouteThreads) {
      const int rr = e / d, t = e % d;
      const int64_t i = i0 + rr;
      Xs[rr * dpad + t] = (i < n) ? ld(xh + i * sn + t) : 0.0f;
    }
    __syncthreads();
    if (lane_ok) {
      const float* wr = Ws + s * dpad;
      float acc[kRouteRowsPerThread];
#pragma unroll
      for (int u = 0; u < kRouteRowsPerThread; ++u) acc[u] = 0.0f;
      for (int t = 0; t < d; t += 4) {
        const float4 wv = *reinterpret_cast<const float4*>(wr + t);
#pragma unroll
        for (int u = 0; u < kRouteRowsPerThread; ++u) {
          const float4 xv =
              *reinterpret_cast<const float4*>(Xs + (r + u * rows_per_pass) * dpad + t);
          acc[u] = fma_rn(xv.x, wv.x, acc[u]);
          acc[u] = fma_rn(xv.y, wv.y, acc[u]);
          acc[u] = fma_rn(xv.z, wv.z, acc[u]);
          acc[u] = fma_rn(xv.w, wv.w, acc[u]);
        }
      }
#pragma unroll
      for (int u = 0; u < kRouteRowsPerThread; ++u) sum[u] = (gg == 0) ? acc[u] : sum[u] + acc[u];
    }
  }

  float val[kRouteRowsPerThread];
#pragma unroll
  for (int u = 0; u < kRouteRowsPerThread; ++u) {
    val[u] = sum[u] / static_cast<float>(group);
    if (lane_ok) red[(r + u * rows_per_pass) * d_s + s] = val[u];
  }
  __syncthreads();
  if (!lane_ok) return;
#pragma unroll
  for (int u = 0; u < kRouteRowsPerThread; ++u) {
    const int rr = r + u * rows_per_pass;
    if (i0 + rr >= n) continue;
    const float* y = red + rr * d_s;
    float nrm = 0.0f;
    for (int v = 0; v < d_s; ++v) nrm = fma_rn(y[v], y[v], nrm);
    const float den = fmaxf(sqrtf(nrm), 1e-12f);
    out[(bh * n + i0 + rr) * d_s + s] = val[u] / den;
  }
}

// route_dim <= 32: 64-row tiles, each thread a 2-row x 4-coordinate register
// tile (eight coordinate groups x 32 row pairs), so every 4-dim step reads two
// x and four w float4s from LDS for 32 fmaf.  Same per-score chains as above:
// one fmaf chain over t ascending per head, the group summed in head order,
// then / group and normalized.  x rows are staged with 4-element vector loads
// (strides and base aligned to 4 elements).
constexpr int kRvRows = 64;

__device__ __forceinline__ float4 load4(const float* p) { return *reinterpret_cast<const float4*>(p); }
__device__ __forceinline__ float4 load4(const uint16_t* p) {
  const uint2 u = *reinterpret_cast<const uint2*>(p);
  return make_float4(__uint_as_float(u.x << 16), __uint_as_float(u.x & 0xFFFF0000u),
                     __uint_as_float(u.y << 16), __uint_as_float(u.y & 0xFFFF0000u));
}

template <typename T>
__global__ __launch_bounds__(256) void route_vectors_tile_kernel(
    const T* __restrict__ x, int64_t n, int h_in, int group, int d, int64_t sb, int64_t sn,
    int64_t sh, const float* __restrict__ w, int d_s, float* __restrict__ out) {
  extern __shared__ __align__(16) float smem[];
  const int dpad = d + 4;
  float* Ws = smem;                   // [32][dpad], coordinates >= d_s are zero
  float* Xs = Ws + 32 * dpad;         // [kRvRows][dpad]
  float* red = Xs + kRvRows * dpad;   // [kRvRows][32]
  const int h_out = h_in / group;
  const int64_t tiles = (n + kRvRows - 1) / kRvRows;
  const int64_t bh = udiv32(blockIdx.x, tiles);
  const int64_t i0 = (blockIdx.x - bh * tiles) * kRvRows;
  const int64_t b = udiv32(bh, h_out);
  const int h = static_cast<int>(bh - b * h_out);
  const int tid = threadIdx.x;
  const int cg = tid & 7;   // coordinates 4*cg .. 4*cg+3
  const int rg = tid >> 3;  // rows 2*rg, 2*rg+1
  const int d4 = d / 4;

  for (int e = tid; e < 32 * d4; e += 256) {
    const int sc = e / d4, t = 4 * (e % d4);
    *reinterpret_cast<float4*>(Ws + sc * dpad + t) =
        (sc < d_s) ? *reinterpret_cast<const float4*>(w + static_cast<int64_t>(sc) * d + t)
                   : make_float4(0.f, 0.f, 0.f, 0.f);
  }
  float sum[2][4];
  for (int gg = 0; gg < group; ++gg) {
    __syncthreads();
    const T* xh = x + b * sb + static_cast<int64_t>(h * group + gg) * sh;
    for (int e = tid; e < kRvRows * d4; e += 256) {
      const int rr = e / d4, t = 4 * (e % d4);
      const int64_t i = i0 + rr;
      *reinterpret_cast<float4*>(Xs + rr * dpad + t) = (i < n) ? load4(xh + i * sn + t)
                                                                : make_float4(0.f, 0.f, 0.f, 0.f);
    }
    __syncthreads();
    float acc[2][4];
#pragma unroll
    for (int r = 0; r < 2; ++r)
#pragma unroll
      for (int c = 0; c < 4; ++c) acc[r][c] = 0.0f;
    const float* xr = Xs + (2 * rg) * dpad;
    const float* wr = Ws + (4 * cg) * dpad;
    for (int t = 0; t < d; t += 4) {
      float4 xv[2], wv[4];
#pragma unroll
      for (int r = 0; r < 2; ++r) xv[r] = *reinterpret_cast<const float4*>(xr + r * dpad + t);
#pragma unroll
      for (int c = 0; c < 4; ++c) wv[c] = *reinterpret_cast<const float4*>(wr + c * dpad + t);
#pragma unroll
      for (int r = 0; r < 2; ++r)
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          acc[r][c] = fma_rn(xv[r].x, wv[c].x, acc[r][c]);
          acc[r][c] = fma_rn(xv[r].y, wv[c].y, acc[r][c]);
          acc[r][c] = fma_rn(xv[r].z, wv[c].z, acc[r][c]);
          acc[r][c] = fma_rn(xv[r].w, wv[c].w, acc[r][c]);
        }
    }
#pragma unroll
    for (int r = 0; r < 2; ++r)
#pragma unroll
      for (int c = 0; c < 4; ++c) sum[r][c] = (gg == 0) ? acc[r][c] : sum[r][c] + acc[r][c];
  }
  float val[2][4];
#pragma unroll
  for (int r = 0; r < 2; ++r)
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      val[r][c] = sum[r][c] / static_cast<float>(group);
      red[(2 * rg + r) * 32 + 4 * cg + c] = val[r][c];
    }
  __syncthreads();
#pragma unroll
  for (int r = 0; r < 2; ++r) {
    const int64_t i = i0 + 2 * rg + r;
    if (i >= n) continue;
    const float* y = red + (2 * rg + r) * 32;
    float nrm = 0.0f;
    for (int v = 0; v < d_s; ++v) nrm = fma_rn(y[v], y[v], nrm);
    const float den = fmaxf(sqrtf(nrm), 1e-12f);
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const int sc = 4 * cg + c;
      if (sc < d_s) out[(bh * n + i) * d_s + sc] = val[r][c] / den;
    }
  }
}

size_t route_vectors_tile_smem(int d) {
  return sizeof(float) * (static_cast<size_t>(32 + kRvRows) * (d + 4) + static_cast<size_t>(kRvRows) * 32);
}

// route_dim == 32, head_dim a multiple of 8: one lane per output row, all 32
// coordinates in registers.  W is the same for every lane, so its
// entries are wave-uniform scalar loads (s_load) and every fmaf takes its W
// operand from an SGPR: no LDS traffic.  The lane reads its own x row in
// 8-element pieces, one piece ahead of the one being multiplied.  Same per-score
// chains as the kernels above: one fmaf chain over t ascending per head, the
// group summed in head order, then / group and normalized.
constexpr int kRrThreads = 256;

struct Piece8 {
  float v[8];
};
__device__ __forceinline__ Piece8 load8(const uint16_t* p) {
  const uint4 u = *reinterpret_cast<const uint4*>(p);
  Piece8 r;
  const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    r.v[2 * e] = __uint_as_float(w[e] << 16);
    r.v[2 * e + 1] = __uint_as_float(w[e] & 0xFFFF0000u);
  }
  return r;
}
__device__ __forceinline__ Piece8 load8(const float* p) {
  const float4 a = reinterpret_cast<const float4*>(p)[0];
  const float4 b = reinterpret_cast<const float4*>(p)[1];
  return Piece8{{a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w}};
}

template <typename T, int DC>
__global__ __launch_bounds__(kRrThreads) void route_vectors_row_kernel(
    const T* __restrict__ x, int64_t n, int h_in, int group, int d_rt, int64_t sb, int64_t sn,
    int64_t sh, const float* __restrict__ w, float* __restrict__ out) {
  constexpr int d_s = 32;
  const int d = DC > 0 ? DC : d_rt;
  const int h_out = h_in / group;
  const int64_t tiles = (n + kRrThreads - 1) / kRrThreads;
  const int64_t bh = udiv32(blockIdx.x, tiles);
  const int64_t i = (blockIdx.x - bh * tiles) * kRrThreads + threadIdx.x;
  const int64_t b = udiv32(bh, h_out);
  const int h = static_cast<int>(bh - b * h_out);
  const int64_t ic = i < n ? i : n - 1;  // lanes past n compute row n-1 and store nothing
  const T* xb = x + b * sb + static_cast<int64_t>(h) * group * sh + ic * sn;
  const int pieces = d / 8;
  const int total = group * pieces;

  float sum[32], acc[32];
#pragma unroll
  for (int s = 0; s < 32; ++s) sum[s] = acc[s] = 0.0f;
  // With d fixed at compile time, 8 pieces per unrolled step: every W
  // operand of the step is an immediate offset from one base, so the scalar
  // loads of several pieces go out together (one piece per step waits on its
  // W loads every dozen fmas).
  constexpr int UNR = DC > 0 && DC % 64 == 0 ? 8 : 1;
  Piece8 cur = load8(xb);
#pragma unroll 1
  for (int c0 = 0; c0 < total; c0 += UNR) {
#pragma unroll
    for (int u = 0; u < UNR; ++u) {
      const int c = c0 + u;
      const int gg = c / pieces;
      const int t0 = (c - gg * pieces) * 8;
      const int cn = c + 1 < total ? c + 1 : c;
      const int ggn = cn / pieces;
      const Piece8 nxt = load8(xb + static_cast<int64_t>(ggn) * sh + (cn - ggn * pieces) * 8);
#pragma unroll
      for (int s = 0; s < d_s; ++s) {
        const float* ws = w + static_cast<int64_t>(s) * d + t0;
#pragma unroll
        for (int e = 0; e < 8; ++e) acc[s] = fma_rn(cur.v[e], ws[e], acc[s]);
      }
      if (t0 + 8 == d) {  // head gg complete: fold its chain into the group sum
#pragma unroll
        for (int s = 0; s < 32; ++s) {
          sum[s] = (gg == 0) ? acc[s] : sum[s] + acc[s];
          acc[s] = 0.0f;
        }
      }
      cur = nxt;
    }
  }
  float nrm = 0.0f;
#pragma unroll
  for (int s = 0; s < d_s; ++s) {
    sum[s] = sum[s] / static_cast<float>(group);
    nrm = fma_rn(sum[s], sum[s], nrm);
  }
  const float den = fmaxf(sqrtf(nrm), 1e-12f);
  if (i < n) {
    float* o = out + (bh * n + i) * d_s;
#pragma unroll
    for (int s = 0; s < d_s; ++s) o[s] = sum[s] / den;
  }
}

// One head per output row (group == 1, the keys), route_dim == 32, bf16 rows of
// a fixed head dim: route_vectors_row_kernel with each row's 32 coordinates
// split over two waves of a block (wave 0: coordinates 0-15, wave 1: 16-31,
// the same 64 rows), so twice the waves share the same fmaf chains and each
// wave's W rows are still wave-uniform scalar loads.  The norm chain runs over
// the coordinates in order: wave 0 passes its partial sum of squares to wave 1
// through LDS, wave 1 finishes it and passes the denominator back.  Same
// results as route_vectors_row_kernel, bit for bit.
constexpr int kRhRows = 64;
template <int DC>
__global__ __launch_bounds__(128) void route_vectors_half_kernel(
    const uint16_t* __restrict__ x, int64_t n, int h_in, int64_t sb, int64_t sn, int64_t sh,
    const float* __restrict__ w, float* __restrict__ out) {
  constexpr int HS = 16;  // coordinates per wave
  constexpr int pieces = DC / 8;
  constexpr int UNR = pieces % 8 == 0 ? 8 : 1;
  __shared__ float s_nrm[kRhRows], s_den[kRhRows];
  const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
  const int lane = threadIdx.x & 63;
  const int64_t tiles = (n + kRhRows - 1) / kRhRows;
  const int64_t bh = udiv32(blockIdx.x, tiles);
  const int64_t i = (blockIdx.x - bh * tiles) * kRhRows + lane;
  const int64_t b = udiv32(bh, h_in);
  const int h = static_cast<int>(bh - b * h_in);
  const int64_t ic = i < n ? i : n - 1;  // lanes past n compute row n-1 and store nothing
  const uint16_t* xr = x + b * sb + static_cast<int64_t>(h) * sh + ic * sn;
  const float* wh = w + static_cast<int64_t>(wave * HS) * DC;
  float acc[HS];
#pragma unroll
  for (int s = 0; s < HS; ++s) acc[s] = 0.0f;
  Piece8 cur = load8(xr);
#pragma unroll 1
  for (int c0 = 0; c0 < pieces; c0 += UNR) {
#pragma unroll
    for (int u = 0; u < UNR; ++u) {
      const int c = c0 + u;
      const int cn = c + 1 < pieces ? c + 1 : c;
      const Piece8 nxt = load8(xr + cn * 8);
#pragma unroll
      for (int s = 0; s < HS; ++s) {
        const float* ws = wh + s * DC + c * 8;
#pragma unroll
        for (int e = 0; e < 8; ++e) acc[s] = fma_rn(cur.v[e], ws[e], acc[s]);
      }
      cur = nxt;
    }
  }
  // (the group mean divides by 1: unchanged)
  float nrm = 0.0f;
  if (wave == 0) {
#pragma unroll
    for (int s = 0; s < HS; ++s) nrm = fma_rn(acc[s], acc[s], nrm);
    s_nrm[lane] = nrm;
  }
  __syncthreads();
  if (wave == 1) {
    nrm = s_nrm[lane];
#pragma unroll
    for (int s = 0; s < HS; ++s) nrm = fma_rn(acc[s], acc[s], nrm);
    s_den[lane] = fmaxf(sqrtf(nrm), 1e-12f);
  }
  __syncthreads();
  const float den = s_den[lane];
  if (i < n) {
    float* o = out + (bh * n + i) * 32 + wave * HS;
#pragma unroll
    for (int s = 0; s < HS; ++s) o[s] = acc[s] / den;
  }
}

// GQA groups (group > 1), route_dim == 32, head_dim a multiple of 8: 64 rows
// per block and the group's heads spread over the block's 4 waves (wave w
// takes heads w, w+4, ...), so a head's chain runs in a wave of its own with W
// in SGPRs as above.  Each round of 4 heads passes its per-head chains through
// LDS, where thread t (row t / 4, coordinates 8 (t % 4) .. +7) adds them to the
// group sum in head order, which keeps the sum bit-identical with one thread
// per row.  The norm is then the canonical chain over the row's 32 means.
constexpr int kRsRows = 64;

// One 128-byte line of a row, raw (8 x 16 bytes); pieces past the row end are
// not loaded.
struct Line128 {
  uint4 u[8];
};
template <typename T>
__device__ __forceinline__ Line128 load_line(const T* p, int left) {
  Line128 l;
  const int np = min(128 / static_cast<int>(sizeof(T)), left) * static_cast<int>(sizeof(T)) / 16;
#pragma unroll
  for (int k = 0; k < 8; ++k) l.u[k] = k < np ? reinterpret_cast<const uint4*>(p)[k] : make_uint4(0u, 0u, 0u, 0u);
  return l;
}
// 8-element piece pi of a line: bf16 elements 8 pi .. 8 pi + 7 (one uint4), or
// fp32 elements 8 pi .. 8 pi + 7 (two uint4).
template <typename T>
__device__ __forceinline__ Piece8 line_piece(const Line128& l, int pi) {
  Piece8 r;
  if constexpr (sizeof(T) == 2) {
    const uint32_t w[4] = {l.u[pi].x, l.u[pi].y, l.u[pi].z, l.u[pi].w};
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      r.v[2 * e] = __uint_as_float(w[e] << 16);
      r.v[2 * e + 1] = __uint_as_float(w[e] & 0xFFFF0000u);
    }
  } else {
    const uint4 a = l.u[2 * pi], b = l.u[2 * pi + 1];
    const uint32_t w[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
#pragma unroll
    for (int e = 0; e < 8; ++e) r.v[e] = __uint_as_float(w[e]);
  }
  return r;
}

template <typename T, int DC>
__global__ __launch_bounds__(256) void route_vectors_split_kernel(
    const T* __restrict__ x, int64_t n, int h_in, int group, int d_rt, int64_t sb, int64_t sn,
    int64_t sh, const float* __restrict__ w, float* __restrict__ out) {
  constexpr int d_s = 32;
  const int d = DC > 0 ? DC : d_rt;
  __shared__ float part[4][kRsRows][d_s + 1];  // per-wave head chains, padded rows
  __shared__ float mean[kRsRows][d_s + 1];
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int h_out = h_in / group;
  const int64_t tiles = (n + kRsRows - 1) / kRsRows;
  const int64_t bh = udiv32(blockIdx.x, tiles);
  const int64_t i0 = (blockIdx.x - bh * tiles) * kRsRows;
  const int64_t b = udiv32(bh, h_out);
  const int h = static_cast<int>(bh - b * h_out);
  const int64_t ic = (i0 + lane < n) ? i0 + lane : n - 1;  // rows past n: row n-1, not stored
  const T* xr = x + b * sb + static_cast<int64_t>(h) * group * sh + ic * sn;
  const int cr = threadIdx.x >> 2, cs0 = 8 * (threadIdx.x & 3);
  float sum[8];
#pragma unroll
  for (int k = 0; k < 8; ++k) sum[k] = 0.0f;
  for (int r0 = 0; r0 < group; r0 += 4) {
    const int gg = r0 + wave;
    if (gg < group) {  // wave-uniform
      float acc[d_s];
#pragma unroll
      for (int s = 0; s < d_s; ++s) acc[s] = 0.0f;
      // The lane reads its head row a whole 128-byte line at a time, one line
      // ahead of the one being multiplied: every line is fetched once (16-byte
      // pieces spread over time re-fetched lines evicted in between).
      const T* xh = xr + static_cast<int64_t>(gg) * sh;
      constexpr int CE = 128 / sizeof(T);  // elements per line
      const int nlines = (d + CE - 1) / CE;
      Line128 cur = load_line(xh, d), nxt{};
#pragma unroll 1
      for (int c = 0; c < nlines; ++c) {
        if (c + 1 < nlines) nxt = load_line(xh + (c + 1) * CE, d - (c + 1) * CE);
        const int np = min(CE, d - c * CE) / 8;  // pieces of this line inside the row
#pragma unroll
        for (int pi = 0; pi < CE / 8; ++pi) {
          if (pi < np) {  // uniform
            const Piece8 pc = line_piece<T>(cur, pi);
            const float* wc = w + c * CE + pi * 8;
#pragma unroll
            for (int s = 0; s < d_s; ++s) {
              const float* ws = wc + static_cast<int64_t>(s) * d;
#pragma unroll
              for (int e = 0; e < 8; ++e) acc[s] = fma_rn(pc.v[e], ws[e], acc[s]);
            }
          }
        }
        cur = nxt;
      }
#pragma unroll
      for (int s = 0; s < d_s; ++s) part[wave][lane][s] = acc[s];
    }
    __syncthreads();
    for (int j = 0; j < 4 && r0 + j < group; ++j) {
#pragma unroll
      for (int k = 0; k < 8; ++k) sum[k] = (r0 + j == 0) ? part[j][cr][cs0 + k] : sum[k] + part[j][cr][cs0 + k];
    }
    __syncthreads();
  }
#pragma unroll
  for (int k = 0; k < 8; ++k) {
    sum[k] = sum[k] / static_cast<float>(group);
    mean[cr][cs0 + k] = sum[k];
  }
  __syncthreads();
  float nrm = 0.0f;
#pragma unroll
  for (int s = 0; s < d_s; ++s) nrm = fma_rn(mean[cr][s], mean[cr][s], nrm);
  const float den = fmaxf(sqrtf(nrm), 1e-12f);
  if (i0 + cr < n) {
    float* o = out + (bh * n + i0 + cr) * d_s + cs0;
#pragma unroll
    for (int k = 0; k < 8; ++k) o[k] = sum[k] / den;
  }
}


// Row-wise F.normalize: one thread per row.  Rows of 32 floats (the route
// dim of every config) at 16-byte aligned addresses take a register copy
// loaded in 16-byte pieces, all out before the chain starts (one scalar load
// per element waited on each in turn).
__global__ void normalize_rows_kernel(const float* __restrict__ x, int64_t rows, int d_s,
                                      float* __restrict__ out) {
  const int64_t r = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (r >= rows) return;
  const float* xr = x + r * d_s;
  if (d_s == 32 && ((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(out)) & 15) == 0) {
    float v[32];
#pragma unroll
    for (int q = 0; q < 8; ++q) {
      const float4 f = reinterpret_cast<const float4*>(xr)[q];
      v[4 * q] = f.x;
      v[4 * q + 1] = f.y;
      v[4 * q + 2] = f.z;
      v[4 * q + 3] = f.w;
    }
    float nrm = 0.0f;
#pragma unroll
    for (int s = 0; s < 32; ++s) nrm = fma_rn(v[s], v[s], nrm);
    const float den = fmaxf(sqrtf(nrm), 1e-12f);
#pragma unroll
    for (int q = 0; q < 8; ++q)
      reinterpret_cast<float4*>(out + r * 32)[q] =
          make_float4(v[4 * q] / den, v[4 * q + 1] / den, v[4 * q + 2] / den, v[4 * q + 3] / den);
    return;
  }
  float nrm = 0.0f;
  for (int s = 0; s < d_s; ++s) nrm = fma_rn(xr[s], xr[s], nrm);
  const float den = fmaxf(sqrtf(nrm), 1e-12f);
  for (int s = 0; s < d_s; ++s) out[r * d_s + s] = xr[s] / den;
}

constexpr int kTopRows = 64;   // rows (tokens) per block
constexpr int kTopCodes = 64;  // codes per streamed tile
constexpr int kTopThreads = 256;

__host__ __device__ inline size_t code_topk_smem(int d_s, int top) {
  return sizeof(float) * static_cast<size_t>(d_s) * ((kTopRows + 4) + (kTopCodes + 4)) +
         sizeof(uint64_t) * (static_cast<size_t>(kTopRows) * kTopCodes +
                             static_cast<size_t>(kTopRows) * top + kTopRows) +
         sizeof(int) * 2 * kTopRows;
}

// Scores a 64-row tile against the codebook in 64-code tiles (each thread owns a
// 4x4 register tile, one fmaf chain over s per score) and keeps each row's
// top-`top` composite keys in LDS.  A score enters a row's candidate buffer only
// if it beats the row's current top-th key; one thread per row merges the buffer
// by insertion after each tile.
__global__ __launch_bounds__(kTopThreads) void code_topk_kernel(
    const float* __restrict__ xhat, int64_t rows, int h, const float* __restrict__ chat, int n_c,
    int d_s, float temperature, int top, int32_t* __restrict__ codes) {
  extern __shared__ __align__(16) unsigned char smem_raw[];
  constexpr int rpad = kTopRows + 4, cpad = kTopCodes + 4;
  float* Xs = reinterpret_cast<float*>(smem_raw);                // [d_s][rpad]
  float* Cs = Xs + d_s * rpad;                                   // [d_s][cpad]
  uint64_t* cand = reinterpret_cast<uint64_t*>(Cs + d_s * cpad);  // [rows][codes]
  uint64_t* best = cand + kTopRows * kTopCodes;                  // [rows][top]
  uint64_t* thr = best + kTopRows * top;                         // [rows]
  int* cnt = reinterpret_cast<int*>(thr + kTopRows);             // [rows]
  int* bcnt = cnt + kTopRows;                                    // [rows]

  const int64_t tiles = (rows + kTopRows - 1) / kTopRows;
  const int64_t bh = udiv32(blockIdx.x, tiles);
  const int64_t r0 = (blockIdx.x - bh * tiles) * kTopRows;
  const int hh = static_cast<int>(bh % h);
  const float* xb = xhat + bh * rows * d_s;
  const float* cb = chat + static_cast<int64_t>(hh) * n_c * d_s;
  const int tid = threadIdx.x;

  for (int e = tid; e < kTopRows * d_s; e += kTopThreads) {
    const int r = e / d_s, s = e % d_s;
    Xs[s * rpad + r] = (r0 + r < rows) ? xb[(r0 + r) * d_s + s] : 0.0f;
  }
  if (tid < kTopRows) {
    thr[tid] = 0ull;
    cnt[tid] = 0;
    bcnt[tid] = 0;
  }
  const int rg = tid >> 4, cg = tid & 15;
  const bool scale = (temperature != 1.0f);

  for (int c0 = 0; c0 < n_c; c0 += kTopCodes) {
    for (int e = tid; e < kTopCodes * d_s; e += kTopThreads) {
      const int c = e / d_s, s = e % d_s;
      Cs[s * cpad + c] = (c0 + c < n_c) ? cb[static_cast<int64_t>(c0 + c) * d_s + s] : 0.0f;
    }
    __syncthreads();
    float acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j) acc[i][j] = 0.0f;
    for (int s = 0; s < d_s; ++s) {
      const float4 xv = *reinterpret_cast<const float4*>(Xs + s * rpad + rg * 4);
      const float4 cv = *reinterpret_cast<const float4*>(Cs + s * cpad + cg * 4);
      const float xa[4] = {xv.x, xv.y, xv.z, xv.w};
      const float ca[4] = {cv.x, cv.y, cv.z, cv.w};
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = fma_rn(xa[i], ca[j], acc[i][j]);
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int r = rg * 4 + i;
      if (r0 + r >= rows) continue;
      const uint64_t th = thr[r];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int c = c0 + cg * 4 + j;
        if (c >= n_c) continue;
        float sc = acc[i][j];
        if (scale) sc = sc / temperature;
        const uint64_t key = composite_key(sc, static_cast<uint32_t>(c));
        if (key > th) {
          const int slot = atomicAdd(&cnt[r], 1);
          cand[r * kTopCodes + slot] = key;
        }
      }
    }
    __syncthreads();
    if (tid < kTopRows) {
      const int r = tid;
      int nb = bcnt[r];
      const int nc = cnt[r];
      uint64_t* bl = best + r * top;
      for (int m = 0; m < nc; ++m) {
        const uint64_t key = cand[r * kTopCodes + m];
        if (nb == top && key <= bl[top - 1]) continue;
        int p = (nb < top) ? nb++ : top - 1;
        while (p > 0 && bl[p - 1] < key) {
          bl[p] = bl[p - 1];
          --p;
        }
        bl[p] = key;
      }
      bcnt[r] = nb;
      cnt[r] = 0;
      thr[r] = (nb == top) ? bl[top - 1] : 0ull;
    }
  }
  __syncthreads();
  for (int e = tid; e < kTopRows * top; e += kTopThreads) {
    const int r = e / top, m = e % top;
    if (r0 + r < rows) codes[(bh * rows + r0 + r) * top + m] = static_cast<int32_t>(key_index(best[r * top + m]));
  }
}


// ---------------------------------------------------------------------------
// Matrix-core filter for the top-`top` codes (top <= 32, d_s <= 32).
//
// Pass 1 scores 256 rows x all codes with one bf16 MFMA (16x16x32) per 16x16
// tile (codes = A from LDS, rows = B in registers) and keeps, per lane and
// row, the running maxima of M disjoint code segments; the 4 lanes holding a
// row cover 4M >= top disjoint segments.  Each maximum is an actual
// approximate score, so L = the top-th largest of those 4M maxima is a lower
// bound on the row's top-th largest approximate score.
//
// Error bound.  x~, c~ are the bf16 roundings (relative error <= 2^-9 each) and
// the MFMA sums their exact products in fp32, so
//   |approx - sum x c| <= sum|x c| (2^-8 + 2^-18) + 32 * 2^-23 sum|x~ c~|
//   |exact  - sum x c| <= 32 * 2^-24 sum|x c|        (the canonical fmaf chain)
// and with sum|x c| <= ||x|| ||c||:  |approx - exact| <= eps =
// 1.02 * 2^-8 * ||x|| * max_c ||c||.  Every code of the exact top-`top` therefore
// scores approx >= L - 2 eps.  Pass 2 re-runs the MFMAs and collects those codes:
// each lane appends the hits of its own (row, code quarter) to a private LDS
// list with a register counter (at most mf_cap per list), so no atomics and no
// LDS round trips; a lane visits the append code only for the scores that hit.
// Pass 3 rescores a row's four lists in the canonical fp32 order and keeps the
// exact top-`top` (score desc, code asc).  Rows with an overflowing list (or
// non-finite inputs) are flagged, and code_topk_rows_kernel recomputes them
// exhaustively, one wave per row.
typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float floatx4_t __attribute__((ext_vector_type(4)));

constexpr int kMfRows = 256;     // rows per block: 4 waves x 4 row tiles of 16
constexpr float kMfEps = 0.0039844f;  // 1.02 * 2^-8

__device__ __forceinline__ uint16_t bf16_rne(float f) {
  uint32_t u = __float_as_uint(f);
  u += 0x7FFFu + ((u >> 16) & 1u);
  return static_cast<uint16_t>(u >> 16);
}

__host__ __device__ inline int n_c_padded(int n_c) { return (n_c + 15) / 16 * 16; }

// Template instance per `top` (Q = 1, 2, 4, 8) and its segment maxima per lane
// and row (M).  The 4M maxima of a row must be >= top; for top <= 16, M = 2Q
// capped at 8.  For top 17..32 the screen keeps 32 per lane: with only 8 (4M =
// top) the bound L would be the smallest maximum and collect about 140 codes per
// row at N_c = 8192; with 32 it collects about 45.  mf_cap: list capacity per
// (row, code quarter).  At config 3 a row collects about 6 codes for top 4 and
// 25 for top 16 (at most 10 and 19 in one quarter in a sample of 8192 rows).
__host__ __device__ constexpr int mf_q(int top) { return top <= 4 ? 1 : top <= 8 ? 2 : top <= 16 ? 4 : 8; }
__host__ __device__ constexpr int mf_segments(int q) { return q >= 8 ? 32 : (2 * q < 8 ? 2 * q : 8); }
__host__ __device__ constexpr int mf_cap(int q) { return q <= 1 ? 16 : q <= 2 ? 20 : q <= 4 ? 24 : 32; }

// LDS: one region used first for the segment maxima ([4 waves][4M][64] fp32),
// then for the pass-3 lists ([4][top][64] u64, top > 16 only: smaller tops keep
// them in registers) followed by the pass-2 candidates ([4 waves][4 row
// tiles][mf_cap][64 lanes] u16).  The list counts stay in registers and reach
// pass 3 by cross-lane shuffles.
__host__ __device__ constexpr size_t mf_list_bytes(int top) {
  return mf_q(top) >= 8 ? static_cast<size_t>(4) * top * 64 * sizeof(uint64_t) : 0;
}
__host__ __device__ inline size_t code_topk_mfma_region(int top) {
  const size_t lists = mf_list_bytes(top);
  const size_t cand = sizeof(uint16_t) * 4 * 4 * mf_cap(mf_q(top)) * 64;
  const size_t segs = sizeof(float) * 4 * 4 * mf_segments(mf_q(top)) * 64;
  return lists + cand > segs ? lists + cand : segs;
}

__host__ __device__ inline size_t code_topk_mfma_smem(int top) { return code_topk_mfma_region(top); }

// bf16 copy of the codebook, zero-padded to [h][n_c_pad][32], and the largest
// row norm per head accumulated by atomicMax on the (non-negative) float bits
// into cmax_bits[h], which the caller zeroes first.  A non-finite entry stores
// +inf bits, which makes the bound non-finite and sends every row of that head
// to the exhaustive kernel.
__global__ __launch_bounds__(256) void codebook_prep_kernel(const float* __restrict__ chat, int n_c,
                                                            int n_c_pad, int d_s,
                                                            uint16_t* __restrict__ cbf,
                                                            uint32_t* __restrict__ cmax_bits) {
  __shared__ float red[256];
  const int hh = blockIdx.y;
  const int c = blockIdx.x * 256 + threadIdx.x;
  float nrm = 0.0f;
  if (c < n_c_pad) {
    const float* cr = chat + (static_cast<int64_t>(hh) * n_c + c) * d_s;
    uint16_t* o = cbf + (static_cast<int64_t>(hh) * n_c_pad + c) * 32;
    float nrm2 = 0.0f;
    uint16_t tmp[32];
#pragma unroll
    for (int s = 0; s < 32; ++s) {
      const float v = (c < n_c && s < d_s) ? cr[s] : 0.0f;
      nrm2 = fma_rn(v, v, nrm2);
      tmp[s] = bf16_rne(v);
    }
#pragma unroll
    for (int s4 = 0; s4 < 4; ++s4)
      reinterpret_cast<uint4*>(o)[s4] = __builtin_bit_cast(uint4, *reinterpret_cast<const uint16_t(*)[8]>(tmp + 8 * s4));
    nrm = (nrm2 <= 3.0e38f) ? sqrtf(nrm2) : INFINITY;
  }
  red[threadIdx.x] = nrm;
  __syncthreads();
  for (int w = 128; w > 0; w >>= 1) {
    if (static_cast<int>(threadIdx.x) < w) red[threadIdx.x] = fmaxf(red[threadIdx.x], red[threadIdx.x + w]);
    __syncthreads();
  }
  if (threadIdx.x == 0) atomicMax(&cmax_bits[hh], __float_as_uint(red[0]));
}

__global__ void zero_u32_kernel(uint32_t* __restrict__ p, int count) {
  const int e = blockIdx.x * blockDim.x + threadIdx.x;
  if (e < count) p[e] = 0u;
}

// NaN-propagating maximum (v_maximum3_f32 on gfx950).  Unlike fmaxf it needs no
// canonicalizing v_max of each matrix-core result first, so the screen's
// running maxima cost one instruction per two scores.  A NaN score can only
// come from a non-finite input row or code, whose group is flagged anyway.
__device__ __forceinline__ float vmax(float a, float b) { return __builtin_elementwise_maximum(a, b); }

template <int N>
__device__ __forceinline__ void sort_desc(float (&v)[N]) {
#pragma unroll
  for (int size = 2; size <= N; size <<= 1)
#pragma unroll
    for (int stride = size >> 1; stride > 0; stride >>= 1)
#pragma unroll
      for (int i = 0; i < N; ++i) {
        const int j = i ^ stride;
        if (j > i) {
          const bool desc = (i & size) == 0;
          const float a = v[i], b = v[j];
          v[i] = desc ? fmaxf(a, b) : fminf(a, b);
          v[j] = desc ? fminf(a, b) : fmaxf(a, b);
        }
      }
}

// v and w sorted descending: v becomes the N largest of v and w, sorted
// descending.  max(v[i], w[N-1-i]) holds those N values as a bitonic sequence,
// which the half-cleaner cascade sorts.
template <int N>
__device__ __forceinline__ void merge_top_desc(float (&v)[N], const float (&w)[N]) {
#pragma unroll
  for (int i = 0; i < N; ++i) v[i] = fmaxf(v[i], w[N - 1 - i]);
#pragma unroll
  for (int stride = N >> 1; stride > 0; stride >>= 1)
#pragma unroll
    for (int i = 0; i < N; ++i) {
      const int j = i ^ stride;
      if (j > i) {
        const float a = v[i], b = v[j];
        v[i] = fmaxf(a, b);
        v[j] = fminf(a, b);
      }
    }
}

// Top <= 4 fits 128 VGPRs and 36 KB of LDS: 4 blocks per CU, so the grid of a
// config-3 head set (1024 blocks) runs in one round.
// One block's 256 rows (block index blk of the grid batch * h * ceil(rows /
// 256)); the kernels below run it for their own blocks.
template <int Q>
__device__ __forceinline__ void code_topk_mfma_block(
    const float* __restrict__ xhat, int64_t rows, int h, const float* __restrict__ chat,
    const uint16_t* __restrict__ cbf, const uint32_t* __restrict__ cmax_bits, int n_c, int d_s,
    float temperature, int top, int32_t* __restrict__ codes, uint8_t* __restrict__ flags, int64_t blk) {
  constexpr int M = mf_segments(Q);  // segment maxima per lane and row
  constexpr int CAP = mf_cap(Q);
  extern __shared__ __align__(16) unsigned char smem_raw[];
  const size_t list_bytes = mf_list_bytes(top);
  uint64_t* lists = reinterpret_cast<uint64_t*>(smem_raw);               // [4][top][64] (pass 3, Q = 8)
  uint16_t* cand = reinterpret_cast<uint16_t*>(smem_raw + list_bytes);   // [4][4][CAP][64] (pass 2)

  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int q4 = lane >> 4, c16 = lane & 15;
  const int n_c_pad = n_c_padded(n_c);
  const int64_t tiles = (rows + kMfRows - 1) / kMfRows;
  const int64_t bh = udiv32(blk, tiles);  // (block indices are below 2^31)
  const int64_t r0 = (blk - bh * tiles) * kMfRows + wave * 64;
  const int hh = static_cast<int>(bh - udiv32(bh, h) * h);
  const float* xb = xhat + bh * rows * d_s;
  const uint16_t* cbh = cbf + static_cast<int64_t>(hh) * n_c_pad * 32;

  // Rows load as float4s (d_s is a multiple of 4, so a row starts 16-byte
  // aligned and a float4 lies wholly below d_s or wholly above it); all of a
  // lane's loads are issued before the first use.
  auto row4 = [&](int64_t row, int s4) -> float4 {
    return (row < rows && 4 * s4 < d_s) ? *reinterpret_cast<const float4*>(xb + row * d_s + 4 * s4)
                                        : make_float4(0.f, 0.f, 0.f, 0.f);
  };
  float4 xl[4][2];
#pragma unroll
  for (int nt = 0; nt < 4; ++nt)
#pragma unroll
    for (int j = 0; j < 2; ++j) xl[nt][j] = row4(r0 + nt * 16 + c16, 2 * q4 + j);
  float4 xe[8];
#pragma unroll
  for (int s4 = 0; s4 < 8; ++s4) xe[s4] = row4(r0 + lane, s4);
  bf16x8_t bfrag[4];
#pragma unroll
  for (int nt = 0; nt < 4; ++nt) {
    const float f[8] = {xl[nt][0].x, xl[nt][0].y, xl[nt][0].z, xl[nt][0].w,
                        xl[nt][1].x, xl[nt][1].y, xl[nt][1].z, xl[nt][1].w};
    uint16_t tmp[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) tmp[e] = bf16_rne(f[e]);
    bfrag[nt] = __builtin_bit_cast(bf16x8_t, tmp);
  }
  float eps_l = 0.0f;
  if (r0 + lane < rows) {
    float nrm2 = 0.0f;
#pragma unroll
    for (int s4 = 0; s4 < 8; ++s4) {  // entries past d_s are zero
      nrm2 = fma_rn(xe[s4].x, xe[s4].x, nrm2);
      nrm2 = fma_rn(xe[s4].y, xe[s4].y, nrm2);
      nrm2 = fma_rn(xe[s4].z, xe[s4].z, nrm2);
      nrm2 = fma_rn(xe[s4].w, xe[s4].w, nrm2);
    }
    eps_l = kMfEps * sqrtf(nrm2) * __uint_as_float(cmax_bits[hh]) * 1.0001f;
  }
  const bool bad_l = !(eps_l <= 3.0e38f);

  float smax[4][M];
#pragma unroll
  for (int nt = 0; nt < 4; ++nt)
#pragma unroll
    for (int u = 0; u < M; ++u) smax[nt][u] = -INFINITY;

  // ---- pass 1: segment maxima.  Codebook fragments come straight from the
  // (L2-resident) bf16 codebook: lane (q4, c16) reads 16 bytes of code
  // tile*16 + c16.  Each tile feeds four independent MFMAs (one per 16-row
  // tile); tile t of the codebook updates segment t % M, so one lane's segments
  // stay disjoint, which is all the bound needs.  Tiles go in groups of GT, the
  // next group's fragments loading while the current group's MFMAs run (the
  // prefetch start is clamped to the last full group, so every load is in
  // range).  Only the last tile can hold codes past n_c and is masked.
  constexpr int GT = 4;                      // tiles per load group
  constexpr int STEP = M > GT ? M : GT;      // tiles per unrolled step (segment period)
  const int ntile_full = n_c / 16;
  const int ntile = n_c_pad / 16;
  auto frag = [&](int tile) -> bf16x8_t {
    return *reinterpret_cast<const bf16x8_t*>(cbh + (static_cast<int64_t>(tile) * 16 + c16) * 32 + q4 * 8);
  };
  const int lastg = ntile_full - GT;  // first tile of the last full group (used when >= 0)
  auto loadg = [&](bf16x8_t (&a)[GT], int t) {
#pragma unroll
    for (int u = 0; u < GT; ++u) a[u] = frag(t + u);
  };
  {
    int t = 0;
    bf16x8_t a[GT];
    if (ntile_full >= GT) loadg(a, 0);
    for (; t + STEP <= ntile_full; t += STEP) {
#pragma unroll
      for (int gi = 0; gi < STEP / GT; ++gi) {
        bf16x8_t an[GT];
        loadg(an, min(t + GT * (gi + 1), lastg));
#pragma unroll
        for (int u = 0; u < GT; ++u) {
          floatx4_t sc[4];
#pragma unroll
          for (int nt = 0; nt < 4; ++nt)
            sc[nt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[u], bfrag[nt], floatx4_t{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
#pragma unroll
          for (int nt = 0; nt < 4; ++nt) {
            float& m = smax[nt][(gi * GT + u) % M];
            m = vmax(vmax(vmax(sc[nt][0], sc[nt][1]), sc[nt][2]), vmax(sc[nt][3], m));
          }
        }
#pragma unroll
        for (int u = 0; u < GT; ++u) a[u] = an[u];
      }
    }
    // the remaining tiles (fewer than STEP), the last one masked past n_c;
    // tile t still updates segment t % M
    for (; t < ntile; ++t) {
      const bf16x8_t af = frag(t);
      const int cbase = t * 16 + q4 * 4;
      const int seg = t % M;
#pragma unroll
      for (int nt = 0; nt < 4; ++nt) {
        const floatx4_t sc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(af, bfrag[nt], floatx4_t{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
        float m = -INFINITY;
#pragma unroll
        for (int e = 0; e < 4; ++e)
          if (cbase + e < n_c) m = vmax(m, sc[e]);
#pragma unroll
        for (int u = 0; u < M; ++u)
          if (u == seg) smax[nt][u] = vmax(smax[nt][u], m);
      }
    }
  }

  // L per row = top-th largest of the 4M segment maxima of its 4 lanes: the
  // maxima go through LDS (the start of the shared region, unused until pass 2)
  // so that lane r of the wave can sort row r's 4M values.
  float* segs = reinterpret_cast<float*>(smem_raw) + static_cast<size_t>(wave) * 4 * M * 64;  // [4M][64]
#pragma unroll
  for (int nt = 0; nt < 4; ++nt)
#pragma unroll
    for (int u = 0; u < M; ++u) segs[(q4 * M + u) * 64 + nt * 16 + c16] = smax[nt][u];
  __syncthreads();
  // Chunks of at most 32 values are sorted and merged keeping the largest 32
  // (top <= 32), so every register index stays static.
  float thr_l;
  {
    constexpr int C = (4 * M < 32) ? 4 * M : 32;
    float v[C];
#pragma unroll
    for (int i = 0; i < C; ++i) v[i] = segs[i * 64 + lane];
    sort_desc<C>(v);
#pragma unroll
    for (int k = 1; k < 4 * M / C; ++k) {
      float w[C];
#pragma unroll
      for (int i = 0; i < C; ++i) w[i] = segs[(k * C + i) * 64 + lane];
      sort_desc<C>(w);
      merge_top_desc<C>(v, w);
    }
    float lb = v[0];
#pragma unroll
    for (int i = 1; i < C; ++i)
      if (i == top - 1) lb = v[i];
    thr_l = lb - 2.0f * eps_l;
    // padding rows and rows with a non-finite bound collect nothing (the
    // latter are flagged for the exhaustive kernel)
    if (r0 + lane >= rows || bad_l || !(thr_l == thr_l)) thr_l = INFINITY;
  }
  __syncthreads();  // pass 2 writes candidates over other waves' maxima

  // ---- pass 2: collect codes whose approximate score reaches the threshold.
  // The MFMA starts from C = -thr of each lane's row, so it yields D = score -
  // thr (the bound below covers the extra rounding), and a score hits exactly
  // when D's sign bit is clear.  Each score costs one v_alignbit that shifts
  // that sign bit into the lane's word for its row tile: after a group of 8
  // tiles, bit 31 - (4u + e) of hits[nt] belongs to code (t0 + u) * 16 +
  // 4 q4 + e.  The set bits of the inverted words are then appended to the
  // lane's list of (row nt*16 + c16, code quarter q4) -- a few iterations per
  // group, instead of a compare and branch per score.  Past CAP entries the
  // last slot is overwritten and the count flags the row.
  floatx4_t cneg[4];
#pragma unroll
  for (int nt = 0; nt < 4; ++nt) {
    const float t = -__shfl(thr_l, nt * 16 + c16);
    cneg[nt] = floatx4_t{t, t, t, t};
  }
  uint16_t* cl = cand + static_cast<size_t>(wave) * 4 * CAP * 64 + lane;  // list nt: cl[(nt*CAP + pos)*64]
  int qc[4] = {0, 0, 0, 0};
  uint32_t bits[4];
  auto shift_in = [&](const floatx4_t& d, int nt) {
#pragma unroll
    for (int e = 0; e < 4; ++e) bits[nt] = __builtin_amdgcn_alignbit(bits[nt], __float_as_uint(d[e]), 31);
  };
  auto append = [&](int t0, bool partial) {
#pragma unroll
    for (int nt = 0; nt < 4; ++nt) {
      uint32_t hm = ~bits[nt];
      while (hm) {
        const int b = __builtin_ctz(hm);
        hm &= hm - 1u;
        const int v = 31 - b;  // 4u + e
        const int code = t0 * 16 + ((v >> 2) << 4) + 4 * q4 + (v & 3);
        if (!partial || code < n_c) {
          cl[(nt * CAP + min(qc[nt], CAP - 1)) * 64] = static_cast<uint16_t>(code);
          ++qc[nt];
        }
      }
    }
  };
  {
    int t = 0;
    bf16x8_t a[GT];
    if (ntile_full >= GT) loadg(a, 0);
    for (; t + 8 <= ntile_full; t += 8) {
#pragma unroll
      for (int nt = 0; nt < 4; ++nt) bits[nt] = 0u;
#pragma unroll
      for (int gi = 0; gi < 8 / GT; ++gi) {
        bf16x8_t an[GT];
        loadg(an, min(t + GT * (gi + 1), lastg));
#pragma unroll
        for (int u = 0; u < GT; ++u) {
          floatx4_t sc[4];
#pragma unroll
          for (int nt = 0; nt < 4; ++nt) sc[nt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[u], bfrag[nt], cneg[nt], 0, 0, 0);
#pragma unroll
          for (int nt = 0; nt < 4; ++nt) shift_in(sc[nt], nt);
        }
#pragma unroll
        for (int u = 0; u < GT; ++u) a[u] = an[u];
      }
      // every shift of the group happens here, before the append loops: left
      // to itself the compiler sinks them past the first loop and keeps the
      // group's 32 MFMA results live across it
      asm volatile("" : "+v"(bits[0]), "+v"(bits[1]), "+v"(bits[2]), "+v"(bits[3]));
      append(t, false);
    }
    if (t < ntile) {
      // the last, partial group: tiles past ntile shift in misses
#pragma unroll
      for (int nt = 0; nt < 4; ++nt) bits[nt] = 0u;
      for (int u = 0; u < 8; ++u) {
        if (t + u < ntile) {
          const bf16x8_t af = frag(t + u);
#pragma unroll
          for (int nt = 0; nt < 4; ++nt)
            shift_in(__builtin_amdgcn_mfma_f32_16x16x32_bf16(af, bfrag[nt], cneg[nt], 0, 0, 0), nt);
        } else {
#pragma unroll
          for (int nt = 0; nt < 4; ++nt) bits[nt] = (bits[nt] << 4) | 0xFu;
        }
      }
      asm volatile("" : "+v"(bits[0]), "+v"(bits[1]), "+v"(bits[2]), "+v"(bits[3]));
      append(t, true);
    }
  }
  __syncthreads();  // every wave's lists are complete

  // ---- pass 3: exact rescoring of the collected codes (one lane per row).
  // Row `lane` is row tile lane / 16, column lane % 16; its four quarter lists
  // belong to lanes q*16 + lane % 16 of that row tile.
  const int64_t row = r0 + lane;
  const int rt = lane >> 4, rc = lane & 15;
  int qn[4], m = 0;
  bool list_over = false;
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    // lane q*16 + rc holds the counts of quarter q for the four row tiles
    int c = 0;
#pragma unroll
    for (int nt = 0; nt < 4; ++nt) {
      const int v = __shfl(qc[nt], q * 16 + rc);
      c = (rt == nt) ? v : c;
    }
    qn[q] = c;
    list_over = list_over || qn[q] > CAP;
    m += qn[q];
  }
  const bool over = bad_l || list_over || m < top;
  if (row < rows && !over) {
    float xr[32];
#pragma unroll
    for (int s = 0; s < 32; ++s) xr[s] = (s < d_s) ? xb[row * d_s + s] : 0.0f;
    const float* cb = chat + static_cast<int64_t>(hh) * n_c * d_s;
    // The temperature division as a compile-time choice: left to a runtime
    // flag the compiler computed the division for every code and selected.
    auto rescore = [&](auto scale_c) {
      const uint16_t* rl = cand + (static_cast<size_t>(wave) * 4 + rt) * CAP * 64 + rc;
      const int b1 = qn[0], b2 = b1 + qn[1], b3 = b2 + qn[2];  // list starts in row order
      auto code_at = [&](int i) -> int {  // entry i of the row: list q, position j
        const int q = (i >= b1 ? 1 : 0) + (i >= b2 ? 1 : 0) + (i >= b3 ? 1 : 0);
        const int j = i - (q == 0 ? 0 : q == 1 ? b1 : q == 2 ? b2 : b3);
        return rl[(j * 64) + q * 16];
      };
      auto code_row = [&](int c, float4 (&cv)[8]) {
        const float4* cr = reinterpret_cast<const float4*>(cb + static_cast<int64_t>(c) * d_s);
#pragma unroll
        for (int s4 = 0; s4 < 8; ++s4) cv[s4] = (s4 * 4 < d_s) ? cr[s4] : make_float4(0.f, 0.f, 0.f, 0.f);
      };
      auto exact_key = [&](int c, const float4 (&cv)[8]) -> uint64_t {
        float acc = 0.0f;
#pragma unroll
        for (int s4 = 0; s4 < 8; ++s4) {
          if (s4 * 4 < d_s) {
            acc = fma_rn(xr[s4 * 4 + 0], cv[s4].x, acc);
            acc = fma_rn(xr[s4 * 4 + 1], cv[s4].y, acc);
            acc = fma_rn(xr[s4 * 4 + 2], cv[s4].z, acc);
            acc = fma_rn(xr[s4 * 4 + 3], cv[s4].w, acc);
          }
        }
        if constexpr (decltype(scale_c)::value) acc = acc / temperature;
        return composite_key(acc, static_cast<uint32_t>(c));
      };
      // One code row in flight per lane (a second buffer would hold 32 more
      // VGPRs for the whole kernel; the other resident waves cover the latency).
      int c = code_at(0);
      float4 cv[8];
      code_row(c, cv);
      int32_t* out = codes + (bh * rows + row) * top;
      if constexpr (Q <= 4) {
        // top <= 16: a sorted register list (static indices), insertion by a
        // compare-and-shift pass from the bottom
        constexpr int TM = 4 * Q;
        uint64_t best[TM];
#pragma unroll
        for (int p = 0; p < TM; ++p) best[p] = 0ull;  // below every key
        for (int i = 0; i < m; ++i) {
          if (i > 0) { c = code_at(i); code_row(c, cv); }
          const uint64_t key = exact_key(c, cv);
#pragma unroll
          for (int p = TM - 1; p > 0; --p) best[p] = key > best[p - 1] ? best[p - 1] : (key > best[p] ? key : best[p]);
          best[0] = key > best[0] ? key : best[0];
        }
#pragma unroll
        for (int p = 0; p < TM; ++p)
          if (p < top) out[p] = static_cast<int32_t>(key_index(best[p]));
      } else {
        uint64_t* my = lists + static_cast<int64_t>(wave) * top * 64 + lane;  // entry p at my[p * 64]
        int nb = 0;
        for (int i = 0; i < m; ++i) {
          const int cn = code_at(min(i + 1, m - 1));
          float4 cvn[8];
          code_row(cn, cvn);
          const uint64_t key = exact_key(c, cv);
          c = cn;
#pragma unroll
          for (int s4 = 0; s4 < 8; ++s4) cv[s4] = cvn[s4];
          if (nb == top && key <= my[(top - 1) * 64]) continue;
          int p = (nb < top) ? nb++ : top - 1;
          while (p > 0 && my[(p - 1) * 64] < key) {
            my[p * 64] = my[(p - 1) * 64];
            --p;
          }
          my[p * 64] = key;
        }
        for (int p = 0; p < top; ++p) out[p] = static_cast<int32_t>(key_index(my[p * 64]));
      }
  
    };
    if (temperature != 1.0f) rescore(std::true_type{});
    else rescore(std::false_type{});
}
  if (row < rows) flags[bh * rows + row] = over ? 1 : 0;
}

template <int Q>
__global__ __launch_bounds__(256, Q == 1 ? 4 : 1) void code_topk_mfma_kernel(
    const float* __restrict__ xhat, int64_t rows, int h, const float* __restrict__ chat,
    const uint16_t* __restrict__ cbf, const uint32_t* __restrict__ cmax_bits, int n_c, int d_s,
    float temperature, int top, int32_t* __restrict__ codes, uint8_t* __restrict__ flags) {
  code_topk_mfma_block<Q>(xhat, rows, h, chat, cbf, cmax_bits, n_c, d_s, temperature, top, codes, flags,
                          blockIdx.x);
}

// The query screen (blocks [0, grid_a)) and the key screen (the rest) in one
// launch: the query screen's grid fills 4/3 of the blocks a CU holds at once,
// and the key screen's blocks then run in what its last round leaves idle.
template <int QA, int QB>
__global__ __launch_bounds__(256, 1) void code_topk_mfma_pair_kernel(
    const float* __restrict__ xa, const float* __restrict__ xb, int64_t rows, int h,
    const float* __restrict__ chat, const uint16_t* __restrict__ cbf, const uint32_t* __restrict__ cmax_bits,
    int n_c, int d_s, float temperature, int top_a, int top_b, int32_t* __restrict__ codes_a,
    int32_t* __restrict__ codes_b, uint8_t* __restrict__ flags_a, uint8_t* __restrict__ flags_b,
    int64_t grid_a) {
  // Logical block L: (batch, kv head) L / (2T), then that head's T query blocks
  // and T key blocks (T row tiles per head).  xcd_block gives XCD x the
  // contiguous range [x per, (x + 1) per), so one XCD's L2 holds the bf16 and
  // fp32 codebooks of about one head instead of a slice of every head's.
  const int64_t tiles = (rows + kMfRows - 1) / kMfRows;
  const int64_t lb = xcd_block(blockIdx.x, xcd_per(2 * grid_a));
  if (lb >= 2 * grid_a) return;
  const int64_t bh = udiv32(lb, 2 * tiles), i = lb - bh * 2 * tiles;
  if (i < tiles)
    code_topk_mfma_block<QA>(xa, rows, h, chat, cbf, cmax_bits, n_c, d_s, temperature, top_a, codes_a, flags_a,
                             bh * tiles + i);
  else
    code_topk_mfma_block<QB>(xb, rows, h, chat, cbf, cmax_bits, n_c, d_s, temperature, top_b, codes_b, flags_b,
                             bh * tiles + i - tiles);
}

// Exact top-`top` codes of the rows flagged by the matrix-core filter
// (flags[bh * rows + row] != 0), one wave per row: lane l scores codes l, l + 64,
// ... in the canonical fp32 order (one fmaf chain over d_s, then / temperature)
// and keeps its best TM composite keys in a sorted register list; `top` rounds
// of a wave-wide maximum then take the row's keys in descending order.  The
// result is the top-`top` by (score desc, code asc), as code_topk_kernel gives.
// Each wave scans the flags of 64 consecutive rows per step, so unflagged rows
// cost one byte read.
template <int TM>
__global__ __launch_bounds__(256) void code_topk_rows_kernel(const float* __restrict__ xhat, int64_t total,
                                                             int64_t rows, int h, const float* __restrict__ chat,
                                                             int n_c, int d_s, float temperature, int top,
                                                             int32_t* __restrict__ codes,
                                                             const uint8_t* __restrict__ flags) {
  const int lane = threadIdx.x & 63;
  const int64_t gw = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
  const int64_t nw = static_cast<int64_t>(gridDim.x) * 4;
  const bool scale = (temperature != 1.0f);
  for (int64_t base = gw * 64; base < total; base += nw * 64) {
    const bool f = base + lane < total && flags[base + lane] != 0;
    for (uint64_t m = __ballot(f); m != 0ull; m &= m - 1ull) {
      const int64_t grow = base + (__ffsll(static_cast<long long>(m)) - 1);  // bh * rows + row
      const int hh = static_cast<int>((grow / rows) % h);
      const float* xr = xhat + grow * d_s;
      const float* cb = chat + static_cast<int64_t>(hh) * n_c * d_s;
      float x[32];
#pragma unroll
      for (int s = 0; s < 32; ++s) x[s] = (s < d_s) ? xr[s] : 0.0f;
      uint64_t best[TM];
#pragma unroll
      for (int p = 0; p < TM; ++p) best[p] = 0ull;  // below every key
      auto insert = [&](uint64_t key) {
#pragma unroll
        for (int p = TM - 1; p > 0; --p) best[p] = key > best[p - 1] ? best[p - 1] : (key > best[p] ? key : best[p]);
        best[0] = key > best[0] ? key : best[0];
      };
      auto load = [&](int c, float4 (&cv)[8]) {
        const float4* cr = reinterpret_cast<const float4*>(cb + static_cast<int64_t>(c) * d_s);
#pragma unroll
        for (int s4 = 0; s4 < 8; ++s4) cv[s4] = (s4 * 4 < d_s) ? cr[s4] : make_float4(0.f, 0.f, 0.f, 0.f);
      };
      auto key_of = [&](int c, const float4 (&cv)[8]) -> uint64_t {
        float acc = 0.0f;
#pragma unroll
        for (int s4 = 0; s4 < 8; ++s4) {
          if (s4 * 4 < d_s) {
            acc = fma_rn(x[s4 * 4 + 0], cv[s4].x, acc);
            acc = fma_rn(x[s4 * 4 + 1], cv[s4].y, acc);
            acc = fma_rn(x[s4 * 4 + 2], cv[s4].z, acc);
            acc = fma_rn(x[s4 * 4 + 3], cv[s4].w, acc);
          }
        }
        if (scale) acc = acc / temperature;
        return composite_key(acc, static_cast<uint32_t>(c));
      };
      // two codes per step, both code rows in flight before either is scored
      for (int c = lane; c < n_c; c += 128) {
        const bool two = c + 64 < n_c;
        float4 cv0[8], cv1[8];
        load(c, cv0);
        load(two ? c + 64 : c, cv1);
        insert(key_of(c, cv0));
        if (two) insert(key_of(c + 64, cv1));
      }
      int32_t* out = codes + grow * top;
      for (int p = 0; p < top; ++p) {
        uint64_t v = best[0];
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) {
          const uint32_t lo = static_cast<uint32_t>(__shfl_xor(static_cast<int>(v & 0xFFFFFFFFull), o));
          const uint32_t hi = static_cast<uint32_t>(__shfl_xor(static_cast<int>(v >> 32), o));
          const uint64_t w = (static_cast<uint64_t>(hi) << 32) | lo;
          v = w > v ? w : v;
        }
        const bool win = best[0] == v;  // keys are distinct, so one lane holds v
#pragma unroll
        for (int q = 0; q < TM - 1; ++q) best[q] = win ? best[q + 1] : best[q];
        best[TM - 1] = win ? 0ull : best[TM - 1];
        if (lane == 0) out[p] = static_cast<int32_t>(key_index(v));
      }
    }
  }
}

// Few rows (decoding): one block per (batch, output head, row).  W [d_s][d]
// (rows padded to d + 1 floats: no bank conflicts) and the group's x rows are
// staged in LDS; wave w runs the chains of heads w, w + 4, ..., lane s the
// chain of coordinate s (t ascending), so the group's heads run in parallel;
// wave 0 then adds the heads in order, divides by group and runs the norm
// chain over s on the broadcast coordinates.  Same arithmetic as the
// row-parallel kernels above, which stay in charge of calls with many rows.
constexpr int64_t kLaneRowsMax = 256;

__host__ __device__ inline size_t route_few_smem(int group, int d, int d_s) {
  return sizeof(float) * (static_cast<size_t>(d_s) * (d + 1) + static_cast<size_t>(group) * d +
                          static_cast<size_t>(group) * 64);
}

// One routing task of route_vectors_few_kernel (blockIdx.y picks the task, so
// the queries and the keys of a decoding step route in one launch).
struct FewRoute {
  const void* x;
  int64_t n, sb, sn, sh, rows;  // rows = batch * (h_in / group) * n
  int h_in, group, d, d_s;
  const float* w;
  float* out;
};

template <typename T>
__global__ __launch_bounds__(256) void route_vectors_few_kernel(FewRoute t0, FewRoute t1) {
  extern __shared__ __align__(16) float few_lds[];
  const FewRoute& a = blockIdx.y ? t1 : t0;
  const int64_t row = blockIdx.x;  // (b * h_out + h) * n + i
  if (row >= a.rows) return;
  const int d = a.d, d_s = a.d_s, group = a.group;
  float* wl = few_lds;                                              // [d_s][d + 1]
  float* xl = wl + static_cast<size_t>(d_s) * (d + 1);              // [group][d]
  float* part = xl + static_cast<size_t>(group) * d;                // [group][64]
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int h_out = a.h_in / group;
  const int64_t i = row % a.n;
  const int64_t bh = row / a.n;
  const int h = static_cast<int>(bh % h_out);
  const int64_t b = bh / h_out;
  const T* x = static_cast<const T*>(a.x);
  strided_batches<16, 256>(
      static_cast<int64_t>(d_s) * d, tid, [&](int64_t e) { return a.w[e]; },
      [&](int64_t e, float v) { wl[(e / d) * (d + 1) + e % d] = v; });
  const T* xrow = x + b * a.sb + i * a.sn + static_cast<int64_t>(h * group) * a.sh;
  strided_batches<4, 256>(
      static_cast<int64_t>(group) * d, tid,
      [&](int64_t e) { return ld(xrow + (e / d) * a.sh + e % d); }, [&](int64_t e, float v) { xl[e] = v; });
  __syncthreads();
  if (lane < d_s) {
    const float* wr = wl + static_cast<size_t>(lane) * (d + 1);
    for (int gg = wave; gg < group; gg += 4) {
      const float* xr = xl + static_cast<size_t>(gg) * d;
      float acc = 0.0f;
      for (int t = 0; t < d; ++t) acc = fma_rn(xr[t], wr[t], acc);
      part[gg * 64 + lane] = acc;
    }
  }
  __syncthreads();
  if (wave != 0) return;
  float sum = 0.0f;
  if (lane < d_s) {
    sum = part[lane];
    for (int gg = 1; gg < group; ++gg) sum = sum + part[gg * 64 + lane];
  }
  const float v = sum / static_cast<float>(group);
  float nrm = 0.0f;
  for (int s2 = 0; s2 < d_s; ++s2) {
    const float vs = __shfl(v, s2);
    nrm = fma_rn(vs, vs, nrm);
  }
  const float den = fmaxf(sqrtf(nrm), 1e-12f);
  if (lane < d_s) a.out[row * d_s + lane] = v / den;
}

int launch_route_few(const FewRoute& t0, const FewRoute& t1, int dtype, hipStream_t st) {
  const size_t smem = std::max(route_few_smem(t0.group, t0.d, t0.d_s),
                               t1.rows > 0 ? route_few_smem(t1.group, t1.d, t1.d_s) : size_t(0));
  const dim3 grid(static_cast<unsigned>(std::max(t0.rows, t1.rows)), t1.rows > 0 ? 2u : 1u);
  if (dtype == SSA_DTYPE_BF16) route_vectors_few_kernel<uint16_t><<<grid, 256, smem, st>>>(t0, t1);
  else route_vectors_few_kernel<float><<<grid, 256, smem, st>>>(t0, t1);
  return check_launch("route_vectors_few_kernel");
}

int next_pow2(int v) {
  int p = 1;
  while (p < v) p <<= 1;
  return p;
}

size_t route_vectors_smem(int d, int d_s) {
  const int dsp = next_pow2(d_s);
  const int rb = (kRouteThreads / dsp) * kRouteRowsPerThread;
  return sizeof(float) * (static_cast<size_t>(d_s) * (d + 4) + static_cast<size_t>(rb) * (d + 4) +
                          static_cast<size_t>(rb) * d_s);
}

int check_route_vectors(int dtype, int64_t batch, int64_t n, int h_in, int group, int d, int d_s) {
  if (dtype != SSA_DTYPE_F32 && dtype != SSA_DTYPE_BF16)
    return fail(SSA_ERR_UNSUPPORTED, "route_vectors: dtype %d not supported (f32, bf16)", dtype);
  if (batch < 0 || n < 0 || h_in <= 0 || group <= 0 || d <= 0 || d_s <= 0)
    return fail(SSA_ERR_INVALID_ARGUMENT, "route_vectors: non-positive shape");
  if (h_in % group != 0)
    return fail(SSA_ERR_INVALID_ARGUMENT, "num_q_heads must be divisible by num_kv_heads");
  if (d % 4 != 0 || d_s > 256)
    return fail(SSA_ERR_UNSUPPORTED, "route_vectors: need head_dim %% 4 == 0 and route_dim <= 256");
  if (route_vectors_smem(d, d_s) > 64 * 1024)
    return fail(SSA_ERR_UNSUPPORTED, "route_vectors: head_dim*route_dim too large for LDS");
  return SSA_OK;
}

int launch_route_vectors(const void* x, int dtype, int64_t batch, int64_t n, int h_in, int group,
                         int d, int64_t sb, int64_t sn, int64_t sh, const float* w, int d_s,
                         float* out, hipStream_t st) {
  if (batch == 0 || n == 0) return SSA_OK;
  const int esz = (dtype == SSA_DTYPE_BF16) ? 2 : 4;
  const bool vec4 = (sb % 4 == 0) && (sn % 4 == 0) && (sh % 4 == 0) &&
                    (reinterpret_cast<uintptr_t>(x) % (4 * esz) == 0) &&
                    (reinterpret_cast<uintptr_t>(w) % 16 == 0);
  // 16-byte pieces of 8 elements: element strides and the base aligned to them
  const int64_t pe = 16 / esz;
  const bool piece8 = (d % 8 == 0) && (sb % pe == 0) && (sn % pe == 0) && (sh % pe == 0) &&
                      (reinterpret_cast<uintptr_t>(x) % 16 == 0);
  const int64_t total = batch * (h_in / group) * n;
  if (d_s <= 64 && total <= kLaneRowsMax && route_few_smem(group, d, d_s) <= 64 * 1024) {
    const FewRoute t0{x, n, sb, sn, sh, total, h_in, group, d, d_s, w, out};
    FewRoute none{};
    return launch_route_few(t0, none, dtype, st);
  }
  if (d_s == 32 && piece8 && group > 1) {
    const int64_t grid = batch * (h_in / group) * ceil_div(n, kRsRows);
    if (dtype == SSA_DTYPE_BF16)
      if (d == 128)
        route_vectors_split_kernel<uint16_t, 128><<<dim3(static_cast<unsigned>(grid)), 256, 0, st>>>(
            static_cast<const uint16_t*>(x), n, h_in, group, d, sb, sn, sh, w, out);
      else
        route_vectors_split_kernel<uint16_t, 0><<<dim3(static_cast<unsigned>(grid)), 256, 0, st>>>(
            static_cast<const uint16_t*>(x), n, h_in, group, d, sb, sn, sh, w, out);
    else
      route_vectors_split_kernel<float, 0><<<dim3(static_cast<unsigned>(grid)), 256, 0, st>>>(
          static_cast<const float*>(x), n, h_in, group, d, sb, sn, sh, w, out);
    return check_launch("route_vectors_split_kernel");
  }
  if (d_s == 32 && piece8 && group == 1 && dtype == SSA_DTYPE_BF16 && d == 128) {
    const int64_t grid = batch * h_in * ceil_div(n, kRhRows);
    route_vectors_half_kernel<128><<<dim3(static_cast<unsigned>(grid)), 128, 0, st>>>(
        static_cast<const uint16_t*>(x), n, h_in, sb, sn, sh, w, out);
    return check_launch("route_vectors_half_kernel");
  }
  if (d_s == 32 && piece8) {
    const int64_t grid = batch * (h_in / group) * ceil_div(n, kRrThreads);
    if (dtype == SSA_DTYPE_BF16)
      route_vectors_row_kernel<uint16_t, 0><<<dim3(static_cast<unsigned>(grid)), kRrThreads, 0, st>>>(
          static_cast<const uint16_t*>(x), n, h_in, group, d, sb, sn, sh, w, out);
    else
      route_vectors_row_kernel<float, 0><<<dim3(static_cast<unsigned>(grid)), kRrThreads, 0, st>>>(
          static_cast<const float*>(x), n, h_in, group, d, sb, sn, sh, w, out);
    return check_launch("route_vectors_row_kernel");
  }
  if (d_s <= 32 && vec4 && route_vectors_tile_smem(d) <= 64 * 1024) {
    const int64_t grid = batch * (h_in / group) * ceil_div(n, kRvRows);
    const size_t smem = route_vectors_tile_smem(d);
    if (dtype == SSA_DTYPE_BF16)
      route_vectors_tile_kernel<uint16_t><<<dim3(static_cast<unsigned>(grid)), 256, smem, st>>>(
          static_cast<const uint16_t*>(x), n, h_in, group, d, sb, sn, sh, w, d_s, out);
    else
      route_vectors_tile_kernel<float><<<dim3(static_cast<unsigned>(grid)), 256, smem, st>>>(
          static_cast<const float*>(x), n, h_in, group, d, sb, sn, sh, w, d_s, out);
    return check_launch("route_vectors_tile_kernel");
  }
  const int dsp = next_pow2(d_s);
  const int rb = (kRouteThreads / dsp) * kRouteRowsPerThread;
  const int64_t grid = batch * (h_in / group) * ceil_div(n, rb);
  const size_t smem = route_vectors_smem(d, d_s);
  if (dtype == SSA_DTYPE_BF16)
    route_vectors_kernel<uint16_t><<<dim3(static_cast<unsigned>(grid)), kRouteThreads, smem, st>>>(
        static_cast<const uint16_t*>(x), n, h_in, group, d, sb, sn, sh, w, d_s, dsp, out);
  else
    route_vectors_kernel<float><<<dim3(static_cast<unsigned>(grid)), kRouteThreads, smem, st>>>(
        static_cast<const float*>(x), n, h_in, group, d, sb, sn, sh, w, d_s, dsp, out);
  return check_launch("route_vectors_kernel");
}

int check_code_topk(int64_t batch, int h, int64_t rows, int n_c, int d_s, float temperature,
                    int top) {
  if (batch < 0 || h <= 0 || rows < 0 || n_c <= 0 || d_s <= 0)
    return fail(SSA_ERR_INVALID_ARGUMENT, "code_topk: non-positive shape");
  if (top <= 0 || top > n_c)
    return fail(SSA_ERR_INVALID_ARGUMENT, "code_topk: top=%d must be in [1, num_codebook=%d]",
                top, n_c);
  if (top > 64) return fail(SSA_ERR_UNSUPPORTED, "code_topk: top=%d > 64", top);
  if (d_s > 128) return fail(SSA_ERR_UNSUPPORTED, "code_topk: route_dim %d > 128", d_s);
  if (!(temperature > 0.0f)) return fail(SSA_ERR_INVALID_ARGUMENT, "temperature must be > 0");
  return SSA_OK;
}

// Workspace of the matrix-core path: bf16 codebook, per-head max norm, and a
// fallback flag per 64-row group.
// Exact top-`top` codes of a handful of rows (decoding): one block of 1024
// threads per row (blockIdx.y picks one of two tasks, so the queries' and
// keys' codes come from one launch).  Thread t scores codes t, t + 1024, ...
// in the canonical fp32 order and keeps its best TM composite keys; each wave
// then takes its top `top` by `top` rounds of a wave-wide maximum, and wave 0
// merges the waves' lists the same way: the row's keys in descending order
// (score desc, code asc), as code_topk_kernel orders them.
constexpr int kFewThreads = 1024;
constexpr int kFewWaves = kFewThreads / 64;

struct FewTopk {
  const float* xhat;  // [total][d_s]
  int64_t rows, total;  // rows per (batch, head); total = batch * h * rows
  int top;
  int32_t* codes;     // [total][top]
};

template <int TM>
__device__ __forceinline__ void keep_top(uint64_t (&best)[TM], uint64_t key) {
#pragma unroll
  for (int p = TM - 1; p > 0; --p) best[p] = key > best[p - 1] ? best[p - 1] : (key > best[p] ? key : best[p]);
  best[0] = key > best[0] ? key : best[0];
}

// Pops the wave's largest head entry: returns it (in every lane) and removes
// it from the lane that holds it (keys are distinct).
template <int TM>
__device__ __forceinline__ uint64_t wave_pop_max(uint64_t (&best)[TM]) {
  uint64_t v = best[0];
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    const uint32_t lo = static_cast<uint32_t>(__shfl_xor(static_cast<int>(v & 0xFFFFFFFFull), o));
    const uint32_t hi = static_cast<uint32_t>(__shfl_xor(static_cast<int>(v >> 32), o));
    const uint64_t w = (static_cast<uint64_t>(hi) << 32) | lo;
    v = w > v ? w : v;
  }
  const bool win = best[0] == v;
#pragma unroll
  for (int q = 0; q < TM - 1; ++q) best[q] = win ? best[q + 1] : best[q];
  best[TM - 1] = win ? 0ull : best[TM - 1];
  return v;
}

template <int TM>
__global__ __launch_bounds__(kFewThreads) void code_topk_few_kernel(FewTopk t0, FewTopk t1, int h,
                                                                    const float* __restrict__ chat, int n_c,
                                                                    int d_s, float temperature) {
  __shared__ uint64_t s_top[kFewWaves][TM];
  const FewTopk& a = blockIdx.y ? t1 : t0;
  const int64_t grow = blockIdx.x;  // bh * rows + row
  if (grow >= a.total) return;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int top = a.top;
  const int hh = static_cast<int>((grow / a.rows) % h);
  const float* xr = a.xhat + grow * d_s;
  const float* cb = chat + static_cast<int64_t>(hh) * n_c * d_s;
  const bool scale = (temperature != 1.0f);
  float x[32];
#pragma unroll
  for (int s = 0; s < 32; ++s) x[s] = (s < d_s) ? xr[s] : 0.0f;
  uint64_t best[TM];
#pragma unroll
  for (int p = 0; p < TM; ++p) best[p] = 0ull;  // below every key
  for (int c = tid; c < n_c; c += kFewThreads) {
    const float4* cr = reinterpret_cast<const float4*>(cb + static_cast<int64_t>(c) * d_s);
    float4 cv[8];
#pragma unroll
    for (int s4 = 0; s4 < 8; ++s4) cv[s4] = (s4 * 4 < d_s) ? cr[s4] : make_float4(0.f, 0.f, 0.f, 0.f);
    float acc = 0.0f;
#pragma unroll
    for (int s4 = 0; s4 < 8; ++s4) {
      if (s4 * 4 < d_s) {
        acc = fma_rn(x[s4 * 4 + 0], cv[s4].x, acc);
        acc = fma_rn(x[s4 * 4 + 1], cv[s4].y, acc);
        acc = fma_rn(x[s4 * 4 + 2], cv[s4].z, acc);
        acc = fma_rn(x[s4 * 4 + 3], cv[s4].w, acc);
      }
    }
    if (scale) acc = acc / temperature;
    keep_top<TM>(best, composite_key(acc, static_cast<uint32_t>(c)));
  }
  // each wave's top `top`, then wave 0 merges the waves' lists
  for (int p = 0; p < TM; ++p) {
    const uint64_t v = (p < top) ? wave_pop_max<TM>(best) : 0ull;
    if (lane == 0) s_top[wave][p] = v;
  }
  __syncthreads();
  if (wave != 0) return;
#pragma unroll
  for (int p = 0; p < TM; ++p) best[p] = 0ull;
  for (int e = lane; e < kFewWaves * TM; e += 64) keep_top<TM>(best, s_top[e / TM][e % TM]);
  int32_t* out = a.codes + grow * top;
  for (int p = 0; p < top; ++p) {
    const uint64_t v = wave_pop_max<TM>(best);
    if (lane == 0) out[p] = static_cast<int32_t>(key_index(v));
  }
}

int launch_topk_few(const FewTopk& t0, const FewTopk& t1, int h, const float* chat, int n_c, int d_s,
                    float temperature, hipStream_t st) {
  const int top = std::max(t0.top, t1.total > 0 ? t1.top : 0);
  const dim3 grid(static_cast<unsigned>(std::max(t0.total, t1.total)), t1.total > 0 ? 2u : 1u);
  if (top <= 4) code_topk_few_kernel<4><<<grid, kFewThreads, 0, st>>>(t0, t1, h, chat, n_c, d_s, temperature);
  else if (top <= 8) code_topk_few_kernel<8><<<grid, kFewThreads, 0, st>>>(t0, t1, h, chat, n_c, d_s, temperature);
  else if (top <= 16) code_topk_few_kernel<16><<<grid, kFewThreads, 0, st>>>(t0, t1, h, chat, n_c, d_s, temperature);
  else code_topk_few_kernel<32><<<grid, kFewThreads, 0, st>>>(t0, t1, h, chat, n_c, d_s, temperature);
  return check_launch("code_topk_few_kernel");
}

// Decoding's few rows, in two launches that spread the codebook over the chip
// (one block reading a head's whole codebook is bound by the requests a
// single CU keeps in flight).
//   1. code_scores_few_kernel: block (head, 256-code chunk) loads its codes
//      once and writes score_key(score) of each code for every row of that
//      head in both tasks: scores [row][n_c], canonical fp32 order.
//   2. code_select_few_kernel: one block per row holds the row's n_c keys
//      in registers.  The top-th largest of the threads' maxima bounds the
//      row's top-th key from below; the keys at or above it (about `top`)
//      are ranked exactly against each other.  When too many keys pass
//      (the best keys crowd into few threads) a radix select over the score
//      bits finds the threshold instead (8-bit digits, most significant
//      first; ties on the score at the threshold go to the lowest codes,
//      counted in code order by a block scan).  The row's `top` codes are
//      written in descending key order (score desc, code asc).
struct FewScore {
  const float* xhat;    // [total][d_s]
  int64_t rows, total;  // rows per (batch, head); total = batch * h * rows
  int top;
  uint32_t* scores;     // [total][n_c]
  int32_t* codes;       // [total][top]
};

constexpr int kScoreChunk = 256;
constexpr int kFewSelThreads = 256;
constexpr int kFewSelMaxCodes = 16384;  // n_c keys of 4 bytes in 64 KB of LDS

__global__ __launch_bounds__(kScoreChunk) void code_scores_few_kernel(FewScore t0, FewScore t1, int h,
                                                                      const float* __restrict__ chat,
                                                                      int n_c, int d_s, float temperature) {
  const int hh = blockIdx.x;
  const int c = blockIdx.y * kScoreChunk + threadIdx.x;
  if (c >= n_c) return;
  const float4* cr = reinterpret_cast<const float4*>(chat + (static_cast<int64_t>(hh) * n_c + c) * d_s);
  float4 cv[8];
#pragma unroll
  for (int s4 = 0; s4 < 8; ++s4) cv[s4] = (s4 * 4 < d_s) ? cr[s4] : make_float4(0.f, 0.f, 0.f, 0.f);
  const bool scale = (temperature != 1.0f);
  for (int task = 0; task < 2; ++task) {
    const FewScore& a = task ? t1 : t0;
    if (a.total == 0) continue;
    const int64_t nb = a.total / (a.rows * h);
    for (int64_t b = 0; b < nb; ++b) {
      for (int64_t i = 0; i < a.rows; ++i) {
        const int64_t grow = (b * h + hh) * a.rows + i;
        const float* x = a.xhat + grow * d_s;
        float acc = 0.0f;
#pragma unroll
        for (int s4 = 0; s4 < 8; ++s4) {
          if (s4 * 4 < d_s) {
            acc = fma_rn(x[s4 * 4 + 0], cv[s4].x, acc);
            acc = fma_rn(x[s4 * 4 + 1], cv[s4].y, acc);
            acc = fma_rn(x[s4 * 4 + 2], cv[s4].z, acc);
            acc = fma_rn(x[s4 * 4 + 3], cv[s4].w, acc);
          }
        }
        if (scale) acc = acc / temperature;
        a.scores[grow * n_c + c] = score_key(acc);
      }
    }
  }
}

constexpr int kFewCandMax = 256;

template <int KPT>  // keys per thread: n_c <= KPT * kFewSelThreads
__global__ __launch_bounds__(kFewSelThreads) void code_select_few_kernel(FewScore t0, FewScore t1, int n_c) {
  extern __shared__ __align__(16) uint32_t few_keys[];  // [n_c] (for the radix select)
  __shared__ uint64_t s_max[kFewSelThreads];
  __shared__ uint64_t s_cand[kFewCandMax];
  __shared__ uint64_t s_thr;
  __shared__ uint32_t hist[256];
  __shared__ uint32_t s_wsum[kFewSelThreads / 64];
  __shared__ uint32_t s_lo[kFewSelThreads / 64], s_hi[kFewSelThreads / 64];
  __shared__ uint32_t s_prefix, s_need, s_cnt, s_nsel;
  const FewScore& a = blockIdx.y ? t1 : t0;
  const int64_t grow = blockIdx.x;
  if (grow >= a.total) return;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int top = a.top;
  const uint32_t* src = a.scores + grow * n_c;
  int32_t* out = a.codes + grow * top;
  // thread t holds codes t, t + 256, ... (loads clamped in bounds, all issued at once)
  uint32_t u[KPT];
#pragma unroll
  for (int j = 0; j < KPT; ++j) u[j] = src[min(tid + j * kFewSelThreads, n_c - 1)];
  const auto key_of = [](uint32_t v, int c) {
    return (static_cast<uint64_t>(v) << 32) | static_cast<uint64_t>(0xFFFFFFFFu - static_cast<uint32_t>(c));
  };
  uint64_t best = 0ull;
#pragma unroll
  for (int j = 0; j < KPT; ++j) {
    const int c = tid + j * kFewSelThreads;
    if (c < n_c) {
      few_keys[c] = u[j];
      const uint64_t k = key_of(u[j], c);
      best = k > best ? k : best;
    }
  }
  s_max[tid] = best;
  if (tid == 0) s_cnt = 0u;
  __syncthreads();
  // The top-th largest of the threads' maxima, T, has `top` keys at or above
  // it, so the row's top-th largest key is >= T: the keys >= T are the
  // candidates (about `top` of them unless the best keys crowd into a few
  // threads).  At least `top` threads hold keys (n_c >= top), so exactly one
  // thread's maximum has rank top - 1.
  int r = 0;
#pragma unroll 16
  for (int i = 0; i < kFewSelThreads; ++i) r += (s_max[i] > best) ? 1 : 0;
  if (best != 0ull && r == top - 1) s_thr = best;
  __syncthreads();
  const uint64_t thr = s_thr;
#pragma unroll
  for (int j = 0; j < KPT; ++j) {
    const int c = tid + j * kFewSelThreads;
    const uint64_t k = key_of(u[j], c);
    if (c < n_c && k >= thr) {
      const uint32_t slot = atomicAdd(&s_cnt, 1u);
      if (slot < kFewCandMax) s_cand[slot] = k;
    }
  }
  __syncthreads();
  const uint32_t cnt = s_cnt;
  if (cnt <= kFewCandMax) {
    if (tid < static_cast<int>(cnt)) {
      const uint64_t k = s_cand[tid];
      int rk = 0;
      for (uint32_t j = 0; j < cnt; ++j) rk += (s_cand[j] > k) ? 1 : 0;
      if (rk < top) out[rk] = static_cast<int32_t>(key_index(k));
    }
    return;
  }

  // Too many candidates: radix select of the top-th largest score key over
  // the row in LDS.  The bits every key shares are known from the row's
  // minimum and maximum; the digits start below them.
  uint32_t lo = 0xFFFFFFFFu, hi = 0u;
#pragma unroll
  for (int j = 0; j < KPT; ++j) {
    if (tid + j * kFewSelThreads < n_c) {
      lo = min(lo, u[j]);
      hi = max(hi, u[j]);
    }
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    lo = min(lo, static_cast<uint32_t>(__shfl_xor(static_cast<int>(lo), o)));
    hi = max(hi, static_cast<uint32_t>(__shfl_xor(static_cast<int>(hi), o)));
  }
  if (lane == 0) {
    s_lo[wave] = lo;
    s_hi[wave] = hi;
  }
  if (tid == 0) s_nsel = 0u;
  __syncthreads();
#pragma unroll
  for (int w = 0; w < kFewSelThreads / 64; ++w) {
    lo = min(lo, s_lo[w]);
    hi = max(hi, s_hi[w]);
  }
  int rem = (lo == hi) ? 0 : 32 - __clz(lo ^ hi);
  uint32_t mask = (rem == 32) ? 0u : ~((1u << rem) - 1u);
  uint32_t prefix = hi & mask, need = static_cast<uint32_t>(top);
  while (rem > 0) {
    const int shift = rem > 8 ? rem - 8 : 0;
    hist[tid] = 0u;
    __syncthreads();
#pragma unroll
    for (int j = 0; j < KPT; ++j) {
      if (tid + j * kFewSelThreads < n_c && (u[j] & mask) == prefix)
        atomicAdd(&hist[(u[j] >> shift) & 255u], 1u);
    }
    __syncthreads();
    if (wave == 0) {
      // lane l holds digits 255 - 4l .. 252 - 4l (descending)
      uint32_t hv[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) hv[j] = hist[255 - 4 * lane - j];
      const uint32_t sum = hv[0] + hv[1] + hv[2] + hv[3];
      uint32_t incl = sum;
#pragma unroll
      for (int o = 1; o < 64; o <<= 1) {
        const uint32_t y = __shfl_up(incl, o);
        if (lane >= o) incl += y;
      }
      const uint32_t excl = incl - sum;
      if (excl < need && incl >= need) {
        uint32_t cum = excl, left = 0u;
        int digit = -1;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          if (digit < 0 && cum + hv[j] >= need) {
            digit = 255 - 4 * lane - j;
            left = need - cum;
          }
          cum += hv[j];
        }
        s_prefix = prefix | (static_cast<uint32_t>(digit) << shift);
        s_need = left;
      }
    }
    __syncthreads();
    prefix = s_prefix;
    need = s_need;
    mask |= ((1u << (rem - shift)) - 1u) << shift;
    rem = shift;
  }
  // keys above the threshold, and the `need` lowest codes tied on it
  // (counted in code order: thread t scans codes [t * per, (t + 1) * per))
  const int per = (n_c + kFewSelThreads - 1) / kFewSelThreads;
  const int c0 = tid * per, c1 = min(n_c, c0 + per);
  uint32_t ties = 0u;
  for (int c = c0; c < c1; ++c) ties += (few_keys[c] == prefix) ? 1u : 0u;
  uint32_t incl = ties;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const uint32_t y = __shfl_up(incl, o);
    if (lane >= o) incl += y;
  }
  if (lane == 63) s_wsum[wave] = incl;
  __syncthreads();
  uint32_t rank = incl - ties;
  for (int w = 0; w < wave; ++w) rank += s_wsum[w];
  for (int c = c0; c < c1; ++c) {
    const uint32_t v = few_keys[c];
    bool take = v > prefix;
    if (v == prefix) take = (rank++ < need);
    if (take) s_cand[atomicAdd(&s_nsel, 1u)] = key_of(v, c);  // exactly `top` keys
  }
  __syncthreads();
  if (tid >= top) return;
  const uint64_t k = s_cand[tid];
  int rk = 0;
  for (int j = 0; j < top; ++j) rk += (s_cand[j] > k) ? 1 : 0;
  out[rk] = static_cast<int32_t>(key_index(k));
}

int launch_topk_few_split(const FewScore& t0, const FewScore& t1, int h, const float* chat, int n_c, int d_s,
                          float temperature, hipStream_t st) {
  const dim3 g1(static_cast<unsigned>(h), static_cast<unsigned>(ceil_div(n_c, kScoreChunk)));
  code_scores_few_kernel<<<g1, kScoreChunk, 0, st>>>(t0, t1, h, chat, n_c, d_s, temperature);
  if (int s = check_launch("code_scores_few_kernel")) return s;
  const dim3 g2(static_cast<unsigned>(std::max(t0.total, t1.total)), t1.total > 0 ? 2u : 1u);
  const size_t smem = sizeof(uint32_t) * static_cast<size_t>(n_c);
  if (n_c <= 4 * kFewSelThreads) code_select_few_kernel<4><<<g2, kFewSelThreads, smem, st>>>(t0, t1, n_c);
  else if (n_c <= 16 * kFewSelThreads) code_select_few_kernel<16><<<g2, kFewSelThreads, smem, st>>>(t0, t1, n_c);
  else code_select_few_kernel<64><<<g2, kFewSelThreads, smem, st>>>(t0, t1, n_c);
  return check_launch("code_select_few_kernel");
}

struct TopkWorkspace {
  uint16_t* cbf;
  uint32_t* cmax_bits;
  uint8_t* flags;
};

size_t topk_workspace_bytes(int64_t batch, int h, int64_t rows, int n_c) {
  return align_up(sizeof(uint16_t) * static_cast<size_t>(h) * n_c_padded(n_c) * 32, 256) +
         align_up(sizeof(float) * static_cast<size_t>(h), 256) +
         align_up(static_cast<size_t>(batch * h * rows), 256);  // a flag per row
}

TopkWorkspace carve_topk(void* ws, int h, int n_c) {
  char* p = static_cast<char*>(ws);
  TopkWorkspace w;
  w.cbf = reinterpret_cast<uint16_t*>(p);
  p += align_up(sizeof(uint16_t) * static_cast<size_t>(h) * n_c_padded(n_c) * 32, 256);
  w.cmax_bits = reinterpret_cast<uint32_t*>(p);
  p += align_up(sizeof(float) * static_cast<size_t>(h), 256);
  w.flags = reinterpret_cast<uint8_t*>(p);
  return w;
}

constexpr int64_t kFewTopkRows = 64;

bool mfma_path_ok(int top, int d_s, int n_c) { return top <= 32 && d_s <= 32 && d_s % 4 == 0 && n_c <= 65535; }

int launch_exact_topk(const float* xhat, int64_t batch, int h, int64_t rows, const float* chat,
                      int n_c, int d_s, float temperature, int top, int32_t* codes, hipStream_t st) {
  const int64_t grid = batch * h * ceil_div(rows, kTopRows);
  const size_t smem = code_topk_smem(d_s, top);
  if (int s = reserve_lds(reinterpret_cast<const void*>(code_topk_kernel), smem, "code_topk")) return s;
  code_topk_kernel<<<dim3(static_cast<unsigned>(grid)), kTopThreads, smem, st>>>(
      xhat, rows, h, chat, n_c, d_s, temperature, top, codes);
  return check_launch("code_topk_kernel");
}

template <int TM>
int launch_rows_tm(const float* xhat, int64_t total, int64_t rows, int h, const float* chat, int n_c,
                   int d_s, float temperature, int top, int32_t* codes, const uint8_t* flags,
                   hipStream_t st) {
  const int64_t grid = std::min<int64_t>(ceil_div(total, 256), 1024);
  code_topk_rows_kernel<TM><<<dim3(static_cast<unsigned>(grid)), 256, 0, st>>>(
      xhat, total, rows, h, chat, n_c, d_s, temperature, top, codes, flags);
  return check_launch("code_topk_rows_kernel");
}

// The flagged rows of a matrix-core pass (top <= 32, d_s <= 32).
int launch_flagged_topk(const float* xhat, int64_t batch, int h, int64_t rows, const float* chat,
                        int n_c, int d_s, float temperature, int top, int32_t* codes,
                        const uint8_t* flags, hipStream_t st) {
  const int64_t total = batch * h * rows;
  if (top <= 4) return launch_rows_tm<4>(xhat, total, rows, h, chat, n_c, d_s, temperature, top, codes, flags, st);
  if (top <= 8) return launch_rows_tm<8>(xhat, total, rows, h, chat, n_c, d_s, temperature, top, codes, flags, st);
  if (top <= 16) return launch_rows_tm<16>(xhat, total, rows, h, chat, n_c, d_s, temperature, top, codes, flags, st);
  return launch_rows_tm<32>(xhat, total, rows, h, chat, n_c, d_s, temperature, top, codes, flags, st);
}

int launch_codebook_prep(const float* chat, int h, int n_c, int d_s, const TopkWorkspace& w,
                         hipStream_t st) {
  zero_u32_kernel<<<dim3(static_cast<unsigned>(ceil_div(h, 256))), 256, 0, st>>>(w.cmax_bits, h);
  if (int s = check_launch("zero_u32_kernel")) return s;
  codebook_prep_kernel<<<dim3(static_cast<unsigned>(ceil_div(n_c_padded(n_c), 256)), static_cast<unsigned>(h)),
                         256, 0, st>>>(chat, n_c, n_c_padded(n_c), d_s, w.cbf, w.cmax_bits);
  return check_launch("codebook_prep_kernel");
}

template <int Q>
int launch_mfma_q(const float* xhat, int64_t batch, int h, int64_t rows, const float* chat, int n_c,
                  int d_s, float temperature, int top, int32_t* codes, const TopkWorkspace& w,
                  hipStream_t st) {
  auto kern = code_topk_mfma_kernel<Q>;
  const size_t smem = code_topk_mfma_smem(top);
  if (int s = reserve_lds(reinterpret_cast<const void*>(kern), smem, "code_topk_mfma")) return s;
  const int64_t grid = batch * h * ceil_div(rows, kMfRows);
  kern<<<dim3(static_cast<unsigned>(grid)), 256, smem, st>>>(xhat, rows, h, chat, w.cbf, w.cmax_bits,
                                                             n_c, d_s, temperature, top, codes,
                                                             w.flags);
  return check_launch("code_topk_mfma_kernel");
}

// The query (top_a) and key (top_b) screens of one routing call in one launch
// (code_topk_mfma_pair_kernel); each keeps its own flag bytes for the
// exhaustive pass.
template <int QA, int QB>
int launch_mfma_pair(const float* xa, const float* xb, int64_t batch, int h, int64_t rows, const float* chat,
                     int n_c, int d_s, float temperature, int top_a, int top_b, int32_t* codes_a, int32_t* codes_b,
                     const TopkWorkspace& w, uint8_t* flags_b, hipStream_t st) {
  auto kern = code_topk_mfma_pair_kernel<QA, QB>;
  const size_t smem = std::max(code_topk_mfma_smem(top_a), code_topk_mfma_smem(top_b));
  if (int s = reserve_lds(reinterpret_cast<const void*>(kern), smem, "code_topk_mfma_pair")) return s;
  const int64_t grid_a = batch * h * ceil_div(rows, kMfRows);
  const int64_t grid = kXcds * xcd_per(2 * grid_a);  // whole rounds of the 8 XCDs; extras return at once
  kern<<<dim3(static_cast<unsigned>(grid)), 256, smem, st>>>(xa, xb, rows, h, chat, w.cbf, w.cmax_bits, n_c,
                                                                   d_s, temperature, top_a, top_b, codes_a, codes_b,
                                                                   w.flags, flags_b, grid_a);
  return check_launch("code_topk_mfma_pair_kernel");
}

// Top codes per row.  With a workspace (and top <= 32, d_s <= 32) the matrix-core
// filter runs and the exact kernel recomputes only flagged groups; otherwise the
// exact kernel handles every row.  `prepped` = the bf16 codebook is already in w.
int launch_code_topk_w(const float* xhat, int64_t batch, int h, int64_t rows, const float* chat,
                       int n_c, int d_s, float temperature, int top, int32_t* codes,
                       const TopkWorkspace& w, hipStream_t st) {
  // A handful of rows (decoding): every row exhaustively, one wave each.  The
  // matrix-core screen streams the whole codebook through one block per 256
  // rows, so for a few rows it runs one long dependent chain per head.
  if (batch * h * rows <= kFewTopkRows) {
    const FewTopk t0{xhat, rows, batch * h * rows, top, codes};
    FewTopk none{};
    return launch_topk_few(t0, none, h, chat, n_c, d_s, temperature, st);
  }
  int s;
  if (top <= 4) s = launch_mfma_q<1>(xhat, batch, h, rows, chat, n_c, d_s, temperature, top, codes, w, st);
  else if (top <= 8) s = launch_mfma_q<2>(xhat, batch, h, rows, chat, n_c, d_s, temperature, top, codes, w, st);
  else if (top <= 16) s = launch_mfma_q<4>(xhat, batch, h, rows, chat, n_c, d_s, temperature, top, codes, w, st);
  else s = launch_mfma_q<8>(xhat, batch, h, rows, chat, n_c, d_s, temperature, top, codes, w, st);
  if (s) return s;
  return launch_flagged_topk(xhat, batch, h, rows, chat, n_c, d_s, temperature, top, codes, w.flags, st);
}

int launch_code_topk(const float* xhat, int64_t batch, int h, int64_t rows, const float* chat,
                     int n_c, int d_s, float temperature, int top, int32_t* codes, void* ws,
                     bool prepped, hipStream_t st) {
  if (batch == 0 || rows == 0) return SSA_OK;
  if (!ws || !mfma_path_ok(top, d_s, n_c))
    return launch_exact_topk(xhat, batch, h, rows, chat, n_c, d_s, temperature, top, codes, st);
  const TopkWorkspace w = carve_topk(ws, h, n_c);
  int s;
  if (!prepped && (s = launch_codebook_prep(chat, h, n_c, d_s, w, st))) return s;
  return launch_code_topk_w(xhat, batch, h, rows, chat, n_c, d_s, temperature, top, codes, w, st);
}

int launch_normalize(const float* x, int64_t rows, int d_s, float* out, hipStream_t st) {
  if (rows == 0) return SSA_OK;
  normalize_rows_kernel<<<dim3(static_cast<unsigned>(ceil_div(rows, 256))), 256, 0, st>>>(x, rows, d_s,
                                                                                         out);
  return check_launch("normalize_rows_kernel");
}

}  // namespace

// ---- routing of a few new rows against a codebook prepared once (decoding)

size_t decode_prep_bytes(int h_kv, int n_c, int d_s) {
  return align_up(sizeof(float) * static_cast<size_t>(h_kv) * n_c * d_s, 256) +
         align_up(sizeof(uint16_t) * static_cast<size_t>(h_kv) * n_c_padded(n_c) * 32, 256) +
         align_up(sizeof(float) * static_cast<size_t>(h_kv), 256);
}

namespace {
struct DecodePrep {
  float* chat;
  TopkWorkspace w;
};
DecodePrep carve_prep(const void* prep, int h_kv, int n_c, int d_s) {
  char* c = static_cast<char*>(const_cast<void*>(prep));
  DecodePrep d{};
  d.chat = reinterpret_cast<float*>(c);
  c += align_up(sizeof(float) * static_cast<size_t>(h_kv) * n_c * d_s, 256);
  d.w.cbf = reinterpret_cast<uint16_t*>(c);
  c += align_up(sizeof(uint16_t) * static_cast<size_t>(h_kv) * n_c_padded(n_c) * 32, 256);
  d.w.cmax_bits = reinterpret_cast<uint32_t*>(c);
  d.w.flags = nullptr;
  return d;
}
}  // namespace

int decode_prep(const float* codebook, int h_kv, int n_c, int d_s, void* prep, hipStream_t st) {
  const DecodePrep d = carve_prep(prep, h_kv, n_c, d_s);
  if (int s = launch_normalize(codebook, static_cast<int64_t>(h_kv) * n_c, d_s, d.chat, st)) return s;
  return launch_codebook_prep(d.chat, h_kv, n_c, d_s, d.w, st);
}

size_t route_prepped_ws_bytes(int64_t batch, int64_t n, int h_kv, int d_s, int n_c) {
  const size_t rows = static_cast<size_t>(batch * h_kv * n);
  size_t bytes = 2 * align_up(sizeof(float) * rows * d_s, 256) + align_up(rows, 256);
  if (static_cast<int64_t>(rows) <= kFewTopkRows) bytes += 2 * align_up(sizeof(uint32_t) * rows * n_c, 256);
  return bytes;
}

int route_codes_prepped(const void* q, const void* k, int dtype, int64_t batch, int64_t n, int h_q,
                        int h_kv, int d, int64_t q_sb, int64_t q_sn, int64_t q_sh, int64_t k_sb,
                        int64_t k_sn, int64_t k_sh, const float* w_qr, const float* w_kr,
                        const void* prep, int d_s, int n_c, int a, int b, float temperature,
                        int32_t* q_codes, int32_t* k_codes, void* ws, hipStream_t st) {
  const int g = h_q / h_kv;
  int s = check_route_vectors(dtype, batch, n, h_q, g, d, d_s);
  if (!s) s = check_route_vectors(dtype, batch, n, h_kv, 1, d, d_s);
  if (!s) s = check_code_topk(batch, h_kv, n, n_c, d_s, temperature, a);
  if (!s) s = check_code_topk(batch, h_kv, n, n_c, d_s, temperature, b);
  if (s) return s;
  if (batch * n == 0) return SSA_OK;
  const size_t vec = align_up(sizeof(float) * static_cast<size_t>(batch * h_kv * n * d_s), 256);
  float* qhat = static_cast<float*>(ws);
  float* khat = reinterpret_cast<float*>(static_cast<char*>(ws) + vec);
  DecodePrep dp = carve_prep(prep, h_kv, n_c, d_s);
  dp.w.flags = reinterpret_cast<uint8_t*>(static_cast<char*>(ws) + 2 * vec);
  const int64_t rows = batch * h_kv * n;
  if (rows <= kFewTopkRows && mfma_path_ok(a, d_s, n_c) && mfma_path_ok(b, d_s, n_c) &&
      route_few_smem(g, d, d_s) <= 64 * 1024) {
    // a decoding step's few rows: queries and keys in one launch per stage
    const FewRoute rq{q, n, q_sb, q_sn, q_sh, rows, h_q, g, d, d_s, w_qr, qhat};
    const FewRoute rk{k, n, k_sb, k_sn, k_sh, rows, h_kv, 1, d, d_s, w_kr, khat};
    if ((s = launch_route_few(rq, rk, dtype, st))) return s;
    if (n_c <= kFewSelMaxCodes) {
      char* sc = static_cast<char*>(ws) + 2 * vec + align_up(static_cast<size_t>(rows), 256);
      const size_t sc_bytes = align_up(sizeof(uint32_t) * static_cast<size_t>(rows * n_c), 256);
      const FewScore sq{qhat, n, rows, a, reinterpret_cast<uint32_t*>(sc), q_codes};
      const FewScore sk{khat, n, rows, b, reinterpret_cast<uint32_t*>(sc + sc_bytes), k_codes};
      return launch_topk_few_split(sq, sk, h_kv, dp.chat, n_c, d_s, temperature, st);
    }
    const FewTopk tq{qhat, n, rows, a, q_codes};
    const FewTopk tk{khat, n, rows, b, k_codes};
    return launch_topk_few(tq, tk, h_kv, dp.chat, n_c, d_s, temperature, st);
  }
  if ((s = launch_route_vectors(q, dtype, batch, n, h_q, g, d, q_sb, q_sn, q_sh, w_qr, d_s, qhat, st))) return s;
  if ((s = launch_route_vectors(k, dtype, batch, n, h_kv, 1, d, k_sb, k_sn, k_sh, w_kr, d_s, khat, st))) return s;
  for (int pass = 0; pass < 2; ++pass) {
    const float* x = pass ? khat : qhat;
    const int top = pass ? b : a;
    int32_t* codes = pass ? k_codes : q_codes;
    if (mfma_path_ok(top, d_s, n_c))
      s = launch_code_topk_w(x, batch, h_kv, n, dp.chat, n_c, d_s, temperature, top, codes, dp.w, st);
    else
      s = launch_exact_topk(x, batch, h_kv, n, dp.chat, n_c, d_s, temperature, top, codes, st);
    if (s) return s;
  }
  return SSA_OK;
}

}  // namespace ssa

using namespace ssa;

extern "C" int ssa_route_vectors(const void* x, int dtype, int64_t batch, int64_t n, int h_in,
                                 int group, int d, int64_t x_sb, int64_t x_sn, int64_t x_sh,
                                 const float* w, int d_s, float* out, void* stream) {
  int st = check_route_vectors(dtype, batch, n, h_in, group, d, d_s);
  if (st) return st;
  if (batch * n > 0 && (!x || !w || !out))
    return fail(SSA_ERR_INVALID_ARGUMENT, "route_vectors: null pointer");
  return launch_route_vectors(x, dtype, batch, n, h_in, group, d, x_sb, x_sn, x_sh, w, d_s, out,
                              as_stream(stream));
}

extern "C" int ssa_normalize_rows(const float* x, int64_t rows, int d_s, float* out,
                                  void* stream) {
  if (rows < 0 || d_s <= 0) return fail(SSA_ERR_INVALID_ARGUMENT, "normalize_rows: bad shape");
  if (rows > 0 && (!x || !out)) return fail(SSA_ERR_INVALID_ARGUMENT, "normalize_rows: null pointer");
  return launch_normalize(x, rows, d_s, out, as_stream(stream));
}

extern "C" size_t ssa_code_topk_workspace_bytes(int64_t batch, int h, int64_t rows, int n_c) {
  if (batch < 0 || h <= 0 || rows < 0 || n_c <= 0) return 0;
  return topk_workspace_bytes(batch, h, rows, n_c);
}

extern "C" int ssa_code_topk(const float* xhat, int64_t batch, int h, int64_t rows,
                             const float* chat, int n_c, int d_s, float temperature, int top,
                             int32_t* codes, void* workspace, size_t workspace_bytes,
                             void* stream) {
  int st = check_code_topk(batch, h, rows, n_c, d_s, temperature, top);
  if (st) return st;
  if (batch * rows > 0 && (!xhat || !chat || !codes))
    return fail(SSA_ERR_INVALID_ARGUMENT, "code_topk: null pointer");
  if (workspace && workspace_bytes < topk_workspace_bytes(batch, h, rows, n_c))
    return fail(SSA_ERR_WORKSPACE, "code_topk: workspace %zu < %zu bytes", workspace_bytes,
                topk_workspace_bytes(batch, h, rows, n_c));
  return launch_code_topk(xhat, batch, h, rows, chat, n_c, d_s, temperature, top, codes,
                          workspace, false, as_stream(stream));
}

extern "C" size_t ssa_route_workspace_bytes(int64_t batch, int64_t n, int h_kv, int n_c,
                                            int d_s) {
  if (batch < 0 || n < 0 || h_kv <= 0 || n_c <= 0 || d_s <= 0) return 0;
  const size_t vec = align_up(sizeof(float) * static_cast<size_t>(batch * h_kv * n * d_s), 256);
  const size_t cb = align_up(sizeof(float) * static_cast<size_t>(h_kv) * n_c * d_s, 256);
  // (+ the key screen's flag bytes when both screens run in one launch)
  return 2 * vec + cb + topk_workspace_bytes(batch, h_kv, n, n_c) +
         align_up(static_cast<size_t>(batch * h_kv * n), 256);
}

extern "C" int ssa_route_codes(const void* q, const void* k, int dtype, int64_t batch, int64_t n,
                               int h_q, int h_kv, int d, int64_t q_sb, int64_t q_sn, int64_t q_sh,
                               int64_t k_sb, int64_t k_sn, int64_t k_sh, const float* w_qr,
                               const float* w_kr, const float* codebook, int d_s, int n_c, int a,
                               int b, float temperature, int32_t* q_codes, int32_t* k_codes,
                               void* workspace, size_t workspace_bytes, void* stream) {
  if (h_kv <= 0 || h_q <= 0 || h_q % h_kv != 0)
    return fail(SSA_ERR_INVALID_ARGUMENT, "num_q_heads must be divisible by num_kv_heads");
  const int g = h_q / h_kv;
  int st = check_route_vectors(dtype, batch, n, h_q, g, d, d_s);
  if (!st) st = check_route_vectors(dtype, batch, n, h_kv, 1, d, d_s);
  if (!st) st = check_code_topk(batch, h_kv, n, n_c, d_s, temperature, a);
  if (!st) st = check_code_topk(batch, h_kv, n, n_c, d_s, temperature, b);
  if (st) return st;
  const size_t need = ssa_route_workspace_bytes(batch, n, h_kv, n_c, d_s);
  if (workspace_bytes < need)
    return fail(SSA_ERR_WORKSPACE, "route_codes: workspace %zu < %zu bytes", workspace_bytes, need);
  if (batch * n == 0) return SSA_OK;
  if (!q || !k || !w_qr || !w_kr || !codebook || !q_codes || !k_codes || !workspace)
    return fail(SSA_ERR_INVALID_ARGUMENT, "route_codes: null pointer");
  hipStream_t s = as_stream(stream);
  const size_t vec = align_up(sizeof(float) * static_cast<size_t>(batch * h_kv * n * d_s), 256);
  float* qhat = static_cast<float*>(workspace);
  float* khat = reinterpret_cast<float*>(static_cast<char*>(workspace) + vec);
  float* chat = reinterpret_cast<float*>(static_cast<char*>(workspace) + 2 * vec);
  void* tws = static_cast<char*>(workspace) + 2 * vec +
              align_up(sizeof(float) * static_cast<size_t>(h_kv) * n_c * d_s, 256);
  if ((st = launch_route_vectors(q, dtype, batch, n, h_q, g, d, q_sb, q_sn, q_sh, w_qr, d_s, qhat, s)))
    return st;
  if ((st = launch_route_vectors(k, dtype, batch, n, h_kv, 1, d, k_sb, k_sn, k_sh, w_kr, d_s, khat, s)))
    return st;
  if ((st = launch_normalize(codebook, static_cast<int64_t>(h_kv) * n_c, d_s, chat, s))) return st;
  // top 16 for the queries and top 4 for the keys (config 3's a and b): both
  // screens in one launch, the keys' flag bytes after the workspace's others
  if (mf_q(a) == 4 && mf_q(b) == 1 && mfma_path_ok(a, d_s, n_c) && mfma_path_ok(b, d_s, n_c) &&
      batch * h_kv * n > kFewTopkRows) {
    const TopkWorkspace w = carve_topk(tws, h_kv, n_c);
    uint8_t* flags_b = static_cast<uint8_t*>(tws) + topk_workspace_bytes(batch, h_kv, n, n_c);
    if ((st = launch_codebook_prep(chat, h_kv, n_c, d_s, w, s))) return st;
    if ((st = launch_mfma_pair<4, 1>(qhat, khat, batch, h_kv, n, chat, n_c, d_s, temperature, a, b, q_codes, k_codes,
                                     w, flags_b, s)))
      return st;
    if ((st = launch_flagged_topk(qhat, batch, h_kv, n, chat, n_c, d_s, temperature, a, q_codes, w.flags, s)))
      return st;
    return launch_flagged_topk(khat, batch, h_kv, n, chat, n_c, d_s, temperature, b, k_codes, flags_b, s);
  }
  if ((st = launch_code_topk(qhat, batch, h_kv, n, chat, n_c, d_s, temperature, a, q_codes, tws,
                             false, s)))
    return st;
  return launch_code_topk(khat, batch, h_kv, n, chat, n_c, d_s, temperature, b, k_codes, tws,
                          true, s);
}
