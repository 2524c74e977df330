// Stage (c): candidate union, dedup, full-dimensional rescoring and exact top-k.
//
// Replaces CodebookRouter._select_candidates / _build_candidate_mask
// (ssa/router.py:151-259).  One 256-thread block per (batch, kv-head, query):
//   1. the query's a buckets are clipped to keys j <= i (causal; postings
//      ascend, so one binary search per bucket) and concatenated;
//   2. postings stream through an n-bit LDS bitmap (atomicOr dedup); new keys
//      queue in an LDS batch;
//   3. each batch is rescored in the canonical fp32 order (one thread per key:
//      g fmaf chains over d, / score_div, summed over the group, / g) and the
//      composite keys that beat the running k-th best append to a top buffer,
//      which a bitonic sort truncates back to k whenever it overflows;
//   4. the final top buffer is sorted (score desc, index asc), then the lowest
//      non-candidate indices fill the row up to min(k, n), then zeros pad to k.
#include "ssa_common.h"

namespace ssa {
namespace {

constexpr int kSelThreads = 256;
constexpr int kSelBatch = 512;
constexpr int kMaxA = 64;

struct SelParams {
  const void* q;
  const void* k;
  int64_t n;
  int h_q, h_kv, g, d;
  int64_t q_sb, q_sn, q_sh, k_sb, k_sn, k_sh;
  const int32_t* q_codes;
  int a;
  const int32_t* offsets;
  const int32_t* postings;
  int n_c, b;
  int top_k, k_eff, sortn, mask_mode;
  const uint8_t* mask;
  int64_t mask_sb, mask_si;
  float score_div;
  void* out;
  int out_i64;
  int32_t* stats;
};

__host__ __device__ inline int pow2_at_least(int v) {
  int p = 1;
  while (p < v) p <<= 1;
  return p;
}

inline size_t select_smem(int64_t n, int d, int gmax, int sortn) {
  const size_t words = static_cast<size_t>((n + 31) / 32);
  return sizeof(uint64_t) * sortn + sizeof(float) * static_cast<size_t>(d) * gmax +
         sizeof(uint32_t) * words + sizeof(int32_t) * (kSelBatch + 2 * kMaxA + 1);
}

// 8 consecutive elements widened to fp32 (16-byte aligned for bf16, 32 for f32).
__device__ __forceinline__ void load8(const uint16_t* p, float* o) {
  const uint4 u = *reinterpret_cast<const uint4*>(p);
  const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    o[2 * e] = __uint_as_float(w[e] << 16);
    o[2 * e + 1] = __uint_as_float(w[e] & 0xFFFF0000u);
  }
}
__device__ __forceinline__ void load8(const float* p, float* o) {
  const float4 a = *reinterpret_cast<const float4*>(p);
  const float4 b = *reinterpret_cast<const float4*>(p + 4);
  o[0] = a.x; o[1] = a.y; o[2] = a.z; o[3] = a.w;
  o[4] = b.x; o[5] = b.y; o[6] = b.z; o[7] = b.w;
}

// Descending bitonic sort of buf[0..len) (len a power of two) by the whole block.
__device__ void bitonic_desc(uint64_t* buf, int len) {
  for (int size = 2; size <= len; size <<= 1) {
    for (int stride = size >> 1; stride > 0; stride >>= 1) {
      for (int t = threadIdx.x; t < (len >> 1); t += kSelThreads) {
        const int lo = 2 * t - (t & (stride - 1));
        const int hi = lo + stride;
        const bool desc = (lo & size) == 0;
        const uint64_t x = buf[lo], y = buf[hi];
        if ((x < y) == desc) {
          buf[lo] = y;
          buf[hi] = x;
        }
      }
      __syncthreads();
    }
  }
}

// Exclusive block-wide prefix sum of v; *total receives the block sum.
__device__ int block_exclusive_scan(int v, int* scratch, int* total) {
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  int x = v;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const int y = __shfl_up(x, off, 64);
    if (lane >= off) x += y;
  }
  if (lane == 63) scratch[wave] = x;
  __syncthreads();
  int base = 0, tot = 0;
#pragma unroll
  for (int w = 0; w < kSelThreads / 64; ++w) {
    const int s = scratch[w];
    if (w < wave) base += s;
    tot += s;
  }
  __syncthreads();
  *total = tot;
  return base + x - v;
}

template <typename T, int GMAX>
__global__ __launch_bounds__(kSelThreads) void select_kernel(SelParams p) {
  extern __shared__ __align__(16) unsigned char smem[];
  uint64_t* topbuf = reinterpret_cast<uint64_t*>(smem);
  float* qs = reinterpret_cast<float*>(topbuf + p.sortn);  // [d][GMAX]
  const int words = static_cast<int>((p.n + 31) >> 5);
  uint32_t* bitmap = reinterpret_cast<uint32_t*>(qs + p.d * GMAX);
  int32_t* batch = reinterpret_cast<int32_t*>(bitmap + words);
  int32_t* seg_lo = batch + kSelBatch;
  int32_t* seg_start = seg_lo + kMaxA;  // a + 1 entries
  __shared__ int s_batch_cnt, s_top_cnt, s_cand_total, s_R, s_filled;
  __shared__ uint64_t s_thr;
  __shared__ int s_scan[kSelThreads / 64];

  const int tid = threadIdx.x;
  const int64_t row = blockIdx.x;  // ((b * h_kv + h) * n + i)
  const int64_t i = row % p.n;
  const int64_t bh = row / p.n;
  const int h = static_cast<int>(bh % p.h_kv);
  const int64_t bb = bh / p.h_kv;

  for (int w = tid; w < words; w += kSelThreads) bitmap[w] = 0u;
  const T* qrow = static_cast<const T*>(p.q) + bb * p.q_sb + i * p.q_sn;
  for (int e = tid; e < p.d * GMAX; e += kSelThreads) {
    const int t = e / GMAX, gg = e % GMAX;
    qs[e] = (gg < p.g) ? ld(qrow + static_cast<int64_t>(h * p.g + gg) * p.q_sh + t) : 0.0f;
  }
  const int32_t* pp = p.postings + bh * p.n * p.b;
  if (tid < p.a) {
    const int32_t c = p.q_codes[(bh * p.n + i) * p.a + tid];
    int32_t lo = 0, hi = 0;
    if (static_cast<uint32_t>(c) < static_cast<uint32_t>(p.n_c)) {
      const int32_t* off = p.offsets + bh * (p.n_c + 1);
      const int32_t total = static_cast<int32_t>(p.n * p.b);
      lo = min(max(off[c], 0), total);
      hi = min(max(off[c + 1], lo), total);
      if (p.mask_mode == SSA_MASK_CAUSAL) {
        int32_t L = lo, H = hi;
        while (L < H) {
          const int32_t mid = (L + H) >> 1;
          if (pp[mid] <= i) L = mid + 1;
          else H = mid;
        }
        hi = L;
      }
    }
    seg_lo[tid] = lo;
    seg_start[tid + 1] = hi - lo;
  }
  if (tid == 0) {
    s_batch_cnt = 0;
    s_top_cnt = 0;
    s_cand_total = 0;
    s_thr = 0ull;
    seg_start[0] = 0;
  }
  __syncthreads();
  if (tid == 0) {
    for (int m = 1; m <= p.a; ++m) seg_start[m] += seg_start[m - 1];
    s_R = seg_start[p.a];
  }
  __syncthreads();
  const int R = s_R;
  const uint8_t* mrow =
      (p.mask_mode == SSA_MASK_DENSE) ? p.mask + bb * p.mask_sb + i * p.mask_si : nullptr;
  const T* kbase = static_cast<const T*>(p.k) + bb * p.k_sb + static_cast<int64_t>(h) * p.k_sh;

  for (int base = 0; base < R; base += kSelThreads) {
    const int pidx = base + tid;
    if (pidx < R) {
      int lo_m = 0, hi_m = p.a;
      while (hi_m - lo_m > 1) {
        const int mid = (lo_m + hi_m) >> 1;
        if (seg_start[mid] <= pidx) lo_m = mid;
        else hi_m = mid;
      }
      const int32_t j = pp[seg_lo[lo_m] + (pidx - seg_start[lo_m])];
      const bool allowed = (static_cast<uint32_t>(j) < static_cast<uint32_t>(p.n)) &&
                           ((mrow == nullptr) || (mrow[j] != 0));
      if (allowed) {
        const uint32_t bit = 1u << (j & 31);
        const uint32_t old = atomicOr(&bitmap[j >> 5], bit);
        if (!(old & bit)) batch[atomicAdd(&s_batch_cnt, 1)] = j;
      }
    }
    __syncthreads();
    const int bc = s_batch_cnt;
    __syncthreads();  // every thread holds bc before the next round appends again
    const bool last = (base + kSelThreads >= R);
    if (bc > kSelBatch - kSelThreads || (last && bc > 0)) {
      const uint64_t thr = s_thr;
      for (int e = tid; e < bc; e += kSelThreads) {
        const int32_t j = batch[e];
        const T* kr = kbase + static_cast<int64_t>(j) * p.k_sn;
        float acc[GMAX];
#pragma unroll
        for (int gg = 0; gg < GMAX; ++gg) acc[gg] = 0.0f;
        for (int t0 = 0; t0 < p.d; t0 += 8) {
          float kv[8];
          load8(kr + t0, kv);
#pragma unroll
          for (int u = 0; u < 8; ++u) {
            const float* qv = qs + (t0 + u) * GMAX;
#pragma unroll
            for (int gg = 0; gg < GMAX; ++gg) acc[gg] = fma_rn(qv[gg], kv[u], acc[gg]);
          }
        }
        float s = acc[0] / p.score_div;
#pragma unroll
        for (int gg = 1; gg < GMAX; ++gg)
          if (gg < p.g) s = s + acc[gg] / p.score_div;
        s = s / static_cast<float>(p.g);
        const uint64_t key = composite_key(s, static_cast<uint32_t>(j));
        if (key > thr) topbuf[atomicAdd(&s_top_cnt, 1)] = key;
      }
      __syncthreads();
      const int tc = s_top_cnt;
      if (tc > p.k_eff) {
        const int len = pow2_at_least(tc);
        for (int e = tc + tid; e < len; e += kSelThreads) topbuf[e] = 0ull;
        __syncthreads();
        bitonic_desc(topbuf, len);
      }
      if (tid == 0) {
        if (tc > p.k_eff) {
          s_top_cnt = p.k_eff;
          s_thr = topbuf[p.k_eff - 1];
        }
        s_cand_total += bc;
        s_batch_cnt = 0;
      }
      __syncthreads();
    }
  }

  const int tc = s_top_cnt;
  if (tc > 1) {
    const int len = pow2_at_least(tc);
    for (int e = tc + tid; e < len; e += kSelThreads) topbuf[e] = 0ull;
    __syncthreads();
    bitonic_desc(topbuf, len);
  }
  __syncthreads();

  const int64_t obase = ((bb * p.n + i) * p.h_kv + h) * p.top_k;
  int64_t* out64 = static_cast<int64_t*>(p.out) + obase;
  int32_t* out32 = static_cast<int32_t*>(p.out) + obase;
  auto put = [&](int w, int64_t v) {
    if (p.out_i64) out64[w] = v;
    else out32[w] = static_cast<int32_t>(v);
  };
  const int nsel = tc < p.k_eff ? tc : p.k_eff;
  for (int w = tid; w < nsel; w += kSelThreads) put(w, key_index(topbuf[w]));

  const int need = p.k_eff - nsel;
  if (need > 0) {
    if (tid == 0) s_filled = 0;
    __syncthreads();
    for (int w0 = 0; w0 < words; w0 += kSelThreads) {
      const int filled = s_filled;
      if (filled >= need) break;
      const int w = w0 + tid;
      uint32_t zeros = 0u;
      if (w < words) {
        zeros = ~bitmap[w];
        if (w == words - 1 && (p.n & 31)) zeros &= (1u << (p.n & 31)) - 1u;
      }
      int total = 0;
      int rank = filled + block_exclusive_scan(__popc(zeros), s_scan, &total);
      while (zeros != 0u && rank < need) {
        const int bpos = __ffs(zeros) - 1;
        zeros &= zeros - 1u;
        put(nsel + rank, static_cast<int64_t>(w) * 32 + bpos);
        ++rank;
      }
      __syncthreads();
      if (tid == 0) s_filled = filled + total;
      __syncthreads();
    }
  }
  for (int w = p.k_eff + tid; w < p.top_k; w += kSelThreads) put(w, 0);
  if (p.stats && tid == 0) {
    p.stats[(bh * p.n + i) * 2 + 0] = s_cand_total;
    p.stats[(bh * p.n + i) * 2 + 1] = R;
  }
}

template <typename T, int GMAX>
int launch_select(const SelParams& p, int64_t rows, size_t smem, hipStream_t st) {
  auto kern = select_kernel<T, GMAX>;
  if (int s = reserve_lds(reinterpret_cast<const void*>(kern), smem, "select")) return s;
  kern<<<dim3(static_cast<unsigned>(rows)), kSelThreads, smem, st>>>(p);
  return check_launch("select_kernel");
}

template <typename T>
int dispatch_select(const SelParams& p, int64_t rows, hipStream_t st) {
  if (p.g <= 4) return launch_select<T, 4>(p, rows, select_smem(p.n, p.d, 4, p.sortn), st);
  if (p.g <= 8) return launch_select<T, 8>(p, rows, select_smem(p.n, p.d, 8, p.sortn), st);
  return launch_select<T, 16>(p, rows, select_smem(p.n, p.d, 16, p.sortn), st);
}

}  // namespace
}  // namespace ssa

using namespace ssa;

extern "C" int ssa_select(const void* q, const void* k, int dtype, int64_t batch, int64_t n,
                          int h_q, int h_kv, int d, int64_t q_sb, int64_t q_sn, int64_t q_sh,
                          int64_t k_sb, int64_t k_sn, int64_t k_sh, const int32_t* q_codes, int a,
                          const int32_t* offsets, const int32_t* postings, int n_c, int b,
                          int top_k, int mask_mode, const uint8_t* mask, int64_t mask_sb,
                          int64_t mask_si, float score_div, void* out, int out_index_dtype,
                          int32_t* stats, void* stream) {
  if (dtype != SSA_DTYPE_F32 && dtype != SSA_DTYPE_BF16)
    return fail(SSA_ERR_UNSUPPORTED, "select: dtype %d not supported (f32, bf16)", dtype);
  if (batch < 0 || n < 0 || h_q <= 0 || h_kv <= 0 || d <= 0 || a <= 0 || b <= 0 || n_c <= 0 ||
      top_k <= 0)
    return fail(SSA_ERR_INVALID_ARGUMENT, "select: bad shape");
  if (h_q % h_kv != 0)
    return fail(SSA_ERR_INVALID_ARGUMENT, "num_q_heads must be divisible by num_kv_heads");
  const int g = h_q / h_kv;
  if (g > 16) return fail(SSA_ERR_UNSUPPORTED, "select: group size %d > 16", g);
  if (a > kMaxA) return fail(SSA_ERR_UNSUPPORTED, "select: codes_per_query %d > %d", a, kMaxA);
  if (d % 8 != 0 || d > 256) return fail(SSA_ERR_UNSUPPORTED, "select: head_dim %d (need %%8, <=256)", d);
  if (top_k > 4096) return fail(SSA_ERR_UNSUPPORTED, "select: top_k %d > 4096", top_k);
  if (n >= (int64_t(1) << 31) || n * b >= (int64_t(1) << 31))
    return fail(SSA_ERR_UNSUPPORTED, "select: n*b must be < 2^31");
  if (mask_mode < SSA_MASK_NONE || mask_mode > SSA_MASK_DENSE)
    return fail(SSA_ERR_INVALID_ARGUMENT, "select: mask_mode %d", mask_mode);
  if (mask_mode == SSA_MASK_DENSE && n > 0 && !mask)
    return fail(SSA_ERR_INVALID_ARGUMENT, "select: dense mask pointer is null");
  if (out_index_dtype != SSA_INDEX_I32 && out_index_dtype != SSA_INDEX_I64)
    return fail(SSA_ERR_INVALID_ARGUMENT, "select: out_index_dtype %d", out_index_dtype);
  if (!(score_div > 0.0f)) return fail(SSA_ERR_INVALID_ARGUMENT, "select: score_div must be > 0");
  const int vec = (dtype == SSA_DTYPE_BF16) ? 8 : 4;
  if ((k_sn % vec) || (k_sh % vec) || (k_sb % vec) ||
      (reinterpret_cast<uintptr_t>(k) % 16))
    return fail(SSA_ERR_UNSUPPORTED, "select: k rows must be 16-byte aligned");
  if (batch == 0 || n == 0) return SSA_OK;
  if (!q || !k || !q_codes || !offsets || !postings || !out)
    return fail(SSA_ERR_INVALID_ARGUMENT, "select: null pointer");
  SelParams p{};
  p.q = q;
  p.k = k;
  p.n = n;
  p.h_q = h_q;
  p.h_kv = h_kv;
  p.g = g;
  p.d = d;
  p.q_sb = q_sb; p.q_sn = q_sn; p.q_sh = q_sh;
  p.k_sb = k_sb; p.k_sn = k_sn; p.k_sh = k_sh;
  p.q_codes = q_codes;
  p.a = a;
  p.offsets = offsets;
  p.postings = postings;
  p.n_c = n_c;
  p.b = b;
  p.top_k = top_k;
  p.k_eff = static_cast<int>(top_k < n ? top_k : n);
  p.sortn = pow2_at_least(p.k_eff + kSelBatch);
  p.mask_mode = mask_mode;
  p.mask = mask;
  p.mask_sb = mask_sb;
  p.mask_si = mask_si;
  p.score_div = score_div;
  p.out = out;
  p.out_i64 = (out_index_dtype == SSA_INDEX_I64);
  p.stats = stats;
  const int gmax = g <= 4 ? 4 : (g <= 8 ? 8 : 16);
  const size_t smem = select_smem(n, d, gmax, p.sortn);
  if (smem > 160 * 1024)
    return fail(SSA_ERR_UNSUPPORTED, "select: needs %zu bytes of LDS (n=%lld, top_k=%d)", smem,
                static_cast<long long>(n), top_k);
  const int64_t rows = batch * h_kv * n;
  if (rows >= (int64_t(1) << 31)) return fail(SSA_ERR_UNSUPPORTED, "select: too many rows");
  hipStream_t st = as_stream(stream);
  if (dtype == SSA_DTYPE_BF16) return dispatch_select<uint16_t>(p, rows, st);
  return dispatch_select<float>(p, rows, st);
}
