// Stage (c): candidate union, dedup, full-dimensional rescoring and exact top-k.
//
// Replaces CodebookRouter._select_candidates / _build_candidate_mask
// (ssa/router.py:151-259).  One 256-thread block per (batch, kv-head, query):
//   1. the query's a buckets are concatenated (a wave scan of their sizes);
//   2. postings stream through an n-bit LDS bitmap (atomicOr dedup), keys
//      outside the mask (j > i when causal) skipped;
//   3. candidates are rescored in the canonical fp32 order (one thread per key:
//      g fmaf chains over d with the query operands in scalar registers,
//      / score_div, summed over the group, / g); composite keys that beat the
//      running k-th best append to a top buffer, which a bitonic sort
//      truncates back to k whenever it overflows;
//   4. the row is staged in LDS and stored with coalesced writes.
// Two output orders:
//   sorted   : selected keys by (score desc, index asc), as torch.topk returns
//              them (ssa/router.py:204), then the lowest non-candidate indices
//              up to min(k, n), then zeros;
//   unsorted : the same index set, selected keys ascending, then the same
//              filler.  Rows with at most k candidates need no scores at all in
//              this order (their set is every candidate), so only rows with
//              more than k candidates are rescored.
#include "ssa_common.h"

namespace ssa {
namespace {

constexpr int kSelThreads = 256;
constexpr int kSelBatch = 512;
constexpr int kMaxA = 64;
// Key-row 16-byte loads issued ahead of each rescoring group (4 x 8 features):
// measured fastest at the headline shape against 1, 2 and 8, and against
// broadcasting the query operands from LDS.
constexpr int kRescoreLoads = 4;

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
  int top_k, k_eff, sortn, mask_mode, sorted;
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

inline size_t select_smem(int64_t n, int sortn, int k_eff) {
  const size_t words = static_cast<size_t>((n + 31) / 32);
  return sizeof(uint64_t) * sortn + sizeof(uint32_t) * words +
         sizeof(int32_t) * (kSelBatch + k_eff + 2 * kMaxA + 1);
}

// 8 consecutive elements widened to fp32 (16-byte aligned).
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

// Writes, in ascending order, the first `limit` positions j < n whose bitmap bit
// equals `want_set` to dst[0..]; returns how many were written.  Only words
// below `live` are stored; the rest read as zero.
__device__ int scan_bits(const uint32_t* bitmap, int words, int live, int64_t n, bool want_set,
                         int32_t* dst, int limit, int* scratch) {
  int filled = 0;
  const int wend = want_set ? live : words;
  for (int w0 = 0; w0 < wend && filled < limit; w0 += kSelThreads) {
    const int w = w0 + threadIdx.x;
    uint32_t bits = 0u;
    if (w < wend) {
      const uint32_t stored = (w < live) ? bitmap[w] : 0u;
      bits = want_set ? stored : ~stored;
      if (w == words - 1 && (n & 31)) bits &= (1u << (n & 31)) - 1u;
    }
    int total = 0;
    int rank = filled + block_exclusive_scan(__popc(bits), scratch, &total);
    while (bits != 0u && rank < limit) {
      const int bpos = __ffs(bits) - 1;
      bits &= bits - 1u;
      dst[rank++] = w * 32 + bpos;
    }
    filled += total;
  }
  return filled < limit ? filled : limit;
}

// Canonical rescoring of key row kr (per thread) against the group's query rows
// (uniform: head gg at q0 + gg * q_sh): acc[gg] = fmaf chain over t ascending.
// The query operands are loaded with uniform addresses from a read-only
// argument, so they sit in scalar registers and the chains read no LDS.  D > 0
// fixes the head dim so that each group of 16-byte key loads is issued before
// the chains consume it; D == 0 walks a runtime d.
template <typename T, int GMAX, int D>
__device__ __forceinline__ void rescore_row(const T* kr, const T* q0, int64_t q_sh, int g, int d,
                                            float (&acc)[GMAX]) {
#pragma unroll
  for (int gg = 0; gg < GMAX; ++gg) acc[gg] = 0.0f;
  constexpr int G = kRescoreLoads;
  const int dd = (D > 0) ? D : d;
  // Rolled over groups: unrolling lets the compiler keep all D*GMAX query
  // values live across the candidate loop.
#pragma unroll 1
  for (int t0 = 0; t0 < dd; t0 += 8 * G) {
    float kv[G][8];
#pragma unroll
    for (int u = 0; u < G; ++u)
      if (D > 0 || t0 + 8 * u < dd) load8(kr + t0 + 8 * u, kv[u]);
#pragma unroll
    for (int gg = 0; gg < GMAX; ++gg) {
      if (gg >= g) continue;
      const T* qgp = q0 + static_cast<int64_t>(gg) * q_sh + t0;
#pragma unroll
      for (int u = 0; u < G; ++u) {
        if (D == 0 && t0 + 8 * u >= dd) continue;
        float qv[8];
        load8(qgp + 8 * u, qv);
#pragma unroll
        for (int e = 0; e < 8; ++e) acc[gg] = fma_rn(qv[e], kv[u][e], acc[gg]);
      }
    }
  }
}

// One row ((b * h_kv + h) * n + i) by the whole block.  `heavy`: the row is
// known to have more than k_eff candidates (index order only), so the counting
// pass is skipped.
template <typename T, int GMAX, int D>
__device__ __forceinline__ void select_row(const SelParams& p, const T* __restrict__ qg, int64_t row,
                                           bool heavy) {
  extern __shared__ __align__(16) unsigned char smem[];
  uint64_t* topbuf = reinterpret_cast<uint64_t*>(smem);
  const int words = static_cast<int>((p.n + 31) >> 5);
  uint32_t* bitmap = reinterpret_cast<uint32_t*>(topbuf + p.sortn);
  int32_t* batch = reinterpret_cast<int32_t*>(bitmap + words);
  int32_t* stage = batch + kSelBatch;      // [k_eff] output row before the coalesced store
  int32_t* seg_lo = stage + p.k_eff;
  int32_t* seg_start = seg_lo + kMaxA;     // a + 1 entries
  __shared__ int s_batch_cnt, s_top_cnt, s_cand, s_R;
  __shared__ uint64_t s_thr;
  __shared__ int s_scan[kSelThreads / 64];

  const int tid = threadIdx.x;
  const int64_t i = row % p.n;
  const int64_t bh = row / p.n;
  const int h = static_cast<int>(bh % p.h_kv);
  const int64_t bb = bh / p.h_kv;
  const T* q0 = qg + bb * p.q_sb + i * p.q_sn + static_cast<int64_t>(h * p.g) * p.q_sh;
  const T* kbase = static_cast<const T*>(p.k) + bb * p.k_sb + static_cast<int64_t>(h) * p.k_sh;
  const int32_t* pp = p.postings + bh * p.n * p.b;
  const uint8_t* mrow =
      (p.mask_mode == SSA_MASK_DENSE) ? p.mask + bb * p.mask_sb + i * p.mask_si : nullptr;

  // Under the causal mask every candidate is <= i: only words up to i / 32 are
  // ever set, so only those are cleared and scanned.
  const int live = (p.mask_mode == SSA_MASK_CAUSAL) ? static_cast<int>(i >> 5) + 1 : words;
  for (int w = tid; w < live; w += kSelThreads) bitmap[w] = 0u;
  // Buckets are read whole and filtered by the mask in the union pass (no
  // dependent search over the postings); a wave scan turns their sizes into
  // start positions in the concatenated list.
  if (tid < 64) {
    int32_t lo = 0, len = 0;
    if (tid < p.a) {
      const int32_t c = p.q_codes[(bh * p.n + i) * p.a + tid];
      if (static_cast<uint32_t>(c) < static_cast<uint32_t>(p.n_c)) {
        const int32_t* off = p.offsets + bh * (p.n_c + 1);
        const int32_t total = static_cast<int32_t>(p.n * p.b);
        lo = min(max(off[c], 0), total);
        len = min(max(off[c + 1], lo), total) - lo;
      }
    }
    int32_t x = len;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
      const int32_t y = __shfl_up(x, o, 64);
      if (tid >= o) x += y;
    }
    if (tid < p.a) {
      seg_lo[tid] = lo;
      seg_start[tid + 1] = x;
    }
    if (tid == 0) {
      seg_start[0] = 0;
      s_R = 0;
      s_batch_cnt = 0;
      s_top_cnt = 0;
      s_cand = 0;
      s_thr = 0ull;
    }
  }
  __syncthreads();
  const int R = seg_start[p.a];
  const bool causal = p.mask_mode == SSA_MASK_CAUSAL;

  // Union of the row's postings into the bitmap.  With `collect`, new keys also
  // queue in the batch and are rescored whenever it fills (streaming top-k).
  // `count_raw` tallies the postings inside the causal window (all postings
  // otherwise) for the stats.
  auto union_pass = [&](bool collect, bool count_raw) {
    for (int base = 0; base < R; base += kSelThreads) {
      const int pidx = base + tid;
      bool in_window = false;
      if (pidx < R) {
        int lo_m = 0, hi_m = p.a;
        while (hi_m - lo_m > 1) {
          const int mid = (lo_m + hi_m) >> 1;
          if (seg_start[mid] <= pidx) lo_m = mid;
          else hi_m = mid;
        }
        const int32_t j = pp[seg_lo[lo_m] + (pidx - seg_start[lo_m])];
        in_window = !causal || j <= i;
        const bool allowed = (static_cast<uint32_t>(j) < static_cast<uint32_t>(p.n)) && in_window &&
                             ((mrow == nullptr) || (mrow[j] != 0));
        if (allowed) {
          const uint32_t bit = 1u << (j & 31);
          const uint32_t old = atomicOr(&bitmap[j >> 5], bit);
          if (!(old & bit)) {
            if (collect) batch[atomicAdd(&s_batch_cnt, 1)] = j;
            else atomicAdd(&s_cand, 1);
          }
        }
      }
      if (count_raw) {
        const uint64_t m = __ballot(in_window);
        if ((tid & 63) == 0) atomicAdd(&s_R, __popcll(m));
      }
      __syncthreads();
      if (!collect) continue;
      const int bc = s_batch_cnt;
      __syncthreads();  // every thread holds bc before the next round appends again
      const bool last = (base + kSelThreads >= R);
      if (bc > kSelBatch - kSelThreads || (last && bc > 0)) {
        const uint64_t thr = s_thr;
        for (int e = tid; e < bc; e += kSelThreads) {
          const int32_t j = batch[e];
          float acc[GMAX];
          rescore_row<T, GMAX, D>(kbase + static_cast<int64_t>(j) * p.k_sn, q0, p.q_sh, p.g, p.d, acc);
          float sc = acc[0] / p.score_div;
#pragma unroll
          for (int gg = 1; gg < GMAX; ++gg)
            if (gg < p.g) sc = sc + acc[gg] / p.score_div;
          sc = sc / static_cast<float>(p.g);
          const uint64_t key = composite_key(sc, static_cast<uint32_t>(j));
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
          s_cand += bc;
          s_batch_cnt = 0;
        }
        __syncthreads();
      }
    }
  };

  int nsel = 0;  // selected candidates at the head of `stage`
  const bool want_stats = p.stats != nullptr;
  if (!p.sorted) {
    int C = p.k_eff + 1;
    if (!heavy) {
      union_pass(false, want_stats);
      __syncthreads();
      C = s_cand;
      __syncthreads();  // every thread holds C before thread 0 may reset s_cand below
    }
    if (C <= p.k_eff) {
      nsel = scan_bits(bitmap, words, live, p.n, true, stage, C, s_scan);
    } else {
      if (!heavy) {
        for (int w = tid; w < live; w += kSelThreads) bitmap[w] = 0u;
        if (tid == 0) s_cand = 0;
        __syncthreads();
      }
      union_pass(true, heavy && want_stats);
      // Selected set (top k_eff keys) in ascending index order, via the bitmap.
      for (int w = tid; w < live; w += kSelThreads) bitmap[w] = 0u;
      __syncthreads();
      for (int e = tid; e < p.k_eff; e += kSelThreads) {
        const uint32_t j = key_index(topbuf[e]);
        atomicOr(&bitmap[j >> 5], 1u << (j & 31));
      }
      __syncthreads();
      nsel = scan_bits(bitmap, words, live, p.n, true, stage, p.k_eff, s_scan);
      // Restore the candidate bitmap for the filler: no filler is needed here.
    }
  } else {
    union_pass(true, want_stats);
    const int tc = s_top_cnt;
    if (tc > 1) {
      const int len = pow2_at_least(tc);
      for (int e = tc + tid; e < len; e += kSelThreads) topbuf[e] = 0ull;
      __syncthreads();
      bitonic_desc(topbuf, len);
    }
    __syncthreads();
    nsel = tc < p.k_eff ? tc : p.k_eff;
    for (int w = tid; w < nsel; w += kSelThreads) stage[w] = static_cast<int32_t>(key_index(topbuf[w]));
  }
  __syncthreads();
  if (nsel < p.k_eff) scan_bits(bitmap, words, live, p.n, false, stage + nsel, p.k_eff - nsel, s_scan);
  __syncthreads();

  const int64_t obase = ((bb * p.n + i) * p.h_kv + h) * p.top_k;
  if (p.out_i64) {
    int64_t* out64 = static_cast<int64_t*>(p.out) + obase;
    for (int w = tid; w < p.top_k; w += kSelThreads) out64[w] = (w < p.k_eff) ? stage[w] : 0;
  } else {
    int32_t* out32 = static_cast<int32_t*>(p.out) + obase;
    for (int w = tid; w < p.top_k; w += kSelThreads) out32[w] = (w < p.k_eff) ? stage[w] : 0;
  }
  if (p.stats && tid == 0) {
    p.stats[(bh * p.n + i) * 2 + 0] = s_cand;
    p.stats[(bh * p.n + i) * 2 + 1] = s_R;
  }
}

template <typename T, int GMAX, int D>
__global__ __launch_bounds__(kSelThreads) void select_kernel(SelParams p, const T* __restrict__ qg) {
  select_row<T, GMAX, D>(p, qg, blockIdx.x, false);
}

// The rows select_light_kernel listed (more than k_eff candidates, index
// order): each block takes the next listed row until the list is exhausted.
// ctr[0] = listed rows, ctr[1] = next list position (both from the light pass).
template <typename T, int GMAX, int D>
__global__ __launch_bounds__(kSelThreads) void select_heavy_kernel(SelParams p, const T* __restrict__ qg,
                                                                   const int32_t* __restrict__ list,
                                                                   int32_t* __restrict__ ctr) {
  __shared__ int s_next;
  const int listed = ctr[0];
  for (;;) {
    if (threadIdx.x == 0) s_next = atomicAdd(&ctr[1], 1);
    __syncthreads();
    const int r = s_next;
    __syncthreads();  // every thread holds r before thread 0 takes the next one
    if (r >= listed) break;
    select_row<T, GMAX, D>(p, qg, list[r], true);
    __syncthreads();  // the next row reuses the LDS
  }
}

// Index-order rows, one wave per row, no block barriers: the row's buckets go
// through the wave's LDS bitmap; a row with at most k_eff candidates writes its
// candidates ascending and the filler directly; a row with more is appended
// to `list` (ctr[0] counts them) for select_heavy_kernel.
constexpr int kLightWaves = 4;

__device__ __forceinline__ int wave_excl_scan(int v, int lane, int* total) {
  int x = v;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const int y = __shfl_up(x, o, 64);
    if (lane >= o) x += y;
  }
  *total = __shfl(x, 63);
  return x - v;
}

__global__ __launch_bounds__(64 * kLightWaves) void select_light_kernel(SelParams p, int64_t rows,
                                                                        int32_t* __restrict__ list,
                                                                        int32_t* __restrict__ ctr) {
  extern __shared__ __align__(16) uint32_t lbits[];
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const int64_t row = static_cast<int64_t>(blockIdx.x) * kLightWaves + wave;
  if (row >= rows) return;
  const int words = static_cast<int>((p.n + 31) >> 5);
  uint32_t* bm = lbits + static_cast<int64_t>(wave) * words;
  const int64_t i = row % p.n;
  const int64_t bh = row / p.n;
  const int h = static_cast<int>(bh % p.h_kv);
  const int64_t bb = bh / p.h_kv;
  const int32_t* pp = p.postings + bh * p.n * p.b;
  const bool causal = p.mask_mode == SSA_MASK_CAUSAL;
  const uint8_t* mrow = (p.mask_mode == SSA_MASK_DENSE) ? p.mask + bb * p.mask_sb + i * p.mask_si : nullptr;
  const int live = causal ? static_cast<int>(i >> 5) + 1 : words;
  for (int w = lane; w < live; w += 64) bm[w] = 0u;

  int32_t lo = 0, len = 0;
  if (lane < p.a) {
    const int32_t c = p.q_codes[(bh * p.n + i) * p.a + lane];
    if (static_cast<uint32_t>(c) < static_cast<uint32_t>(p.n_c)) {
      const int32_t* off = p.offsets + bh * (p.n_c + 1);
      const int32_t total = static_cast<int32_t>(p.n * p.b);
      lo = min(max(off[c], 0), total);
      len = min(max(off[c + 1], lo), total) - lo;
    }
  }
  __builtin_amdgcn_wave_barrier();
  int fresh = 0, seen = 0;  // per lane: new keys, postings inside the window
  for (int m = 0; m < p.a; ++m) {
    const int lo_m = __shfl(lo, m), len_m = __shfl(len, m);
    for (int base = 0; base < len_m; base += 64) {
      if (base + lane < len_m) {
        const int32_t j = pp[lo_m + base + lane];
        const bool in_window = !causal || j <= i;
        seen += in_window ? 1 : 0;
        if (static_cast<uint32_t>(j) < static_cast<uint32_t>(p.n) && in_window &&
            (mrow == nullptr || mrow[j] != 0)) {
          const uint32_t bit = 1u << (j & 31);
          if (!(atomicOr(&bm[j >> 5], bit) & bit)) ++fresh;
        }
      }
    }
  }
  int C = 0, raw = 0;
  wave_excl_scan(fresh, lane, &C);
  if (p.stats) wave_excl_scan(seen, lane, &raw);
  if (p.stats && lane == 0) {
    p.stats[(bh * p.n + i) * 2 + 0] = C;
    p.stats[(bh * p.n + i) * 2 + 1] = raw;
  }
  if (C > p.k_eff) {
    if (lane == 0) list[atomicAdd(&ctr[0], 1)] = static_cast<int32_t>(row);
    return;
  }
  __builtin_amdgcn_wave_barrier();

  const int64_t obase = ((bb * p.n + i) * p.h_kv + h) * p.top_k;
  int32_t* o32 = static_cast<int32_t*>(p.out) + obase;
  int64_t* o64 = static_cast<int64_t*>(p.out) + obase;
  auto put = [&](int pos, int32_t v) {
    if (p.out_i64) o64[pos] = v;
    else o32[pos] = v;
  };
  // Candidates ascending, then the lowest non-candidates up to k_eff.
  int filled = 0;
  for (int w0 = 0; w0 < live && filled < C; w0 += 64) {
    const int w = w0 + lane;
    uint32_t bits = (w < live) ? bm[w] : 0u;
    int total = 0;
    int pos = filled + wave_excl_scan(__popc(bits), lane, &total);
    while (bits != 0u) {
      put(pos++, w * 32 + __ffs(bits) - 1);
      bits &= bits - 1u;
    }
    filled += total;
  }
  for (int w0 = 0; filled < p.k_eff; w0 += 64) {
    const int w = w0 + lane;
    uint32_t bits = 0u;
    if (w < words) {
      bits = ~((w < live) ? bm[w] : 0u);
      if (w == words - 1 && (p.n & 31)) bits &= (1u << (p.n & 31)) - 1u;
    }
    int total = 0;
    int pos = filled + wave_excl_scan(__popc(bits), lane, &total);
    while (bits != 0u && pos < p.k_eff) {
      put(pos++, w * 32 + __ffs(bits) - 1);
      bits &= bits - 1u;
    }
    filled += total;
  }
  for (int w = p.k_eff + lane; w < p.top_k; w += 64) put(w, 0);
}

__global__ void zero_ctr_kernel(int32_t* __restrict__ ctr) {
  if (threadIdx.x < 2) ctr[threadIdx.x] = 0;
}

size_t light_smem(int64_t n) { return sizeof(uint32_t) * kLightWaves * static_cast<size_t>((n + 31) / 32); }

int heavy_grid(int64_t rows) {
  static int cus[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) dev = 0;
  if (cus[dev] == 0) {
    int c = 0;
    if (hipDeviceGetAttribute(&c, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || c <= 0) c = 256;
    cus[dev] = c;
  }
  const int64_t g = static_cast<int64_t>(cus[dev]) * 8;
  return static_cast<int>(rows < g ? rows : g);
}

// ws (nullable): index order through the light/heavy pair; otherwise one block
// per row.
template <typename T, int GMAX, int D>
int launch_select(const SelParams& p, int64_t rows, size_t smem, int32_t* ws, hipStream_t st) {
  auto kern = select_kernel<T, GMAX, D>;
  if (int s = reserve_lds(reinterpret_cast<const void*>(kern), smem, "select")) return s;
  const T* qg = static_cast<const T*>(p.q);
  if (ws == nullptr || p.sorted || light_smem(p.n) > 64 * 1024) {
    kern<<<dim3(static_cast<unsigned>(rows)), kSelThreads, smem, st>>>(p, qg);
    return check_launch("select_kernel");
  }
  int32_t* ctr = ws;
  int32_t* list = ws + 64;
  zero_ctr_kernel<<<1, 64, 0, st>>>(ctr);
  if (int s = check_launch("zero_ctr_kernel")) return s;
  select_light_kernel<<<dim3(static_cast<unsigned>(ceil_div(rows, kLightWaves))), 64 * kLightWaves,
                        light_smem(p.n), st>>>(p, rows, list, ctr);
  if (int s = check_launch("select_light_kernel")) return s;
  auto hk = select_heavy_kernel<T, GMAX, D>;
  if (int s = reserve_lds(reinterpret_cast<const void*>(hk), smem, "select")) return s;
  hk<<<dim3(static_cast<unsigned>(heavy_grid(rows))), kSelThreads, smem, st>>>(p, qg, list, ctr);
  return check_launch("select_heavy_kernel");
}

template <typename T, int GMAX>
int dispatch_select_d(const SelParams& p, int64_t rows, size_t smem, int32_t* ws, hipStream_t st) {
  switch (p.d) {
    case 64: return launch_select<T, GMAX, 64>(p, rows, smem, ws, st);
    case 128: return launch_select<T, GMAX, 128>(p, rows, smem, ws, st);
    case 256: return launch_select<T, GMAX, 256>(p, rows, smem, ws, st);
    default: return launch_select<T, GMAX, 0>(p, rows, smem, ws, st);
  }
}

template <typename T>
int dispatch_select(const SelParams& p, int64_t rows, size_t smem, int32_t* ws, hipStream_t st) {
  if (p.g <= 4) return dispatch_select_d<T, 4>(p, rows, smem, ws, st);
  if (p.g <= 8) return dispatch_select_d<T, 8>(p, rows, smem, ws, st);
  return dispatch_select_d<T, 16>(p, rows, smem, ws, st);
}

}  // namespace
}  // namespace ssa

using namespace ssa;

extern "C" size_t ssa_select_workspace_bytes(int64_t batch, int64_t n, int h_kv) {
  if (batch < 0 || n < 0 || h_kv <= 0) return 0;
  return align_up(256 + sizeof(int32_t) * static_cast<size_t>(batch * h_kv * n), 256);
}

extern "C" int ssa_select(const void* q, const void* k, int dtype, int64_t batch, int64_t n,
                          int h_q, int h_kv, int d, int64_t q_sb, int64_t q_sn, int64_t q_sh,
                          int64_t k_sb, int64_t k_sn, int64_t k_sh, const int32_t* q_codes, int a,
                          const int32_t* offsets, const int32_t* postings, int n_c, int b,
                          int top_k, int mask_mode, const uint8_t* mask, int64_t mask_sb,
                          int64_t mask_si, float score_div, int sorted, void* out,
                          int out_index_dtype, int32_t* stats, void* workspace,
                          size_t workspace_bytes, void* stream) {
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
  if ((k_sn % vec) || (k_sh % vec) || (k_sb % vec) || (reinterpret_cast<uintptr_t>(k) % 16) ||
      (q_sn % vec) || (q_sh % vec) || (q_sb % vec) || (reinterpret_cast<uintptr_t>(q) % 16))
    return fail(SSA_ERR_UNSUPPORTED, "select: q and k rows must be 16-byte aligned");
  if (workspace && workspace_bytes < ssa_select_workspace_bytes(batch, n, h_kv))
    return fail(SSA_ERR_WORKSPACE, "select: workspace %zu < %zu bytes", workspace_bytes,
                ssa_select_workspace_bytes(batch, n, h_kv));
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
  p.sorted = sorted ? 1 : 0;
  p.mask_mode = mask_mode;
  p.mask = mask;
  p.mask_sb = mask_sb;
  p.mask_si = mask_si;
  p.score_div = score_div;
  p.out = out;
  p.out_i64 = (out_index_dtype == SSA_INDEX_I64);
  p.stats = stats;
  const size_t smem = select_smem(n, p.sortn, p.k_eff);
  if (smem > 160 * 1024)
    return fail(SSA_ERR_UNSUPPORTED, "select: needs %zu bytes of LDS (n=%lld, top_k=%d)", smem,
                static_cast<long long>(n), top_k);
  const int64_t rows = batch * h_kv * n;
  if (rows >= (int64_t(1) << 31)) return fail(SSA_ERR_UNSUPPORTED, "select: too many rows");
  hipStream_t st = as_stream(stream);
  int32_t* ws = static_cast<int32_t*>(workspace);
  if (dtype == SSA_DTYPE_BF16) return dispatch_select<uint16_t>(p, rows, smem, ws, st);
  return dispatch_select<float>(p, rows, smem, ws, st);
}
