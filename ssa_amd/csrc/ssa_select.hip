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
#include <mutex>

#include "ssa_common.h"
#include "ssa_internal.h"
#include "ssa_rows.h"

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
  // Nullable [rows]: X per row, the key prefix [0, X) that the row's indices
  // hold exactly once (its lowest-key filler and the candidates below it);
  // 0 for a row without filler.  Stage (d) attends such prefixes densely.
  int32_t* prefix;
  // Nullable [rows] (workspace): candidates per row, written by the light pass
  // when the score order is wanted (select_sort_kernel reorders the index-order
  // rows afterwards).
  int32_t* cnt;
  int64_t n_q, q_pos0;   // query rows (q, q_codes, out, stats) and the position of row 0
  int64_t rows;          // batch * h_kv * n_q
  const int32_t* order;  // nullable [rows]: slot t of head bh runs query row order[bh * n_q + t]
  // Postings per (batch, kv head) of the index: n * b for an index over every
  // key; fewer when a tail index holds the newest keys (incremental decoding).
  int64_t post_bh;
  // Optional second (tail) index over the keys appended since the main index
  // was built: offsets [bh][n_c + 1], postings [bh][tail_bh] holding key -
  // tail_key0.  A row's candidates are the union over both indices' buckets of
  // its codes; nseg = a without a tail, 2a with one (segment s >= a: tail
  // bucket of code s - a).
  const int32_t* tail_offsets;
  const int32_t* tail_postings;
  int64_t tail_bh;
  int32_t tail_key0;
  int nseg;
  // Screen and pick passes: each XCD walks its own slice of the listed rows
  // (set by the launcher when the (batch, kv head) pairs are at least the
  // XCDs; see shard_walk).
  int xcd_slices;
  // Light pass: bitmap words per chunk of a long window (set by the launcher:
  // kLightChunkWords, or the whole key range as one chunk).
  int light_chunk_words;
  // Light pass: the key positions (q_pos0 + r) of the rows a launch takes,
  // [light_pos_lo, light_pos_hi); the launcher splits a whole-range chunk by
  // position so the early rows run with a half-size bitmap.
  int64_t light_pos_lo, light_pos_hi;
};

// Row ((b * h_kv + h) * n_q + r) processed in slot t of the launch
// (t = bh * n_q + u): r = u, or order[t] when an order is given; -1 for an order
// entry outside [0, n_q).  Query row r sits at key position q_pos0 + r (the
// causal window and the dense mask use the position).
__device__ __forceinline__ int64_t row_of_slot(const SelParams& p, int64_t t) {
  if (p.order == nullptr) return t;
  const int32_t o = p.order[t];
  if (static_cast<uint32_t>(o) >= static_cast<uint64_t>(p.n_q)) return -1;
  return udiv32(t, p.n_q) * p.n_q + o;
}

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
  const int x = wave_incl_scan(v);
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

// rescore_row for two key rows at once (the same chains, interleaved): both
// rows' loads are in flight together and each query operand serves both.
template <typename T, int GMAX, int D>
__device__ __forceinline__ void rescore_rows2(const T* kr0, const T* kr1, const T* q0, int64_t q_sh, int g, int d,
                                              float (&acc0)[GMAX], float (&acc1)[GMAX]) {
#pragma unroll
  for (int gg = 0; gg < GMAX; ++gg) {
    acc0[gg] = 0.0f;
    acc1[gg] = 0.0f;
  }
  constexpr int G = kRescoreLoads;
  const int dd = (D > 0) ? D : d;
#pragma unroll 1
  for (int t0 = 0; t0 < dd; t0 += 8 * G) {
    float kv0[G][8], kv1[G][8];
#pragma unroll
    for (int u = 0; u < G; ++u)
      if (D > 0 || t0 + 8 * u < dd) {
        load8(kr0 + t0 + 8 * u, kv0[u]);
        load8(kr1 + t0 + 8 * u, kv1[u]);
      }
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
        for (int e = 0; e < 8; ++e) {
          acc0[gg] = fma_rn(qv[e], kv0[u][e], acc0[gg]);
          acc1[gg] = fma_rn(qv[e], kv1[u][e], acc1[gg]);
        }
      }
    }
  }
}

// rescore_rows2 with the group's query rows already in LDS as fp32 (qs[gg * D
// + t]): each lane reads them as broadcast float4s instead of reloading and
// converting the bf16 rows for every key pair.  The same fmaf chains.
template <int GMAX, int D>
__device__ __forceinline__ void rescore_rows2_qs(const uint16_t* kr0, const uint16_t* kr1, const float* qs, int g,
                                                 float (&acc0)[GMAX], float (&acc1)[GMAX]) {
#pragma unroll
  for (int gg = 0; gg < GMAX; ++gg) {
    acc0[gg] = 0.0f;
    acc1[gg] = 0.0f;
  }
  constexpr int G = kRescoreLoads;
#pragma unroll 1
  for (int t0 = 0; t0 < D; t0 += 8 * G) {
    float kv0[G][8], kv1[G][8];
#pragma unroll
    for (int u = 0; u < G; ++u) {
      load8(kr0 + t0 + 8 * u, kv0[u]);
      load8(kr1 + t0 + 8 * u, kv1[u]);
    }
#pragma unroll
    for (int gg = 0; gg < GMAX; ++gg) {
      if (gg >= g) continue;
#pragma unroll
      for (int u = 0; u < G; ++u) {
        const float4 a = *reinterpret_cast<const float4*>(qs + gg * D + t0 + 8 * u);
        const float4 b = *reinterpret_cast<const float4*>(qs + gg * D + t0 + 8 * u + 4);
        const float qv[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          acc0[gg] = fma_rn(qv[e], kv0[u][e], acc0[gg]);
          acc1[gg] = fma_rn(qv[e], kv1[u][e], acc1[gg]);
        }
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
  const int64_t bh = udiv32(row, p.n_q);
  const int64_t r = row - bh * p.n_q;
  const int64_t i = p.q_pos0 + r;
  const int64_t bb = udiv32(bh, p.h_kv);
  const int h = static_cast<int>(bh - bb * p.h_kv);
  const T* q0 = qg + bb * p.q_sb + r * p.q_sn + static_cast<int64_t>(h * p.g) * p.q_sh;
  const T* kbase = static_cast<const T*>(p.k) + bb * p.k_sb + static_cast<int64_t>(h) * p.k_sh;
  const int32_t* pp = p.postings + bh * p.post_bh;
  const int32_t* tp = p.tail_postings ? p.tail_postings + bh * p.tail_bh : nullptr;
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
    if (tid < p.nseg) {
      const bool tl = tid >= p.a;
      const int32_t c = p.q_codes[(bh * p.n_q + r) * p.a + (tl ? tid - p.a : tid)];
      if (static_cast<uint32_t>(c) < static_cast<uint32_t>(p.n_c)) {
        const int32_t* off = (tl ? p.tail_offsets : p.offsets) + bh * (p.n_c + 1);
        const int32_t total = static_cast<int32_t>(tl ? p.tail_bh : p.post_bh);
        lo = min(max(off[c], 0), total);
        len = min(max(off[c + 1], lo), total) - lo;
      }
    }
    const int32_t x = wave_incl_scan(len);  // the first wave, all lanes active
    if (tid < p.nseg) {
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
  const int R = seg_start[p.nseg];
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
        int lo_m = 0, hi_m = p.nseg;
        while (hi_m - lo_m > 1) {
          const int mid = (lo_m + hi_m) >> 1;
          if (seg_start[mid] <= pidx) lo_m = mid;
          else hi_m = mid;
        }
        const int32_t e = seg_lo[lo_m] + (pidx - seg_start[lo_m]);
        const int32_t j = lo_m < p.a ? pp[e] : tp[e] + p.tail_key0;
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

  const int64_t obase = ((bb * p.n_q + r) * p.h_kv + h) * p.top_k;
  if (p.out_i64) {
    int64_t* out64 = static_cast<int64_t*>(p.out) + obase;
    for (int w = tid; w < p.top_k; w += kSelThreads) out64[w] = (w < p.k_eff) ? stage[w] : 0;
  } else {
    int32_t* out32 = static_cast<int32_t*>(p.out) + obase;
    for (int w = tid; w < p.top_k; w += kSelThreads) out32[w] = (w < p.k_eff) ? stage[w] : 0;
  }
  if (p.stats && tid == 0) {
    p.stats[(bh * p.n_q + r) * 2 + 0] = s_cand;
    p.stats[(bh * p.n_q + r) * 2 + 1] = s_R;
  }
  // the filler stage[nsel .. k_eff) is the lowest keys the row does not hold:
  // every key up to its last one is in the row once (see select_light_kernel)
  if (p.prefix && tid == 0)
    p.prefix[row] = (nsel < p.k_eff && p.k_eff == p.top_k) ? stage[p.k_eff - 1] + 1 : 0;
}

// Score order through the index-order passes: a row's first m = min(C, k_eff)
// slots hold its selected keys ascending; select_sort_kernel (one wave per
// row) rescores them in the canonical order (rescore_row, lane l taking keys
// l, l + 64, ...), sorts the composite keys (score desc, index asc -- unique,
// so the order is total) with the register bitonic network below and writes
// them back; the filler after them keeps its ascending order, as in
// select_kernel.
constexpr int kSortMax = 1024;  // m at most this (k_eff larger: select_kernel)

// Bitonic network of one wave over 64 E keys in registers (lane l holds keys
// l E + r): exchanges between the slots of one lane run in registers, between
// lanes through DPP (lane ^ 1, ^ 2), ds_swizzle (^ 4, ^ 8, ^ 16) or
// ds_bpermute (^ 32).
__device__ __forceinline__ uint32_t lane_xor(uint32_t v, int lx) {
  switch (lx) {
    case 1: return static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(v), 0xB1, 0xF, 0xF, false));
    case 2: return static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(v), 0x4E, 0xF, 0xF, false));
    case 4: return static_cast<uint32_t>(__builtin_amdgcn_ds_swizzle(static_cast<int>(v), 0x101F));
    case 8: return static_cast<uint32_t>(__builtin_amdgcn_ds_swizzle(static_cast<int>(v), 0x201F));
    case 16: return static_cast<uint32_t>(__builtin_amdgcn_ds_swizzle(static_cast<int>(v), 0x401F));
    default: return static_cast<uint32_t>(__shfl_xor(static_cast<int>(v), lx));
  }
}

// Descending bitonic sort of the wave's 64 E keys, key l E + r in x[r] of lane l.
template <int E>
__device__ __forceinline__ void wave_sort_desc(uint64_t (&x)[E], int lane) {
#pragma unroll
  for (int size = 2; size <= 64 * E; size <<= 1) {
#pragma unroll
    for (int stride = size >> 1; stride > 0; stride >>= 1) {
      // One 64-bit compare per exchange: the direction enters as an equality
      // with the comparison (keys are distinct apart from the zero padding,
      // and equal keys may be swapped).
      if (stride >= E) {  // partner: the same slot of lane ^ (stride / E)
        // r < E <= stride, so the stride and size bits of lane * E + r are
        // those of lane * E: one direction for all of the lane's slots
        const bool keep_max = (((lane * E) & stride) == 0) == (((lane * E) & size) == 0);
#pragma unroll
        for (int r = 0; r < E; ++r) {
          const uint32_t lo = lane_xor(static_cast<uint32_t>(x[r]), stride / E);
          const uint32_t hi = lane_xor(static_cast<uint32_t>(x[r] >> 32), stride / E);
          const uint64_t y = (static_cast<uint64_t>(hi) << 32) | lo;
          x[r] = ((y > x[r]) == keep_max) ? y : x[r];
        }
      } else {  // partner: slot r ^ stride of this lane
#pragma unroll
        for (int r = 0; r < E; ++r) {
          if (r & stride) continue;
          const int r2 = r | stride;
          const bool desc = ((lane * E + r) & size) == 0;
          const uint64_t a = x[r], b = x[r2];
          const bool sw = (a < b) == desc;
          x[r] = sw ? b : a;
          x[r2] = sw ? a : b;
        }
      }
    }
  }
}

template <int E>
__device__ __forceinline__ void sort_slots_desc(uint64_t* keys, int lane) {
  uint64_t x[E];
#pragma unroll
  for (int r = 0; r < E; ++r) x[r] = keys[lane * E + r];
  wave_sort_desc<E>(x, lane);
#pragma unroll
  for (int r = 0; r < E; ++r) keys[lane * E + r] = x[r];
}


template <typename T, int GMAX, int D>
__global__ __launch_bounds__(64) void select_sort_kernel(SelParams p, const T* __restrict__ qg) {
  __shared__ uint64_t keys[kSortMax];
  // bf16 inputs of a fixed head dim: the group's query rows as fp32, once per row
  constexpr bool kQs = sizeof(T) == 2 && D > 0;
  __shared__ __align__(16) float qs[kQs ? GMAX * D : 4];
  const int lane = threadIdx.x;
  const int64_t row = row_of_slot(p, blockIdx.x);
  if (row < 0) return;
  const int m = min(p.cnt[row], p.k_eff);
  if (m <= 1) return;
  const int64_t bh = udiv32(row, p.n_q);
  const int64_t r = row - bh * p.n_q;
  const int64_t bb = udiv32(bh, p.h_kv);
  const int h = static_cast<int>(bh - bb * p.h_kv);
  const T* q0 = qg + bb * p.q_sb + r * p.q_sn + static_cast<int64_t>(h * p.g) * p.q_sh;
  const T* kbase = static_cast<const T*>(p.k) + bb * p.k_sb + static_cast<int64_t>(h) * p.k_sh;
  const int64_t obase = ((bb * p.n_q + r) * p.h_kv + h) * p.top_k;
  int32_t* o32 = static_cast<int32_t*>(p.out) + obase;
  int64_t* o64 = static_cast<int64_t*>(p.out) + obase;
  int np = 64;
  while (np < m) np <<= 1;
  if constexpr (kQs) {
    for (int x = lane; x < p.g * (D / 8); x += 64) {
      const int gg = x / (D / 8), t = (x % (D / 8)) * 8;
      float v[8];
      load8(reinterpret_cast<const uint16_t*>(q0) + static_cast<int64_t>(gg) * p.q_sh + t, v);
      *reinterpret_cast<float4*>(qs + gg * D + t) = make_float4(v[0], v[1], v[2], v[3]);
      *reinterpret_cast<float4*>(qs + gg * D + t + 4) = make_float4(v[4], v[5], v[6], v[7]);
    }
    __syncthreads();
  }
  auto score_of = [&](const float (&acc)[GMAX]) {
    float sc = acc[0] / p.score_div;
#pragma unroll
    for (int gg = 1; gg < GMAX; ++gg)
      if (gg < p.g) sc = sc + acc[gg] / p.score_div;
    return sc / static_cast<float>(p.g);
  };
  // slots e and e + 64 together; padding (0) sorts below every real key
  for (int e = lane; e < np; e += 128) {
    const int e2 = e + 64;
    const int32_t j0 = e < m ? (p.out_i64 ? static_cast<int32_t>(o64[e]) : o32[e]) : -1;
    const int32_t j1 = e2 < m ? (p.out_i64 ? static_cast<int32_t>(o64[e2]) : o32[e2]) : -1;
    if (j0 >= 0) {
      float acc0[GMAX], acc1[GMAX];
      if constexpr (kQs)
        rescore_rows2_qs<GMAX, D>(reinterpret_cast<const uint16_t*>(kbase) + static_cast<int64_t>(j0) * p.k_sn,
                                  reinterpret_cast<const uint16_t*>(kbase) +
                                      static_cast<int64_t>(j1 >= 0 ? j1 : j0) * p.k_sn,
                                  qs, p.g, acc0, acc1);
      else
        rescore_rows2<T, GMAX, D>(kbase + static_cast<int64_t>(j0) * p.k_sn,
                                  kbase + static_cast<int64_t>(j1 >= 0 ? j1 : j0) * p.k_sn, q0, p.q_sh, p.g, p.d,
                                  acc0, acc1);
      keys[e] = composite_key(score_of(acc0), static_cast<uint32_t>(j0));
      if (e2 < np) keys[e2] = j1 >= 0 ? composite_key(score_of(acc1), static_cast<uint32_t>(j1)) : 0ull;
    } else {
      keys[e] = 0ull;
      if (e2 < np) keys[e2] = 0ull;
    }
  }
  __syncthreads();
  // descending over np keys (np / 64 per lane, in registers)
  switch (np >> 6) {
    case 1: sort_slots_desc<1>(keys, lane); break;
    case 2: sort_slots_desc<2>(keys, lane); break;
    case 4: sort_slots_desc<4>(keys, lane); break;
    case 8: sort_slots_desc<8>(keys, lane); break;
    default: sort_slots_desc<16>(keys, lane); break;
  }
  __syncthreads();
  for (int e = lane; e < m; e += 64) {
    const int32_t j = static_cast<int32_t>(key_index(keys[e]));
    if (p.out_i64) o64[e] = j;
    else o32[e] = j;
  }
}

template <typename T, int GMAX, int D>
__global__ __launch_bounds__(kSelThreads) void select_kernel(SelParams p, const T* __restrict__ qg) {
  const int64_t row = row_of_slot(p, blockIdx.x);
  if (row >= 0) select_row<T, GMAX, D>(p, qg, row, false);
}

// Workspace of index order (carve_sel_ws).  Rows with more than k candidates
// are listed in kShards shards (light-pass block b writes shard b % kShards),
// each with its own counters and slice of the list space, so no counter is hit
// by more than a 1/kShards share of the rows.
//   ctr    int32: [0] rows for the exact pass, [1] its cursor; shard s at
//          ctr + 16 + 4 s: [0] screened rows, [2..3] int64 list entries used
//   exact  int32 [rows]: rows for select_heavy_kernel
//   scr    int32 [kShards][shard_rows][3]: (row, list offset, candidates)
//   emax   float [kShards][shard_rows]: the screen's error bound per entry
//   cnt    int32 [rows]: candidates per row (score order: for the sort pass)
//   cand   int32 [kShards][cap]: screened rows' candidates, ascending
//   approx float [kShards][cap]: their approximate scores
constexpr int kShards = 64;
constexpr int kScrWaves = 4;    // waves per block of the screen
constexpr int kScrBorder = 64;  // keys near the k-th score rescored exactly per row (more: exact pass)
constexpr int kScrRegs = 48;    // scores held per lane: rows of at most 64 * kScrRegs candidates
constexpr int kPickRegs = 32;   // the pick pass's scores per lane in LDS (longer rows read the workspace)

struct SelWs {
  int32_t* ctr;
  int32_t* exact;
  int32_t* scr;
  int32_t* cand;
  float* approx;
  float* emax;         // [kShards][shard_rows]: the screen's error bound per row (inf: exact pass)
  int32_t* cnt;        // [rows]
  int64_t shard_rows;  // scr entries per shard
  int64_t cap;         // list entries per shard (0: no screen)
};

constexpr size_t kSelCtrBytes = 2048;
static_assert(sizeof(int32_t) * (16 + 4 * kShards) <= kSelCtrBytes, "counter region too small");

// Appends a row for the exact pass (every row is appended at most once, so the
// list of `rows` entries cannot overflow; the check keeps any write in bounds).
__device__ __forceinline__ void push_exact(const SelWs& w, int64_t rows, int64_t row) {
  const int x = atomicAdd(&w.ctr[0], 1);
  if (x >= 0 && x < rows) w.exact[x] = static_cast<int32_t>(row);
}

// The list entries a wave of the screen or pick pass takes (shard, entries
// first, first + step, ... below end).  The grid is a whole number of kXcds x
// kShards / kScrWaves blocks.
//   xcd_slices: each XCD (the launched block b runs on XCD b mod kXcds) walks
//     the same eighth of every shard's list, and a shard's list is in
//     light-pass order, so the rows one XCD works on lie in one slice of the
//     row order (about one (batch, KV head)'s rows when there are at least
//     kXcds of them) and their key rows share that XCD's L2;
//   otherwise wave gw of the grid walks shard gw mod kShards from entry
//     gw / kShards with a step of the grid's waves / kShards, so all XCDs work
//     in the same part of the row order at a time.
struct ShardWalk {
  int shard, first, step, end;
};
__device__ __forceinline__ ShardWalk shard_walk(const SelWs& w, int wave, bool xcd_slices) {
  ShardWalk sw;
  if (xcd_slices) {
    const int xcd = static_cast<int>(blockIdx.x % kXcds);
    const int lw = static_cast<int>(blockIdx.x / kXcds) * kScrWaves + wave;
    const int wx = static_cast<int>(gridDim.x / kXcds) * kScrWaves;
    sw.shard = lw % kShards;
    const int64_t listed = min(static_cast<int64_t>(w.ctr[16 + 4 * sw.shard]), w.shard_rows);
    sw.first = static_cast<int>(listed * xcd / kXcds) + lw / kShards;
    sw.step = wx / kShards;
    sw.end = static_cast<int>(listed * (xcd + 1) / kXcds);
  } else {
    const int gw = static_cast<int>(blockIdx.x) * kScrWaves + wave;
    sw.shard = gw % kShards;
    sw.first = gw / kShards;
    sw.step = static_cast<int>(gridDim.x) * kScrWaves / kShards;
    sw.end = static_cast<int>(min(static_cast<int64_t>(w.ctr[16 + 4 * sw.shard]), w.shard_rows));
  }
  return sw;
}

// The rows listed for the exact pass: each block takes the next listed row
// until the list is exhausted (ctr[0] rows, cursor ctr[1]).
template <typename T, int GMAX, int D>
__global__ __launch_bounds__(kSelThreads) void select_heavy_kernel(SelParams p, const T* __restrict__ qg,
                                                                   SelWs w) {
  __shared__ int s_next;
  const int listed = static_cast<int>(min(static_cast<int64_t>(w.ctr[0]), p.rows));
  // Blocks that find the list empty or used up leave without an atomic: the
  // same-address atomics of a grid of blocks serialize (about 25 us for the
  // 2048 blocks of an empty list at c3); the cursor is read from L2 first.
  if (listed <= 0) return;
  for (;;) {
    if (threadIdx.x == 0) {
      const int seen = __hip_atomic_load(&w.ctr[1], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      s_next = (seen >= listed) ? listed : atomicAdd(&w.ctr[1], 1);
    }
    __syncthreads();
    const int r = s_next;
    __syncthreads();  // every thread holds r before thread 0 takes the next one
    if (r >= listed) break;
    select_row<T, GMAX, D>(p, qg, w.exact[r], true);
    __syncthreads();  // the next row reuses the LDS
  }
}

// Index-order rows, one wave per row, no block barriers: the row's buckets go
// through the wave's LDS bitmap; a row with at most k_eff candidates writes its
// candidates ascending and the filler directly.  A causal window of up to
// kFlatWords bitmap words (32768 keys) uses a flat bitmap, cleared and read back
// whole.  A longer window goes in chunks of 65536 keys through one chunk-sized
// bitmap with a summary level (bit x: bitmap word x was touched by this row):
// both are cleared per chunk (16-byte stores, no waits), and the candidates are
// read back from the touched words only.  Each bucket keeps a cursor, so its
// ascending postings are marked once over the chunks; chunk 0's first words
// are kept for the filler.  The LDS per wave is thus bounded (9.5 KB) for any
// n: a bitmap of the whole window (16 KB at n = 131072) let only 9 waves of
// this pass share a CU there.  A row with more than k_eff candidates writes
// its list into the workspace for select_screen_kernel when it fits (w.cap;
// a chunked row marks its window a second time for that), and is listed for
// the exact pass otherwise.  One wave per block, so no row waits for a longer
// one before its LDS is released.
constexpr int kFlatWords = 1024;  // windows of up to 32768 keys use the flat bitmap
constexpr int kLightBatch = 4;    // buckets whose postings load together
constexpr int kFillWords = 2 * 4096 / 32 + 8;     // filler words kept from chunk 0 (top_k <= 4096)

__device__ __forceinline__ int wave_excl_scan(int v, int lane, int* total) {
  (void)lane;
  const int x = wave_incl_scan(v);
  *total = __builtin_amdgcn_readlane(x, 63);
  return x - v;
}

// Summary words of a chunk of `cwords` bitmap words (one bit per word, padded
// to 4 words).
__host__ __device__ inline int light_chunk_summary(int cwords) { return ((cwords + 31) / 32 + 3) & ~3; }
// LDS words per wave: the flat bitmap of a window up to kFlatWords words, and
// for longer windows one chunk's summary and bitmap plus the filler words.
__host__ __device__ inline int light_words(int64_t n, int cwords) {
  const int64_t words = (n + 31) / 32;
  if (words <= kFlatWords) return static_cast<int>(words);
  // one chunk over all keys keeps its bitmap for the filler: no copy
  return light_chunk_summary(cwords) + cwords + (cwords < words ? kFillWords : 0);
}
// Chunk size of the light pass for n keys: kLightChunkWords (65536 keys, or
// the whole range when shorter) when a row's postings are few (estimated
// nseg * post_bh / n_c <= kLightChunkPostings), so that the chunk bitmap keeps
// enough waves per CU (n = 131072, 16 codes of 32 postings: light pass 5.9 ->
// 5.1 ms with 32768-key chunks; 65536-key chunks halve the chunk passes, each
// of which reloads the row's buckets: stage (c) 8.93 -> 8.61 ms there, and
// 3.50 -> 3.03 ms at n = 65536, one chunk); the whole key range as one chunk
// when they are many (c5: 32 codes of 64 postings), where the rows are long
// enough to hide their latency at low occupancy and chunking would mark the
// windows of the rows with more than k candidates twice.
constexpr double kLightChunkPostings = 1024.0;
constexpr size_t kLdsBytesPerCu = 160 * 1024;
constexpr int kLightChunkWords = 2 * kFlatWords;
inline int light_chunk_words(const SelParams& p) {
  const int64_t words = (p.n + 31) / 32;
  if (words <= kFlatWords) return kFlatWords;
  const double ppr = static_cast<double>(p.nseg) * static_cast<double>(p.post_bh + p.tail_bh) /
                     static_cast<double>(p.n_c);
  return ppr <= kLightChunkPostings ? static_cast<int>(min(words, static_cast<int64_t>(kLightChunkWords)))
                                    : static_cast<int>(words);
}

// Writes the row's candidates (the set bits of the touched bitmap words) in
// ascending order through sink(pos, key) and returns their number.  Lane l
// takes summary words s0 + l of each chunk of 64: it counts the bits of its
// touched words, an exclusive scan over the lanes gives its first position,
// and it writes its keys; lane order is key order within a chunk.
template <typename Sink>
__device__ __forceinline__ int light_emit(const uint32_t* sm, const uint32_t* bm, int slive, int lane, Sink&& sink) {
  int filled = 0;
  for (int s0 = 0; s0 < slive; s0 += 64) {
    const int sx = s0 + lane;
    const uint32_t sbits = (sx < slive) ? sm[sx] : 0u;
    int cnt = 0;
    for (uint32_t t = sbits; t != 0u; t &= t - 1u) cnt += __popc(bm[sx * 32 + __ffs(t) - 1]);
    int total = 0;
    int pos = filled + wave_excl_scan(cnt, lane, &total);
    for (uint32_t t = sbits; t != 0u; t &= t - 1u) {
      const int x = sx * 32 + __ffs(t) - 1;
      for (uint32_t bits = bm[x]; bits != 0u; bits &= bits - 1u) sink(pos++, x * 32 + __ffs(bits) - 1);
    }
    filled += total;
  }
  return filled;
}

// The same from the flat bitmap words [0, live).
template <typename Sink>
__device__ __forceinline__ int light_emit_flat(const uint32_t* bm, int live, int lane, Sink&& sink) {
  int filled = 0;
  for (int w0 = 0; w0 < live; w0 += 64) {
    const int x = w0 + lane;
    uint32_t bits = (x < live) ? bm[x] : 0u;
    int total = 0;
    int pos = filled + wave_excl_scan(__popc(bits), lane, &total);
    for (; bits != 0u; bits &= bits - 1u) sink(pos++, x * 32 + __ffs(bits) - 1);
    filled += total;
  }
  return filled;
}

// MINW: waves per SIMD the build must allow (amdgpu_waves_per_eu).  8 when a
// wave's bitmap is small enough for 32 waves per CU (the flat windows of n up
// to about 40K keys): the build then keeps to 78 SGPRs (spilling some to VGPR
// lanes) instead of the 106 that allow 7.  Longer windows are bound by their
// LDS bitmaps and keep the unconstrained build.
template <int MINW>
__global__ __launch_bounds__(64) __attribute__((amdgpu_waves_per_eu(MINW, 8))) void select_light_kernel(
    SelParams p, int64_t rows, SelWs w) {
  extern __shared__ __align__(16) uint32_t lbits[];
  const int lane = threadIdx.x & 63;
  const int64_t slot = blockIdx.x;
  if (slot >= rows) return;
  const int64_t row = row_of_slot(p, slot);
  if (row < 0) return;
  const int words = static_cast<int>((p.n + 31) >> 5);
  const int64_t bh = udiv32(row, p.n_q);
  const int64_t r = row - bh * p.n_q;
  const int64_t i = p.q_pos0 + r;
  if (i < p.light_pos_lo || i >= p.light_pos_hi) return;  // the other launch's row
  const int64_t bb = udiv32(bh, p.h_kv);
  const int h = static_cast<int>(bh - bb * p.h_kv);
  const int32_t* pp = p.postings + bh * p.post_bh;
  const int32_t* tp = p.tail_postings ? p.tail_postings + bh * p.tail_bh : nullptr;
  const bool causal = p.mask_mode == SSA_MASK_CAUSAL;
  const uint8_t* mrow = (p.mask_mode == SSA_MASK_DENSE) ? p.mask + bb * p.mask_sb + i * p.mask_si : nullptr;
  const int live = causal ? static_cast<int>(i >> 5) + 1 : words;
  const bool flat = live <= kFlatWords;
  // flat: the bitmap of the window; chunked: one chunk's summary and bitmap,
  // then the filler words (a copy of chunk 0's first fwn words)
  const int cwords = p.light_chunk_words;                  // bitmap words per chunk
  const int csum = light_chunk_summary(cwords);
  uint32_t* sm = lbits;
  uint32_t* bm = flat ? lbits : lbits + csum;
  uint32_t* fw = lbits + csum + cwords;
  const int fwn = min(words, (2 * p.k_eff + 31) / 32 + 1);
  const int64_t wend = static_cast<int64_t>(live) * 32;  // keys of the window's words

  int32_t lo = 0, len = 0;
  if (lane < p.nseg) {
    const bool tl = lane >= p.a;
    const int32_t c = p.q_codes[(bh * p.n_q + r) * p.a + (tl ? lane - p.a : lane)];
    if (static_cast<uint32_t>(c) < static_cast<uint32_t>(p.n_c)) {
      const int32_t* off = (tl ? p.tail_offsets : p.offsets) + bh * (p.n_c + 1);
      const int32_t total = static_cast<int32_t>(tl ? p.tail_bh : p.post_bh);
      lo = min(max(off[c], 0), total);
      len = min(max(off[c + 1], lo), total) - lo;
    }
  }
  int fresh = 0, seen = 0;  // per lane: new keys, postings inside the window
  // Buffer descriptors of this (batch, kv head)'s postings (the host keeps
  // them below 2^31 entries); no tail index: an empty range.
  const __amdgpu_buffer_rsrc_t prs = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<int32_t*>(pp), 0, static_cast<int>(min(p.post_bh * 4, int64_t(0x7FFFFFFF))), kBufferWord3);
  const __amdgpu_buffer_rsrc_t trs = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<int32_t*>(tp ? tp : pp), 0, tp ? static_cast<int>(min(p.tail_bh * 4, int64_t(0x7FFFFFFF))) : 0,
      kBufferWord3);

  const int64_t obase = ((bb * p.n_q + r) * p.h_kv + h) * p.top_k;
  int32_t* o32 = static_cast<int32_t*>(p.out) + obase;
  int64_t* o64 = static_cast<int64_t*>(p.out) + obase;
  auto put = [&](int pos, int32_t v) {
    if (p.out_i64) o64[pos] = v;
    else o32[pos] = v;
  };

  // Marks the row's window keys in [kbeg, kend) (bits relative to kbeg) and,
  // for a chunk, its summary, and counts (when `count`) the postings inside the
  // window.
  // Buckets go kLightBatch at a time, their postings loaded together before
  // any is marked (the bitmap, the counts and the summary do not depend on the
  // order).  cur_lo / cur_len (lane m: bucket m) are the bucket cursors: the
  // postings below kend are consumed and the cursors advance past them, so
  // chunk after chunk every posting is marked once (postings ascend inside a
  // bucket).  A flat window is one chunk [0, wend).
  int32_t cur_lo = lo, cur_len = len;
  const bool half_buckets = tp == nullptr && p.post_bh <= int64_t(32) * p.n_c;
  auto mark_range = [&](int64_t kbeg, int64_t kend, bool summary, bool count, bool cursors)
                        __attribute__((always_inline)) {
    auto add = [&](int32_t j) __attribute__((always_inline)) {
      const bool in_window = !causal || j <= i;
      if (count) seen += in_window ? 1 : 0;
      if (static_cast<uint32_t>(j) < static_cast<uint32_t>(p.n) && in_window &&
          (mrow == nullptr || mrow[j] != 0)) {
        const int jr = static_cast<int>(j - kbeg);
        const int x = jr >> 5;
        // no atomic's return is waited for: the bitmap was cleared before the
        // marking, and the new keys are counted from it afterwards
        if (summary) atomicOr(&sm[x >> 5], 1u << (x & 31));
        atomicOr(&bm[x], 1u << (jr & 31));
      }
    };
    if (!cursors) {
      // The whole window in one chunk: every posting of every bucket.  With
      // buckets of at most 32 postings on average and no tail index, each
      // half-wave takes a bucket (two per load), so half the lanes are not
      // idle on short buckets.
      if (half_buckets) {
        const int sub = lane >> 5, ll = lane & 31;
        for (int m0 = 0; m0 < p.nseg; m0 += 2 * kLightBatch) {
          int lo_u[kLightBatch], len_u[kLightBatch], most = 0;
#pragma unroll
          for (int u = 0; u < kLightBatch; ++u) {
            const int b = m0 + 2 * u + sub;
            lo_u[u] = __shfl(lo, min(b, 63));
            len_u[u] = (b < p.nseg) ? __shfl(len, min(b, 63)) : 0;
            most = max(most, len_u[u]);
          }
          for (int base = 0; __ballot(base + ll < most) != 0ull; base += 32) {
            int32_t j_u[kLightBatch];
#pragma unroll
            for (int u = 0; u < kLightBatch; ++u) {
              const int e = lo_u[u] + min(base + ll, len_u[u] - 1);
              j_u[u] = __builtin_amdgcn_raw_buffer_load_b32(prs, e * 4, 0, 0);
            }
#pragma unroll
            for (int u = 0; u < kLightBatch; ++u)
              if (base + ll < len_u[u]) add(j_u[u]);
          }
        }
        return;
      }
      for (int m0 = 0; m0 < p.nseg; m0 += kLightBatch) {
        int lo_u[kLightBatch], len_u[kLightBatch], most = 0;
#pragma unroll
        for (int u = 0; u < kLightBatch; ++u) {
          lo_u[u] = __shfl(lo, min(m0 + u, 63));
          len_u[u] = (m0 + u < p.nseg) ? __shfl(len, min(m0 + u, 63)) : 0;
          most = max(most, len_u[u]);
        }
        for (int base = 0; base < most; base += 64) {
          // Every lane loads, with no branch (past a bucket's end it reloads
          // the bucket's last posting; an empty bucket reads out of the
          // buffer's range, which loads 0), so all kLightBatch loads are out
          // before the first add.
          int32_t j_u[kLightBatch];
#pragma unroll
          for (int u = 0; u < kLightBatch; ++u) {
            const int e = lo_u[u] + min(base + lane, len_u[u] - 1);
            j_u[u] = __builtin_amdgcn_raw_buffer_load_b32(m0 + u < p.a ? prs : trs, e * 4, 0, 0);
          }
#pragma unroll
          for (int u = 0; u < kLightBatch; ++u)
            if (base + lane < len_u[u]) add(m0 + u < p.a ? j_u[u] : j_u[u] + p.tail_key0);
        }
      }
      return;
    }
    if (half_buckets) {
      // The cursor loop with a bucket per half-wave, as above: a half takes
      // its bucket's postings below kend 32 at a time; its ballot half counts
      // them, and lane m0 + 2u + s advances bucket m0 + 2u + s's cursor by the
      // count of half s.
      const int sub = lane >> 5, ll = lane & 31;
      for (int m0 = 0; m0 < p.nseg; m0 += 2 * kLightBatch) {
        int lo_u[kLightBatch], len_u[kLightBatch], took[kLightBatch];
#pragma unroll
        for (int u = 0; u < kLightBatch; ++u) {
          const int b = m0 + 2 * u + sub;
          lo_u[u] = __shfl(cur_lo, min(b, 63));
          len_u[u] = (b < p.nseg) ? __shfl(cur_len, min(b, 63)) : 0;
          took[u] = 0;
        }
        for (int base = 0;; base += 32) {
          int32_t j_u[kLightBatch];
#pragma unroll
          for (int u = 0; u < kLightBatch; ++u) {
            const int e = lo_u[u] + min(base + ll, len_u[u] - 1);
            j_u[u] = __builtin_amdgcn_raw_buffer_load_b32(prs, e * 4, 0, 0);
          }
          bool more = false;
#pragma unroll
          for (int u = 0; u < kLightBatch; ++u) {
            const bool in_range = base + ll < len_u[u] && j_u[u] < kend;
            const uint32_t half = static_cast<uint32_t>(__ballot(in_range) >> (32 * sub));
            took[u] += __popc(half);
            more = more || half == 0xFFFFFFFFu;
            if (in_range) add(j_u[u]);
          }
          if (__ballot(more) == 0ull) break;
        }
#pragma unroll
        for (int u = 0; u < kLightBatch; ++u) {
          const int t0 = __shfl(took[u], 0), t1 = __shfl(took[u], 32);
          if (lane == m0 + 2 * u) {
            cur_lo += t0;
            cur_len -= t0;
          }
          if (lane == m0 + 2 * u + 1) {
            cur_lo += t1;
            cur_len -= t1;
          }
        }
      }
      return;
    }
    for (int m0 = 0; m0 < p.nseg; m0 += kLightBatch) {
      int lo_u[kLightBatch], len_u[kLightBatch], took[kLightBatch];
#pragma unroll
      for (int u = 0; u < kLightBatch; ++u) {
        lo_u[u] = __shfl(cur_lo, min(m0 + u, 63));
        len_u[u] = (m0 + u < p.nseg) ? __shfl(cur_len, min(m0 + u, 63)) : 0;
        took[u] = 0;
      }
      for (int base = 0;; base += 64) {
        // Every lane loads, with no branch (past a bucket's end it reloads the
        // bucket's last posting; an empty bucket reads out of the buffer's
        // range, which loads 0), so all kLightBatch loads are out before the
        // first add.
        int32_t j_u[kLightBatch];
#pragma unroll
        for (int u = 0; u < kLightBatch; ++u) {
          const int e = lo_u[u] + min(base + lane, len_u[u] - 1);
          j_u[u] = __builtin_amdgcn_raw_buffer_load_b32(m0 + u < p.a ? prs : trs, e * 4, 0, 0);
        }
        bool more = false;
#pragma unroll
        for (int u = 0; u < kLightBatch; ++u) {
          const int32_t j = m0 + u < p.a ? j_u[u] : j_u[u] + p.tail_key0;
          const bool in_range = base + lane < len_u[u] && j < kend;
          const uint64_t bal = __ballot(in_range);
          took[u] += __popcll(bal);
          more = more || bal == ~0ull;
          if (in_range) add(j);
        }
        if (!more) break;
      }
#pragma unroll
      for (int u = 0; u < kLightBatch; ++u)
        if (lane == m0 + u) {
          cur_lo += took[u];
          cur_len -= took[u];
        }
    }
  };

  // Window of more than kFlatWords words: cwords words (65536 keys, or all
  // keys as one chunk) at a time, each chunk with a summary level (bit x:
  // bitmap word x was touched by this row): the chunk's bitmap and summary are
  // cleared (16-byte stores, no waits) and marked with ors whose return no lane
  // waits for (a wave's LDS operations run in program order), and the chunk's
  // candidates are read back from the touched words only.  `sink(pos, key)`
  // receives them ascending; returns their number.  Chunk 0's first fwn words
  // are kept for the filler.
  const int64_t ckeys = static_cast<int64_t>(cwords) * 32;
  const bool one_chunk = wend <= ckeys;
  int last_cs = 0;  // summary words of the last chunk marked
  auto run_chunks = [&](bool count, auto&& sink) __attribute__((always_inline)) -> int {
    cur_lo = lo;
    cur_len = len;
    int emitted = 0;
    for (int64_t kbeg = 0; kbeg < wend; kbeg += ckeys) {
      const int64_t kend = min(kbeg + ckeys, wend);
      const int cw = static_cast<int>((kend - kbeg + 31) >> 5);
      const int cs = (cw + 31) >> 5;
      last_cs = cs;
      for (int x = lane; x < cs; x += 64) sm[x] = 0u;
      // (bm is 16-byte aligned: the summary takes a multiple of 4 words)
      for (int x = 4 * lane; x + 3 < cw; x += 256) *reinterpret_cast<uint4*>(bm + x) = make_uint4(0u, 0u, 0u, 0u);
      for (int x = (cw & ~3) + lane; x < cw; x += 64) bm[x] = 0u;
      __builtin_amdgcn_wave_barrier();
      mark_range(kbeg, kend, true, count, !one_chunk);
      if (!(count && one_chunk)) {  // one chunk: emitted once C is known
        const int base = emitted;
        emitted += light_emit(sm, bm, cs, lane, [&](int pos, int key) {
          sink(base + pos, static_cast<int32_t>(kbeg + key));
        });
      }
      if (kbeg == 0 && count && !one_chunk)
        for (int x = lane; x < fwn; x += 64) fw[x] = ((sm[x >> 5] >> (x & 31)) & 1u) ? bm[x] : 0u;
    }
    return emitted;
  };

  int filled = 0;
  if (flat) {
    for (int x = lane; x < live; x += 64) bm[x] = 0u;
    __builtin_amdgcn_wave_barrier();
    mark_range(0, wend, false, true, false);
    __builtin_amdgcn_wave_barrier();
    for (int x = lane; x < live; x += 64) fresh += __popc(bm[x]);
  } else {
    // candidates to the output as they come (a row that turns out to have more
    // than k_eff writes at most top_k of them there; its final row is written
    // by the screen and pick passes or the exact pass, which run later)
    filled = run_chunks(true, [&](int pos, int32_t key) {
      if (pos < p.top_k) put(pos, key);
    });
    if (one_chunk) {
      // the new keys: the touched words' bits (emitted once C is known)
      const int cw = static_cast<int>((wend + 31) >> 5);
      for (int x = lane; x < cw; x += 64) fresh += __popc(bm[x]);
    } else {
      fresh = (lane == 0) ? filled : 0;  // every chunk's keys were emitted
    }
  }
  int C = 0, raw = 0;
  wave_excl_scan(fresh, lane, &C);
  if (p.stats) wave_excl_scan(seen, lane, &raw);
  if (p.stats && lane == 0) {
    p.stats[(bh * p.n_q + r) * 2 + 0] = C;
    p.stats[(bh * p.n_q + r) * 2 + 1] = raw;
  }
  if (p.cnt && lane == 0) p.cnt[row] = C;
  __builtin_amdgcn_wave_barrier();

  if (C > p.k_eff) {
    if (p.prefix && lane == 0) p.prefix[row] = 0;
    const int shard = static_cast<int>(blockIdx.x % kShards);
    int32_t* sc = w.ctr + 16 + 4 * shard;
    int64_t off = -1;
    if (w.cap > 0 && C <= 64 * kScrRegs) {
      // whole 128-byte lines per row (32 entries), so no two rows share a line
      const unsigned long long cpad = static_cast<unsigned long long>((C + 31) & ~31);
      unsigned long long o = 0ull;
      if (lane == 0) o = atomicAdd(reinterpret_cast<unsigned long long*>(sc + 2), cpad);
      const uint32_t olo = static_cast<uint32_t>(__shfl(static_cast<int>(o & 0xFFFFFFFFull), 0));
      const uint32_t ohi = static_cast<uint32_t>(__shfl(static_cast<int>(o >> 32), 0));
      o = (static_cast<unsigned long long>(ohi) << 32) | olo;
      if (o + cpad <= static_cast<unsigned long long>(w.cap))
        off = static_cast<int64_t>(shard) * w.cap + static_cast<int64_t>(o);
    }
    if (off < 0) {
      if (lane == 0) push_exact(w, p.rows, row);
      return;
    }
    int32_t* dst = w.cand + off;
    auto to_list = [&](int pos, int32_t v) {
      if (pos < C) dst[pos] = v;
    };
    if (flat) light_emit_flat(bm, live, lane, to_list);
    else if (one_chunk) light_emit(sm, bm, last_cs, lane, to_list);  // the window's bitmap is still there
    else run_chunks(false, to_list);  // the same marks again, now into the list
    if (lane == 0) {
      const int slot = atomicAdd(&sc[0], 1);
      if (slot >= 0 && slot < w.shard_rows) {
        int32_t* ent = w.scr + (static_cast<int64_t>(shard) * w.shard_rows + slot) * 3;
        ent[0] = static_cast<int32_t>(row);
        ent[1] = static_cast<int32_t>(off - static_cast<int64_t>(shard) * w.cap);
        ent[2] = C;
      } else {
        push_exact(w, p.rows, row);  // not reached: shard_rows bounds a shard
      }
    }
    return;
  }

  // Candidates ascending (already written by a window of several chunks), then
  // the lowest non-candidates up to k_eff.
  if (flat) filled = light_emit_flat(bm, live, lane, put);
  else if (one_chunk) filled = light_emit(sm, bm, last_cs, lane, put);
  // Keys of word x the row holds: the flat bitmap, the one chunk's touched
  // words, or chunk 0's copy (the filler lies in the keys below k_eff + C <=
  // 2 k_eff, inside the copy).
  auto held = [&](int x) -> uint32_t {
    if (flat) return x < live ? bm[x] : 0u;
    if (one_chunk) return (x < live && ((sm[x >> 5] >> (x & 31)) & 1u)) ? bm[x] : 0u;
    return x < fwn ? fw[x] : 0u;
  };
  // The filler is the k_eff - C lowest keys the row does not hold, so every key
  // up to the last one is in the row, once: X = last filler key + 1 (0 without
  // filler, and 0 when index-0 padding repeats a key).
  const bool want_x = p.prefix != nullptr && p.k_eff == p.top_k;
  if (p.prefix && lane == 0 && (filled >= p.k_eff || !want_x)) p.prefix[row] = 0;
  // One key per lane: 64 consecutive keys (two bitmap words) per step, lane l
  // taking key w0*32 + l; a key the row does not hold goes to position
  // `filled` + the number of such keys on lower lanes (one mask count).  The
  // filler lies in the keys below k_eff + C <= 2 k_eff, so at most 2 k_eff / 64
  // + 1 steps run, each a few instructions with no per-bit loop, and the
  // stores of a step are contiguous.
  for (int w0 = 0; filled < p.k_eff; w0 += 2) {
    const int x = w0 + (lane >> 5);
    uint32_t nb = 0u;  // keys of word x the row does not hold (and that exist)
    if (x < words) {
      nb = ~held(x);
      if (x == words - 1 && (p.n & 31)) nb &= (1u << (p.n & 31)) - 1u;
    }
    const bool mine = (nb >> (lane & 31)) & 1u;
    const uint64_t bal = __ballot(mine);
    const int pos = filled + static_cast<int>(__builtin_amdgcn_mbcnt_hi(
                                 static_cast<uint32_t>(bal >> 32),
                                 __builtin_amdgcn_mbcnt_lo(static_cast<uint32_t>(bal), 0u)));
    if (mine && pos < p.k_eff) {
      const int key = x * 32 + (lane & 31);
      if (want_x && pos == p.k_eff - 1) p.prefix[row] = key + 1;
      put(pos, key);
    }
    filled += __popcll(bal);
  }
  for (int x = p.k_eff + lane; x < p.top_k; x += 64) put(x, 0);
}

// ---- rows with more than k candidates: matrix-core screen (bf16) -----------
//
// One wave per listed row.  Approximate scores A_j = (k_j . q_s) * r, r the
// fp32 reciprocal of score_div * g, with q_s = sum_g q_g split as q_s = hi + lo in bf16 (|q_s - hi - lo| <=
// 2^-18 |q_s|): K rows are gathered whole into LDS (row_issue) and one 16x16x32
// MFMA per 32 dims scores 16 keys against the columns (hi, lo); a second one
// against |K| and the column up(sum_g |q_g|) (rounded up to bf16) gives P_j >=
// sum_t |k_jt| sum_g |q_gt|.
//
// Bound.  With u = 2^-24, the canonical fp32 score E_j (g fmaf chains of d
// terms, / score_div, summed, / g) is within (d + g + 3) u P/sd/g of the real
// value, and A_j within (4.04 d + 64 + g + 9) u P/sd/g (MFMA sums of exact
// products with per-add error <= 2u, the dropped 2^-18 remainder, the fp32
// head sum of q_s, and 3u for the scaling by r: sd * g, its reciprocal and the
// product each round once; one multiply instead of two correctly rounded
// divisions, which cost about ten instructions each for every lane).  So |A_j - E_j| <= e_j = (6 d + 2 g + 100) u * 1.02 *
// P_j (1 + 4 d u) / sd / g + 1e-30, and e = max_j e_j.
//
// Selection (select_pick_kernel).  T = the k-th largest A lies in a band
// [lo, hi] of A values found by at most two 256-bin histogram passes.  At
// least k keys have A >= lo, so the k-th largest exact score E* >= lo - e;
// fewer than k keys have A > hi, so E* <= hi + e.  Every key with A_j > hi + 2e
// then has E_j > E* and is selected; every key with A_j < lo - 2e has E_j < E*
// and is not.  The keys between (at most kScrBorder, else the row takes the
// exact pass) are rescored in the canonical order, and the best (k - #above)
// of them by (score desc, index asc) complete the set: the selected set's
// members among them are exactly those.  The row is written in index order.
// Non-finite scores or bounds send the row to the exact pass.


__device__ __forceinline__ uint16_t bf16_rne_bits(float f) {
  uint32_t u = __float_as_uint(f);
  u += 0x7FFFu + ((u >> 16) & 1u);
  return static_cast<uint16_t>(u >> 16);
}
// Smallest bf16 >= f for finite f >= 0.
__device__ __forceinline__ uint16_t bf16_up_bits(float f) {
  const uint32_t u = __float_as_uint(f);
  return static_cast<uint16_t>((u >> 16) + ((u & 0xFFFFu) ? 1u : 0u));
}
// lane p of each 16-lane row reads lane p + 1 (lane 15 reads 0)
__device__ __forceinline__ float dpp_from_plus1(float x) {
  return __uint_as_float(__builtin_amdgcn_update_dpp(0u, __float_as_uint(x), 0x101, 0xF, 0xF, false));
}

// Entry e of a shard's list (the waves' assignment is shard_walk's).
struct ScrEntry {
  int64_t row, off;  // off: list position of the row's first candidate
  int C;
  bool ok;
};
__device__ __forceinline__ ScrEntry scr_entry(const SelParams& p, const SelWs& w, int shard, int e) {
  const int32_t* ent = w.scr + (static_cast<int64_t>(shard) * w.shard_rows + e) * 3;
  ScrEntry x;
  x.row = ent[0];
  x.off = static_cast<int64_t>(shard) * w.cap + ent[1];
  x.C = ent[2];
  x.ok = x.row >= 0 && x.row < p.rows && ent[1] >= 0 && x.C > p.k_eff && x.C <= 64 * kScrRegs &&
         static_cast<int64_t>(ent[1]) + x.C <= w.cap;
  return x;
}

template <int D, int GMAX>
// (4 waves per SIMD: at most 128 registers, which the d = 128 build meets
// without spilling)
__global__ __launch_bounds__(64 * kScrWaves) __attribute__((amdgpu_waves_per_eu(4, 8))) void
select_screen_kernel(SelParams p, SelWs w) {
  using S = MfShape<D>;
  __shared__ __align__(16) unsigned char kst[kScrWaves][kMfChunk * S::ROW];
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const int q4 = lane >> 4, c16 = lane & 15;
  unsigned char* kl = kst[wave];
  uint32_t seg16[S::SWZ_PERIOD];
  row_seg16<D>(lane, seg16);
  const int kswz = mf_swz<D>(c16);
  const uint32_t ksn2 = 2u * static_cast<uint32_t>(p.k_sn);
  const int kbytes = static_cast<int>((p.n - 1) * p.k_sn * 2 + 2 * D);
  const ShardWalk sw = shard_walk(w, wave, p.xcd_slices != 0);
  const int shard = sw.shard;
  const float gf = static_cast<float>(p.g);
  const float ce = (6.0f * D + 2.0f * static_cast<float>(p.g) + 100.0f) * 5.9604645e-8f * 1.02f *
                   (1.0f + 4.0f * D * 5.9604645e-8f);
  const float rsg = 1.0f / (p.score_div * gf);
  for (int e = sw.first; e < sw.end; e += sw.step) {
    const ScrEntry x = scr_entry(p, w, shard, e);
    if (!x.ok) continue;  // the pick pass sends the row to the exact pass
    const int C = x.C;
    const int64_t off = x.off;
    const int64_t bh = udiv32(x.row, p.n_q);
    const int64_t r = x.row - bh * p.n_q;
    const int64_t bb = udiv32(bh, p.h_kv);
    const int h = static_cast<int>(bh - bb * p.h_kv);
    const uint16_t* q0 = static_cast<const uint16_t*>(p.q) + bb * p.q_sb + r * p.q_sn +
                         static_cast<int64_t>(h * p.g) * p.q_sh;
    const uint16_t* kbase = static_cast<const uint16_t*>(p.k) + bb * p.k_sb + static_cast<int64_t>(h) * p.k_sh;
    const __amdgpu_buffer_rsrc_t krs =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(kbase), 0, kbytes, kBufferWord3);

    // B operands (lane (q4, c16): column c16, dims 8*q4 .. +8 of each 32-dim
    // block): column 0 = bf16 hi of the head sum q_s, column 1 = its bf16 lo;
    // qa column 0 = sum_g |q_g| rounded up to bf16.  The group's q rows pass
    // through the K buffer (free between rows): one wave-wide load per 64/SEGS
    // heads (lane l: head l / SEGS, segment l % SEGS), then LDS reads.
#pragma unroll
    for (int g0 = 0; g0 < GMAX; g0 += S::KPI) {
      const int gg = g0 + lane / S::SEGS;
      if (g0 < p.g) {
        const uint4 v = (gg < p.g) ? *reinterpret_cast<const uint4*>(q0 + static_cast<int64_t>(gg) * p.q_sh +
                                                                      (lane % S::SEGS) * 8)
                                   : make_uint4(0u, 0u, 0u, 0u);
        *reinterpret_cast<uint4*>(kl + (g0 / S::KPI) * 1024 + lane * 16) = v;
      }
    }
    __builtin_amdgcn_s_waitcnt(kWaitLgkm0);
    __builtin_amdgcn_wave_barrier();
    bf16x8_t qf[S::KB], qa[S::KB];
#pragma unroll
    for (int kb = 0; kb < S::KB; ++kb) {
      float sv[8], sa[8];
#pragma unroll
      for (int xx = 0; xx < 8; ++xx) sv[xx] = sa[xx] = 0.0f;
      for (int gg = 0; gg < p.g; ++gg) {  // head gg, segment kb*4 + q4 at byte gg*ROW + seg*16
        const uint4 u = *reinterpret_cast<const uint4*>(kl + gg * S::ROW + (kb * 4 + q4) * 16);
        const uint32_t wq[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
        for (int xx = 0; xx < 8; ++xx) {
          const float v = __uint_as_float((xx & 1) ? (wq[xx >> 1] & 0xFFFF0000u) : (wq[xx >> 1] << 16));
          sv[xx] += v;
          sa[xx] += fabsf(v);
        }
      }
      uint16_t hv[8], av[8];
#pragma unroll
      for (int xx = 0; xx < 8; ++xx) {
        const uint16_t hi = bf16_rne_bits(sv[xx]);
        const uint16_t lo = bf16_rne_bits(sv[xx] - __uint_as_float(static_cast<uint32_t>(hi) << 16));
        hv[xx] = (c16 == 0) ? hi : (c16 == 1) ? lo : static_cast<uint16_t>(0);
        av[xx] = (c16 == 0) ? bf16_up_bits(sa[xx] * (1.0f + 9.5367432e-7f)) : static_cast<uint16_t>(0);
      }
      qf[kb] = __builtin_bit_cast(bf16x8_t, hv);
      qa[kb] = __builtin_bit_cast(bf16x8_t, av);
    }
    __builtin_amdgcn_s_waitcnt(kWaitLgkm0);  // q reads done before the K rows land in the buffer

    // 32-candidate chunks: the rows of chunk c + 1 are in flight while chunk c
    // is scored (as in the attention kernel).
    float emax = 0.0f;
    bool bad = false;
    const int nch = (C + kMfChunk - 1) / kMfChunk;
    auto idx_at = [&](int ch) -> int {
      const int pos = ch * kMfChunk + lane;
      return (lane < kMfChunk && pos < C) ? w.cand[off + pos] : -1;
    };
    row_issue<D>(krs, kl, idx_at(0), lane, ksn2, seg16);
    int jn = (nch > 1) ? idx_at(1) : -1;
    for (int ch = 0; ch < nch; ++ch) {
      __builtin_amdgcn_s_waitcnt(kWaitVm0);
      bf16x8_t kf[2][S::KB];
#pragma unroll
      for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int kb = 0; kb < S::KB; ++kb)
          kf[t][kb] = *(lds_bf16x8_ptr)(kl + (16 * t + c16) * S::ROW + (((kb * 4 + q4) ^ kswz) << 4));
      __builtin_amdgcn_s_waitcnt(kWaitLgkm0);
      if (ch + 1 < nch) {
        row_issue<D>(krs, kl, jn, lane, ksn2, seg16);
        jn = (ch + 2 < nch) ? idx_at(ch + 2) : -1;
      }
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        floatx4_t sv = {0.f, 0.f, 0.f, 0.f}, pv = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int kb = 0; kb < S::KB; ++kb) {
          sv = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kf[t][kb], qf[kb], sv, 0, 0, 0);
          uint4 ak = __builtin_bit_cast(uint4, kf[t][kb]);
          ak.x &= 0x7FFF7FFFu; ak.y &= 0x7FFF7FFFu; ak.z &= 0x7FFF7FFFu; ak.w &= 0x7FFF7FFFu;
          pv = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, ak), qa[kb], pv, 0, 0, 0);
        }
#pragma unroll
        for (int e4 = 0; e4 < 4; ++e4) {
          const float slo = dpp_from_plus1(sv[e4]);  // column 1 (lo) of the same keys
          const int pos = ch * kMfChunk + 16 * t + 4 * q4 + e4;
          if (c16 == 0 && pos < C) {
            const float a = (sv[e4] + slo) * rsg;
            const float ej = ce * pv[e4] * rsg + 1e-30f;
            w.approx[off + pos] = a;
            emax = fmaxf(emax, ej);
            bad = bad || !(fabsf(a) <= 3.0e38f) || !(ej <= 3.0e38f);
          }
        }
      }
    }
    emax = wave_allreduce(emax, [](float a, float b) { return fmaxf(a, b); });
    bad = __ballot(bad) != 0ull;
    if (lane == 0) w.emax[static_cast<int64_t>(shard) * w.shard_rows + e] = bad ? INFINITY : emax;
  }
}

// Per listed row, from the screen's scores (a separate kernel, so they are
// visible): the band holding the k_eff-th largest score, the keys above and
// below it by more than 2 e, the exact rescoring of the keys between, and the
// row in index order.
// Bin of a score in [lo, hi] (scale = 256 / (hi - lo)): monotone in a, in
// [0, 255] also when scale overflows to infinity.
__device__ __forceinline__ int band_bin(float a, float lo, float scale) {
  const float t = (a - lo) * scale;
  return (t >= 255.0f) ? 255 : (t >= 0.0f) ? static_cast<int>(t) : 0;
}

template <int D, int GMAX>
__global__ __launch_bounds__(64 * kScrWaves) void select_pick_kernel(SelParams p, SelWs w) {
  __shared__ __align__(16) float avs[kScrWaves][64 * kPickRegs];  // position pos at [pos]
  __shared__ int32_t hst[kScrWaves][256];
  __shared__ int32_t bps[kScrWaves][kScrBorder];
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const uint64_t below = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
  float* av = avs[wave];
  int32_t* hs = hst[wave];
  int32_t* bp = bps[wave];
  const ShardWalk sw = shard_walk(w, wave, p.xcd_slices != 0);
  const int shard = sw.shard;
  const float gf = static_cast<float>(p.g);
  for (int e = sw.first; e < sw.end; e += sw.step) {
    const ScrEntry x = scr_entry(p, w, shard, e);
    if (x.row < 0 || x.row >= p.rows) continue;  // cannot happen: the light pass wrote every entry
    const float emax = w.emax[static_cast<int64_t>(shard) * w.shard_rows + e];
    if (!x.ok || !(emax <= 3.0e38f)) {
      if (lane == 0) push_exact(w, p.rows, x.row);
      continue;
    }
    const int C = x.C;
    const int64_t off = x.off;
    const int64_t row = x.row;
    const int64_t bh = udiv32(row, p.n_q);
    const int64_t r = row - bh * p.n_q;
    const int64_t bb = udiv32(bh, p.h_kv);
    const int h = static_cast<int>(bh - bb * p.h_kv);
    const int R = (C + 63) / 64;  // positions lane + 64 r, r < R

    // The row's scores into LDS (coalesced), with their range: eight loads at
    // a time, all out before the first is used (positions past C reload score
    // C - 1, C >= 1 for a listed row).  A row longer than 64 * kPickRegs keeps
    // them in the workspace and the passes below read them there: the smaller
    // LDS buffer lets 4 blocks share a CU instead of 3.
    const bool in_lds = C <= 64 * kPickRegs;
    const float* ag = w.approx + off;
    float amin = INFINITY, amax = -INFINITY;
    for (int r0 = 0; r0 < R; r0 += 8) {
      float a8[8];
#pragma unroll
      for (int t = 0; t < 8; ++t) a8[t] = ag[min(lane + 64 * (r0 + t), C - 1)];
#pragma unroll
      for (int t = 0; t < 8; ++t) {
        const int pos = lane + 64 * (r0 + t);
        if (r0 + t < R) {
          const float a = (pos < C) ? a8[t] : -INFINITY;
          if (in_lds) av[pos] = a;
          if (pos < C) {
            amin = fminf(amin, a);
            amax = fmaxf(amax, a);
          }
        }
      }
    }
    amin = wave_allreduce(amin, [](float a, float b) { return fminf(a, b); });
    amax = wave_allreduce(amax, [](float a, float b) { return fmaxf(a, b); });

    float lo, hi;
    int m_in, nb;
    uint32_t* sm = reinterpret_cast<uint32_t*>(hs);
    auto band_and_classify = [&](auto score_at) {
      // Band [lo, hi] holding the k_eff-th largest score: 256 bins over the band
      // (bin = floor((a - lo) * 256 / (hi - lo)), monotone in a), keep the bin
      // where the count from the top reaches the rank, shrink the band to the
      // smallest and largest score in that bin; at most two passes.
      lo = amin;
      hi = amax;
      int kk = p.k_eff;
      for (int pass = 0; pass < 2 && hi > lo; ++pass) {
        const float scale = 256.0f / (hi - lo);
        for (int xx = lane; xx < 256; xx += 64) hs[xx] = 0;
        __builtin_amdgcn_wave_barrier();
#pragma unroll 4
        for (int r = 0; r < R; ++r) {
          const float a = score_at(lane + 64 * r);
          if (a >= lo && a <= hi) atomicAdd(&hs[band_bin(a, lo, scale)], 1);
        }
        __builtin_amdgcn_wave_barrier();
        int c4[4], tot = 0;
#pragma unroll
        for (int xx = 0; xx < 4; ++xx) {
          c4[xx] = hs[255 - 4 * lane - xx];  // lanes walk the bins from the top
          tot += c4[xx];
        }
        int all = 0;
        const int before = wave_excl_scan(tot, lane, &all);
        int bin = -1, nk = 0, inbin = 0;
        if (before < kk && kk <= before + tot) {
          int acc = before;
#pragma unroll
          for (int xx = 0; xx < 4; ++xx) {
            if (bin < 0 && kk <= acc + c4[xx]) {
              bin = 255 - 4 * lane - xx;
              nk = kk - acc;
              inbin = c4[xx];
            }
            acc += c4[xx];
          }
        }
        const int src = __ffsll(static_cast<unsigned long long>(__ballot(bin >= 0))) - 1;
        if (src < 0) break;  // cannot happen: kk <= keys in the band
        bin = lane_value(bin, src);
        nk = lane_value(nk, src);
        inbin = lane_value(inbin, src);
        float blo = INFINITY, bhi = -INFINITY;
#pragma unroll 4
        for (int r = 0; r < R; ++r) {
          const float a = score_at(lane + 64 * r);
          if (a >= lo && a <= hi && band_bin(a, lo, scale) == bin) {
            blo = fminf(blo, a);
            bhi = fmaxf(bhi, a);
          }
        }
        blo = wave_allreduce(blo, [](float a, float b) { return fminf(a, b); });
        bhi = wave_allreduce(bhi, [](float a, float b) { return fmaxf(a, b); });
        lo = blo;
        hi = bhi;
        kk = nk;
        __builtin_amdgcn_wave_barrier();
        if (inbin <= 32) break;
      }
      const float e2 = 2.0f * 1.02f * emax + 2e-30f;
      const float thr_in = hi + e2, thr_out = lo - e2;

      // Classify: keys surely in the top k_eff go to the selection mask (bit pos
      // of word pos / 32, in hs), keys within 2 e of the band to bp (ascending).
      m_in = 0;
      nb = 0;
      for (int r = 0; r < R; ++r) {
        const int pos = lane + 64 * r;
        const float a = score_at(pos);
        const bool in = a > thr_in;
        const bool border = pos < C && !in && a >= thr_out;
        m_in += in ? 1 : 0;
        const uint64_t imask = __ballot(in);
        const uint64_t bmask = __ballot(border);
        if (lane < 2) sm[2 * r + lane] = static_cast<uint32_t>(imask >> (32 * lane));
        if (border) {
          const int sl = nb + __popcll(bmask & below);
          if (sl < kScrBorder) bp[sl] = pos;
        }
        nb += __popcll(bmask);
      }
    };
    if (in_lds) band_and_classify([&](int pos) { return av[pos]; });
    else band_and_classify([&](int pos) { return pos < C ? ag[pos] : -INFINITY; });
    int n_in = 0;
    wave_excl_scan(m_in, lane, &n_in);
    const int need = p.k_eff - n_in;
    if (nb > kScrBorder || need < 0 || need > nb) {
      if (lane == 0) push_exact(w, p.rows, row);
      __builtin_amdgcn_wave_barrier();
      continue;
    }

    // The group's q rows into the score area (free now): head gg at gg * D.
    const uint16_t* q0 = static_cast<const uint16_t*>(p.q) + bb * p.q_sb + r * p.q_sn +
                         static_cast<int64_t>(h * p.g) * p.q_sh;
    uint16_t* ql = reinterpret_cast<uint16_t*>(av);
    for (int t = lane; t < p.g * (D / 8); t += 64) {
      const int gg = t / (D / 8), sg = t % (D / 8);
      *reinterpret_cast<uint4*>(ql + gg * D + sg * 8) =
          *reinterpret_cast<const uint4*>(q0 + static_cast<int64_t>(gg) * p.q_sh + sg * 8);
    }
    __builtin_amdgcn_s_waitcnt(kWaitLgkm0);
    __builtin_amdgcn_wave_barrier();

    // Exact scores of the borderline keys (one per lane, the canonical order:
    // per head an fmaf chain over ascending dims from +0) and their ranks.
    uint64_t key = 0ull;
    if (lane < nb) {
      const int32_t j = w.cand[off + bp[lane]];
      const uint16_t* kr = static_cast<const uint16_t*>(p.k) + bb * p.k_sb + static_cast<int64_t>(h) * p.k_sh +
                           static_cast<int64_t>(j) * p.k_sn;
      float acc[GMAX];
#pragma unroll
      for (int gg = 0; gg < GMAX; ++gg) acc[gg] = 0.0f;
      constexpr int KL = 8;  // 16-byte loads in flight per lane: half a D = 128 row
#pragma unroll 1
      for (int t0 = 0; t0 < D; t0 += 8 * KL) {
        float kv[KL][8];
#pragma unroll
        for (int u = 0; u < KL; ++u) load8(kr + t0 + 8 * u, kv[u]);
#pragma unroll
        for (int gg = 0; gg < GMAX; ++gg) {
          if (gg >= p.g) continue;
#pragma unroll
          for (int u = 0; u < KL; ++u) {
            float qv[8];
            load8(ql + gg * D + t0 + 8 * u, qv);  // same address in every lane: a broadcast
#pragma unroll
            for (int e = 0; e < 8; ++e) acc[gg] = fma_rn(qv[e], kv[u][e], acc[gg]);
          }
        }
      }
      float sc = acc[0] / p.score_div;
#pragma unroll
      for (int gg = 1; gg < GMAX; ++gg)
        if (gg < p.g) sc = sc + acc[gg] / p.score_div;
      sc = sc / gf;
      key = composite_key(sc, static_cast<uint32_t>(j));
    }
    int rank = 0;
    for (int b = 0; b < nb; ++b) {
      const uint64_t kb = (static_cast<uint64_t>(static_cast<uint32_t>(lane_value(static_cast<int>(key >> 32), b))) << 32) |
                          static_cast<uint32_t>(lane_value(static_cast<int>(key & 0xFFFFFFFFull), b));
      rank += (kb > key) ? 1 : 0;
    }
    if (lane < nb && rank < need) atomicOr(&sm[bp[lane] >> 5], 1u << (bp[lane] & 31));
    __builtin_amdgcn_wave_barrier();

    // The selected keys in index order.
    const int64_t obase = ((bb * p.n_q + r) * p.h_kv + h) * p.top_k;
    int32_t* o32 = static_cast<int32_t*>(p.out) + obase;
    int64_t* o64 = static_cast<int64_t*>(p.out) + obase;
    int filled = 0;
    for (int r0 = 0; r0 < R; r0 += 8) {
      int32_t jv[8];  // eight list words in flight at once
#pragma unroll
      for (int u = 0; u < 8; ++u) jv[u] = w.cand[off + min(lane + 64 * (r0 + u), C - 1)];
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        const int r = r0 + u;
        if (r >= R) break;
        const uint64_t smask = static_cast<uint64_t>(sm[2 * r]) | (static_cast<uint64_t>(sm[2 * r + 1]) << 32);
        const bool sel = (smask >> lane) & 1ull;
        const int o = filled + __popcll(smask & below);
        if (sel && o < p.k_eff) {
          if (p.out_i64) o64[o] = jv[u];
          else o32[o] = jv[u];
        }
        filled += __popcll(smask);
      }
    }
    __builtin_amdgcn_wave_barrier();  // av, hs and bp are rewritten by the next row
  }
}

__global__ void zero_ctr_kernel(int32_t* __restrict__ ctr) {
  for (int x = threadIdx.x; x < static_cast<int>(kSelCtrBytes / 4); x += blockDim.x) ctr[x] = 0;
}

size_t light_smem(const SelParams& p) {
  return sizeof(uint32_t) * static_cast<size_t>(light_words(p.n, light_chunk_words(p)));
}

// Rows of the light-pass blocks of one shard (block b -> shard b % kShards).
int64_t shard_rows_for(int64_t rows) { return ceil_div(rows, kShards); }

size_t sel_ws_fixed(int64_t rows) {
  return kSelCtrBytes + 2 * align_up(sizeof(int32_t) * static_cast<size_t>(rows), 256) +
         align_up(3 * sizeof(int32_t) * static_cast<size_t>(kShards * shard_rows_for(rows)), 256) +
         align_up(sizeof(float) * static_cast<size_t>(kShards * shard_rows_for(rows)), 256);
}

SelWs carve_sel_ws(void* ws, size_t bytes, int64_t rows, bool screen) {
  char* c = static_cast<char*>(ws);
  SelWs w{};
  w.ctr = reinterpret_cast<int32_t*>(c);
  c += kSelCtrBytes;
  w.exact = reinterpret_cast<int32_t*>(c);
  c += align_up(sizeof(int32_t) * static_cast<size_t>(rows), 256);
  w.shard_rows = shard_rows_for(rows);
  w.scr = reinterpret_cast<int32_t*>(c);
  c += align_up(3 * sizeof(int32_t) * static_cast<size_t>(kShards * w.shard_rows), 256);
  w.emax = reinterpret_cast<float*>(c);
  c += align_up(sizeof(float) * static_cast<size_t>(kShards * w.shard_rows), 256);
  w.cnt = reinterpret_cast<int32_t*>(c);
  c += align_up(sizeof(int32_t) * static_cast<size_t>(rows), 256);
  const size_t fixed = sel_ws_fixed(rows);
  // per shard: cap candidates and cap scores
  int64_t cap = (screen && bytes > fixed + 256) ? static_cast<int64_t>((bytes - fixed - 256) / (8 * kShards)) : 0;
  if (cap > (int64_t(1) << 31) / kShards - 1) cap = (int64_t(1) << 31) / kShards - 1;
  cap &= ~int64_t(31);  // shard slices start on 128-byte lines
  if (cap < 0) cap = 0;
  w.cand = reinterpret_cast<int32_t*>(c);
  w.approx = reinterpret_cast<float*>(c + align_up(sizeof(int32_t) * static_cast<size_t>(cap * kShards), 256));
  w.cap = cap;
  return w;
}

int persistent_grid(int64_t work, int per_cu) {
  static int cus[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) dev = 0;
  if (cus[dev] == 0) {
    int c = 0;
    if (hipDeviceGetAttribute(&c, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || c <= 0) c = 256;
    cus[dev] = c;
  }
  const int64_t g = static_cast<int64_t>(cus[dev]) * per_cu;
  return static_cast<int>(work < g ? (work > 0 ? work : 1) : g);
}

// Grid of the screen (WHICH = 0) or pick (1) kernel: as many blocks as fit on
// the device at once, rounded up so that each XCD's share of the waves is a
// multiple of kShards (shard_walk).
template <int D, int GMAX, int WHICH>
int shard_grid() {
  static int cached[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) dev = 0;
  if (cached[dev] == 0) {
    int per_cu = 0;
    const void* f = (WHICH == 0) ? reinterpret_cast<const void*>(select_screen_kernel<D, GMAX>)
                                 : reinterpret_cast<const void*>(select_pick_kernel<D, GMAX>);
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, f, 64 * kScrWaves, 0) != hipSuccess || per_cu <= 0)
      per_cu = 2;
    constexpr int kBlocksPerShardSet = kXcds * kShards / kScrWaves;
    cached[dev] = static_cast<int>(ceil_div(persistent_grid(int64_t(1) << 40, per_cu), kBlocksPerShardSet) *
                                   kBlocksPerShardSet);
  }
  return cached[dev];
}

// ws (nullable): index order through the light pass, the screen (bf16, d = 64 or
// 128) and the exact pass for the rest; otherwise one block per row.
template <typename T, int GMAX, int D>
int launch_select(const SelParams& p, int64_t rows, size_t smem, void* ws, size_t ws_bytes, hipStream_t st) {
  auto kern = select_kernel<T, GMAX, D>;
  if (int s = reserve_lds(reinterpret_cast<const void*>(kern), smem, "select")) return s;
  const T* qg = static_cast<const T*>(p.q);
  constexpr bool kScreenable = sizeof(T) == 2 && (D == 64 || D == 128);
  // 32-bit buffer offsets of the screen's K gathers
  const bool screen = kScreenable && p.n < (int64_t(1) << 24) && 2 * p.k_sn < (int64_t(1) << 24) &&
                      (p.n - 1) * p.k_sn * 2 + 2 * p.d < (int64_t(1) << 31);
  if (ws == nullptr || (p.sorted && p.k_eff > kSortMax) || light_smem(p) > 64 * 1024) {
    kern<<<dim3(static_cast<unsigned>(rows)), kSelThreads, smem, st>>>(p, qg);
    return check_launch("select_kernel");
  }
  const SelWs w = carve_sel_ws(ws, ws_bytes, rows, screen);
  // score order: the index-order passes, then the sort pass over their rows
  const bool sort_after = p.sorted != 0;
  SelParams pi = p;
  pi.sorted = 0;
  pi.cnt = sort_after ? w.cnt : nullptr;
  zero_ctr_kernel<<<1, 256, 0, st>>>(w.ctr);
  if (int s = check_launch("zero_ctr_kernel")) return s;
  pi.light_chunk_words = light_chunk_words(p);
  // With fewer (batch, kv head) pairs than XCDs the XCDs would share heads:
  // there the slices measured slower (c5: 2 kv heads), so they are kept for
  // the case of at least one pair per XCD.
  pi.xcd_slices = (p.n_q > 0 && rows / p.n_q >= kXcds) ? 1 : 0;
  pi.light_pos_lo = 0;
  pi.light_pos_hi = INT64_MAX;
  // A causal window marked as one chunk over all keys (many postings per row)
  // sizes every wave's bitmap for the whole key range.  The rows whose window
  // ends in the first half of the keys run first, in a launch of their own
  // with a half-size bitmap (about twice the waves per CU); the rest follow.
  const int64_t lwords = (p.n + 31) / 32;
  if (p.mask_mode == SSA_MASK_CAUSAL && pi.light_chunk_words == lwords && lwords > 2 * kFlatWords) {
    SelParams pa = pi;
    pa.light_chunk_words = static_cast<int>(lwords / 2);
    pa.light_pos_hi = (lwords / 2) * 32;  // window of at most lwords / 2 words: one chunk
    const size_t smem_a = sizeof(uint32_t) * static_cast<size_t>(light_words(p.n, pa.light_chunk_words));
    select_light_kernel<1><<<dim3(static_cast<unsigned>(rows)), 64, smem_a, st>>>(pa, rows, w);
    if (int s = check_launch("select_light_kernel")) return s;
    pi.light_pos_lo = pa.light_pos_hi;
  }
  if (light_smem(p) * 32 <= kLdsBytesPerCu)
    select_light_kernel<8><<<dim3(static_cast<unsigned>(rows)), 64, light_smem(p), st>>>(pi, rows, w);
  else
    select_light_kernel<1><<<dim3(static_cast<unsigned>(rows)), 64, light_smem(p), st>>>(pi, rows, w);
  if (int s = check_launch("select_light_kernel")) return s;
  if constexpr (kScreenable) {
    if (w.cap > 0) {
      constexpr int DS = (D == 64) ? 64 : 128;
      select_screen_kernel<DS, GMAX><<<dim3(static_cast<unsigned>(shard_grid<DS, GMAX, 0>())), 64 * kScrWaves, 0,
                                      st>>>(pi, w);
      if (int s = check_launch("select_screen_kernel")) return s;
      select_pick_kernel<DS, GMAX><<<dim3(static_cast<unsigned>(shard_grid<DS, GMAX, 1>())), 64 * kScrWaves, 0,
                                    st>>>(pi, w);
      if (int s = check_launch("select_pick_kernel")) return s;
    }
  }
  auto hk = select_heavy_kernel<T, GMAX, D>;
  if (int s = reserve_lds(reinterpret_cast<const void*>(hk), smem, "select")) return s;
  hk<<<dim3(static_cast<unsigned>(persistent_grid(rows, 8))), kSelThreads, smem, st>>>(pi, qg, w);
  if (int s = check_launch("select_heavy_kernel")) return s;
  if (!sort_after) return SSA_OK;
  select_sort_kernel<T, GMAX, D><<<dim3(static_cast<unsigned>(rows)), 64, 0, st>>>(pi, qg);
  return check_launch("select_sort_kernel");
}

template <typename T, int GMAX>
int dispatch_select_d(const SelParams& p, int64_t rows, size_t smem, void* ws, size_t wb, hipStream_t st) {
  switch (p.d) {
    case 64: return launch_select<T, GMAX, 64>(p, rows, smem, ws, wb, st);
    case 128: return launch_select<T, GMAX, 128>(p, rows, smem, ws, wb, st);
    case 256: return launch_select<T, GMAX, 256>(p, rows, smem, ws, wb, st);
    default: return launch_select<T, GMAX, 0>(p, rows, smem, ws, wb, st);
  }
}

template <typename T>
int dispatch_select(const SelParams& p, int64_t rows, size_t smem, void* ws, size_t wb, hipStream_t st) {
  if (p.g <= 4) return dispatch_select_d<T, 4>(p, rows, smem, ws, wb, st);
  if (p.g <= 8) return dispatch_select_d<T, 8>(p, rows, smem, ws, wb, st);
  return dispatch_select_d<T, 16>(p, rows, smem, ws, wb, st);
}

}  // namespace
}  // namespace ssa

using namespace ssa;

extern "C" int ssa_select_workspace_layout(int64_t batch, int64_t n, int h_kv, size_t workspace_bytes,
                                           int screen, int64_t* layout) {
  if (batch < 0 || n < 0 || h_kv <= 0 || !layout)
    return fail(SSA_ERR_INVALID_ARGUMENT, "select layout: bad arguments");
  const int64_t rows = batch * h_kv * n;
  const size_t min_bytes = sel_ws_fixed(rows) + 256;  // ssa_select_workspace_bytes(.., 0)
  if (workspace_bytes < min_bytes)
    return fail(SSA_ERR_WORKSPACE, "select layout: workspace %zu < %zu bytes", workspace_bytes,
                min_bytes);
  char* base = reinterpret_cast<char*>(uintptr_t(1) << 20);  // never dereferenced
  const SelWs w = carve_sel_ws(base, workspace_bytes, rows, screen != 0);
  auto off = [&](const void* ptr) { return static_cast<int64_t>(static_cast<const char*>(ptr) - base); };
  layout[0] = off(w.ctr);
  layout[1] = off(w.exact);
  layout[2] = off(w.scr);
  layout[3] = off(w.emax);
  layout[4] = off(w.cand);
  layout[5] = off(w.approx);
  layout[6] = w.shard_rows;
  layout[7] = w.cap;
  layout[8] = kShards;
  layout[9] = static_cast<int64_t>(kSelCtrBytes);
  layout[10] = off(w.cnt);
  return SSA_OK;
}

extern "C" size_t ssa_select_workspace_bytes(int64_t batch, int64_t n, int h_kv, int top_k) {
  if (batch < 0 || n < 0 || h_kv <= 0 || top_k < 0) return 0;
  const int64_t rows = batch * h_kv * n;
  const int64_t k_eff = top_k < n ? top_k : n;
  // fixed part, then room for candidate lists and their scores: one entry
  // (8 bytes) per output slot
  return sel_ws_fixed(rows) + 256 + align_up(static_cast<size_t>(rows) * static_cast<size_t>(k_eff), 256) * 8;
}

namespace ssa {
// ssa_select_block, optionally with a tail index (tail_offsets non-null): the
// main index covers post_bh / b keys per (batch, kv head) and the tail index
// the keys from tail_key0 on (see SelParams).
int select_entry(const void* q, const void* k, int dtype, int64_t batch, int64_t n, int64_t n_q,
                 int64_t q_pos0, int h_q, int h_kv, int d, int64_t q_sb, int64_t q_sn, int64_t q_sh,
                 int64_t k_sb, int64_t k_sn, int64_t k_sh, const int32_t* q_codes, int a,
                 const int32_t* offsets, const int32_t* postings, int n_c, int b, int top_k,
                 int mask_mode, const uint8_t* mask, int64_t mask_sb, int64_t mask_si,
                 float score_div, int sorted, const int32_t* row_order, void* out,
                 int out_index_dtype, int32_t* stats, void* workspace, size_t workspace_bytes,
                 void* stream, int64_t post_bh, const int32_t* tail_offsets,
                 const int32_t* tail_postings, int64_t tail_bh, int64_t tail_key0,
                 int32_t* row_prefix) {
  if (n_q < 0 || q_pos0 < 0 || q_pos0 + n_q > n)
    return fail(SSA_ERR_INVALID_ARGUMENT, "select: query rows [%lld, %lld) outside the %lld keys",
                static_cast<long long>(q_pos0), static_cast<long long>(q_pos0 + n_q),
                static_cast<long long>(n));
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
  if (workspace && workspace_bytes < ssa_select_workspace_bytes(batch, n_q, h_kv, 0))
    return fail(SSA_ERR_WORKSPACE, "select: workspace %zu < %zu bytes", workspace_bytes,
                ssa_select_workspace_bytes(batch, n_q, h_kv, 0));
  if (batch == 0 || n == 0 || n_q == 0) return SSA_OK;
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
  p.prefix = row_prefix;
  p.n_q = n_q;
  p.q_pos0 = q_pos0;
  p.rows = batch * h_kv * n_q;
  p.order = row_order;
  p.post_bh = post_bh;
  p.nseg = a;
  if (tail_offsets) {
    if (2 * a > kMaxA)
      return fail(SSA_ERR_UNSUPPORTED, "select: a tail index needs codes_per_query <= %d", kMaxA / 2);
    if (!tail_postings || tail_bh < 0 || tail_key0 < 0 || tail_key0 > n || post_bh < 0 ||
        tail_bh >= (int64_t(1) << 31) || post_bh >= (int64_t(1) << 31))
      return fail(SSA_ERR_INVALID_ARGUMENT, "select: bad tail index");
    p.tail_offsets = tail_offsets;
    p.tail_postings = tail_postings;
    p.tail_bh = tail_bh;
    p.tail_key0 = static_cast<int32_t>(tail_key0);
    p.nseg = 2 * a;
  }
  const size_t smem = select_smem(n, p.sortn, p.k_eff);
  if (smem > 160 * 1024)
    return fail(SSA_ERR_UNSUPPORTED, "select: needs %zu bytes of LDS (n=%lld, top_k=%d)", smem,
                static_cast<long long>(n), top_k);
  const int64_t rows = batch * h_kv * n_q;
  if (rows >= (int64_t(1) << 31)) return fail(SSA_ERR_UNSUPPORTED, "select: too many rows");
  hipStream_t st = as_stream(stream);
  if (dtype == SSA_DTYPE_BF16) return dispatch_select<uint16_t>(p, rows, smem, workspace, workspace_bytes, st);
  return dispatch_select<float>(p, rows, smem, workspace, workspace_bytes, st);
}
}  // namespace ssa

// ---------------------------------------------------------------- no-alloc variant
//
// ssa_select_block_noalloc runs ssa_select_block with its workspace in the
// file-scope array below instead of caller memory, for callers that cannot
// allocate (code under HIP graph capture, serving loops).  The array is a
// host-side symbol: kernels get its device address, looked up once per device
// with hipGetSymbolAddress and cached; every call on one device shares it, so
// calls that overlap on one device race.  Only the counter block must start at
// zero, and the select path clears it with a kernel on every call.

constexpr size_t kSelScratchBytes = size_t(64) << 20;
static __device__ __align__(256) unsigned char scratch[kSelScratchBytes];

namespace ssa {
namespace {

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

// Device address of `scratch` on the current device (nullptr on failure, with
// the status in *st).
void* scratch_address(int* st) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) {
    *st = fail(SSA_ERR_HIP, "select (no alloc): cannot query the current device");
    return nullptr;
  }
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* ptr = nullptr;
    const hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !ptr) {
      *st = fail(SSA_ERR_HIP, "select (no alloc): hipGetSymbolAddress: %s", hipGetErrorString(e));
      return nullptr;
    }
    g_scratch_ptr[dev] = ptr;
  }
  *st = SSA_OK;
  return g_scratch_ptr[dev];
}

}  // namespace
}  // namespace ssa

extern "C" size_t ssa_select_noalloc_scratch_bytes(void) { return kSelScratchBytes; }

extern "C" int ssa_select_block_noalloc(const void* q, const void* k, int dtype, int64_t batch,
                                        int64_t n, int64_t n_q, int64_t q_pos0, int h_q, int h_kv,
                                        int d, int64_t q_sb, int64_t q_sn, int64_t q_sh,
                                        int64_t k_sb, int64_t k_sn, int64_t k_sh,
                                        const int32_t* q_codes, int a, const int32_t* offsets,
                                        const int32_t* postings, int n_c, int b, int top_k,
                                        int mask_mode, const uint8_t* mask, int64_t mask_sb,
                                        int64_t mask_si, float score_div, int sorted,
                                        const int32_t* row_order, void* out, int out_index_dtype,
                                        int32_t* stats, int32_t* row_prefix, void* stream) {
  if (batch < 0 || n_q < 0 || h_kv <= 0 || top_k < 0)
    return fail(SSA_ERR_INVALID_ARGUMENT, "select (no alloc): bad shape");
  const size_t need = ssa_select_workspace_bytes(batch, n_q, h_kv, 0);
  if (need > kSelScratchBytes)
    return fail(SSA_ERR_WORKSPACE,
                "select (no alloc): %lld query rows x %d kv heads need %zu bytes of scratch, more "
                "than its %zu bytes; use ssa_select_block with a workspace",
                static_cast<long long>(batch * n_q), h_kv, need, kSelScratchBytes);
  size_t bytes = ssa_select_workspace_bytes(batch, n_q, h_kv, top_k);
  if (bytes > kSelScratchBytes) bytes = kSelScratchBytes;
  if (batch == 0 || n == 0 || n_q == 0)  // nothing to launch: the scratch is not needed
    return ssa_select_block(q, k, dtype, batch, n, n_q, q_pos0, h_q, h_kv, d, q_sb, q_sn, q_sh,
                            k_sb, k_sn, k_sh, q_codes, a, offsets, postings, n_c, b, top_k,
                            mask_mode, mask, mask_sb, mask_si, score_div, sorted, row_order, out,
                            out_index_dtype, stats, row_prefix, nullptr, 0, stream);
  int st = SSA_OK;
  void* ws = ssa::scratch_address(&st);
  if (!ws) return st;
  return ssa_select_block(q, k, dtype, batch, n, n_q, q_pos0, h_q, h_kv, d, q_sb, q_sn, q_sh, k_sb,
                          k_sn, k_sh, q_codes, a, offsets, postings, n_c, b, top_k, mask_mode, mask,
                          mask_sb, mask_si, score_div, sorted, row_order, out, out_index_dtype,
                          stats, row_prefix, ws, bytes, stream);
}

extern "C" int ssa_select_block(const void* q, const void* k, int dtype, int64_t batch, int64_t n,
                                int64_t n_q, int64_t q_pos0, int h_q, int h_kv, int d, int64_t q_sb,
                                int64_t q_sn, int64_t q_sh, int64_t k_sb, int64_t k_sn, int64_t k_sh,
                                const int32_t* q_codes, int a, const int32_t* offsets,
                                const int32_t* postings, int n_c, int b, int top_k, int mask_mode,
                                const uint8_t* mask, int64_t mask_sb, int64_t mask_si,
                                float score_div, int sorted, const int32_t* row_order, void* out,
                                int out_index_dtype, int32_t* stats, int32_t* row_prefix,
                                void* workspace, size_t workspace_bytes, void* stream) {
  return ssa::select_entry(q, k, dtype, batch, n, n_q, q_pos0, h_q, h_kv, d, q_sb, q_sn, q_sh, k_sb,
                           k_sn, k_sh, q_codes, a, offsets, postings, n_c, b, top_k, mask_mode, mask,
                           mask_sb, mask_si, score_div, sorted, row_order, out, out_index_dtype,
                           stats, workspace, workspace_bytes, stream, n * b, nullptr, nullptr, 0, 0,
                           row_prefix);
}

extern "C" int ssa_select(const void* q, const void* k, int dtype, int64_t batch, int64_t n,
                          int h_q, int h_kv, int d, int64_t q_sb, int64_t q_sn, int64_t q_sh,
                          int64_t k_sb, int64_t k_sn, int64_t k_sh, const int32_t* q_codes, int a,
                          const int32_t* offsets, const int32_t* postings, int n_c, int b,
                          int top_k, int mask_mode, const uint8_t* mask, int64_t mask_sb,
                          int64_t mask_si, float score_div, int sorted, const int32_t* row_order,
                          void* out, int out_index_dtype, int32_t* stats, int32_t* row_prefix,
                          void* workspace, size_t workspace_bytes, void* stream) {
  return ssa_select_block(q, k, dtype, batch, n, n, 0, h_q, h_kv, d, q_sb, q_sn, q_sh, k_sb, k_sn,
                          k_sh, q_codes, a, offsets, postings, n_c, b, top_k, mask_mode, mask,
                          mask_sb, mask_si, score_div, sorted, row_order, out, out_index_dtype,
                          stats, row_prefix, workspace, workspace_bytes, stream);
}
