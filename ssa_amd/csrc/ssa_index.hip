// Stage (b): inverted index code -> keys, deterministic and stable.
//
// No reference counterpart: the reference materialises the [n, h, n] mask by
// broadcast compare (ssa/router.py:241-257).  The index reproduces the same
// key sets per code, and its postings ascend inside each bucket, so offsets and
// postings are bit-identical with the CPU oracle.
//
// Three kernels per (batch, kv-head) pair "bh", keys cut into tiles of
// `tile_keys` keys (tile_keys*b entries):
//   1. index_hist    : per-tile LDS histogram of codes -> hist[bh][tile][c]
//   2. index_scan    : exclusive scan of hist in (code, tile) order -> base
//                      positions; offsets[bh][c] = base of (c, tile 0)
//   3. index_scatter : one wave per tile walks its entries in order; lanes that
//                      share a code rank themselves by ballot (lowest lane =
//                      lowest key first) and advance an LDS cursor per code.
#include "ssa_common.h"
#include "ssa_internal.h"

namespace ssa {
namespace {

constexpr int kHistThreads = 256;
constexpr int kScanThreads = 1024;
constexpr int kScatterBatch = 16;  // rounds of 64 entries whose codes are loaded together

int64_t tile_keys_for(int64_t n) {
  int64_t tk = ceil_div(n, 64);
  tk = ceil_div(tk, 64) * 64;
  return tk < 1024 ? 1024 : tk;
}

// Entry e = j*b + r of a head is code r of key j, stored at j*cstride + r
// (cstride = b for k_codes; the query order reads each row's smallest code
// with b = 1, cstride = 1).  Entries of a head number below 2^31 (run_index checks), so the
// division is 32-bit: no branches between a load's address and its use.
__device__ __forceinline__ uint32_t key_of(int64_t e, int b) {
  return static_cast<uint32_t>(e) / static_cast<uint32_t>(b);
}
__device__ __forceinline__ int64_t code_at(int64_t e, int b, int cstride) {
  const uint32_t j = key_of(e, b);
  return static_cast<int64_t>(j) * cstride + (static_cast<uint32_t>(e) - j * static_cast<uint32_t>(b));
}

__global__ __launch_bounds__(kHistThreads) void index_hist_kernel(
    const int32_t* __restrict__ k_codes, int64_t n, int b, int cstride, int n_c, int64_t tile_keys,
    int64_t tiles, int32_t* __restrict__ hist) {
  extern __shared__ int32_t lds_hist[];
  const int64_t tile = blockIdx.x;
  const int64_t bh = blockIdx.y;
  for (int c = threadIdx.x; c < n_c; c += kHistThreads) lds_hist[c] = 0;
  __syncthreads();
  const int64_t e0 = tile * tile_keys * b;
  int64_t e1 = (tile + 1) * tile_keys * b;
  if (e1 > n * b) e1 = n * b;
  const int32_t* kc = k_codes + bh * n * cstride;
  for (int64_t e = e0 + threadIdx.x; e < e1; e += kHistThreads) {
    const int32_t c = kc[code_at(e, b, cstride)];
    if (static_cast<uint32_t>(c) < static_cast<uint32_t>(n_c)) atomicAdd(&lds_hist[c], 1);
  }
  __syncthreads();
  int32_t* hb = hist + (bh * tiles + tile) * static_cast<int64_t>(n_c);
  for (int c = threadIdx.x; c < n_c; c += kHistThreads) hb[c] = lds_hist[c];
}

// Column c of a head's tile histograms summed over the tiles: eight loads
// issued before their adds, so a column of T tiles waits on T/8 memory
// latencies instead of T (integer sums: the order does not matter).
__device__ __forceinline__ int32_t column_sum(const int32_t* __restrict__ hb, int n_c, int64_t tiles, int c) {
  int32_t tot = 0;
  int64_t t = 0;
  for (; t + 8 <= tiles; t += 8) {
    int32_t v[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) v[u] = hb[(t + u) * n_c + c];
#pragma unroll
    for (int u = 0; u < 8; ++u) tot += v[u];
  }
  for (; t < tiles; ++t) tot += hb[t * n_c + c];
  return tot;
}

// Entries per chunk of kScanThreads codes: block (chunk, bh), one code per
// thread summed over the tiles, then a block sum into sums[bh][chunk].
__global__ __launch_bounds__(kScanThreads) void index_chunk_sum_kernel(const int32_t* __restrict__ hist, int n_c,
                                                                       int64_t tiles, int chunks,
                                                                       int32_t* __restrict__ sums) {
  __shared__ int32_t wsum[kScanThreads / 64];
  const int chunk = blockIdx.x;
  const int64_t bh = blockIdx.y;
  const int c = chunk * kScanThreads + static_cast<int>(threadIdx.x);
  const int32_t* hb = hist + bh * tiles * static_cast<int64_t>(n_c);
  int32_t tot = (c < n_c) ? column_sum(hb, n_c, tiles, c) : 0;
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) tot += __shfl_xor(tot, off, 64);
  if ((threadIdx.x & 63) == 0) wsum[threadIdx.x >> 6] = tot;
  __syncthreads();
  if (threadIdx.x == 0) {
    int32_t all = 0;
    for (int w = 0; w < kScanThreads / 64; ++w) all += wsum[w];
    sums[bh * chunks + chunk] = all;
  }
}

// Bucket base positions, in place: hist[bh][tile][c] (keys of code c in tile)
// becomes the number of entries before them in (code, tile) order, i.e. where
// tile `tile` starts writing bucket c; offsets[bh][c] = start of bucket c.
// Block (chunk, bh) takes kScanThreads codes (one per thread, coalesced over
// codes); its base is the sum of the earlier chunks' entries.
__global__ __launch_bounds__(kScanThreads) void index_scan_kernel(int32_t* __restrict__ hist, int n_c,
                                                                  int64_t tiles, int chunks,
                                                                  const int32_t* __restrict__ sums,
                                                                  int32_t* __restrict__ offsets) {
  __shared__ int32_t wsum[kScanThreads / 64];
  const int chunk = blockIdx.x;
  const int64_t bh = blockIdx.y;
  int32_t* hb = hist + bh * tiles * static_cast<int64_t>(n_c);
  int32_t* ob = offsets + bh * (n_c + 1);
  int32_t carry = 0;
  for (int q = 0; q < chunk; ++q) carry += sums[bh * chunks + q];
  const int c = chunk * kScanThreads + static_cast<int>(threadIdx.x);
  const int32_t tot = (c < n_c) ? column_sum(hb, n_c, tiles, c) : 0;
  const int32_t x = wave_incl_scan(tot);
  const int lane = threadIdx.x & 63;
  if (lane == 63) wsum[threadIdx.x >> 6] = x;
  __syncthreads();
  int32_t before = carry, all = 0;
  for (int w = 0; w < kScanThreads / 64; ++w) {
    const int32_t v = wsum[w];
    if (w < static_cast<int>(threadIdx.x >> 6)) before += v;
    all += v;
  }
  if (c < n_c) {
    int32_t run = before + x - tot;
    ob[c] = run;
    int64_t t = 0;
    for (; t + 8 <= tiles; t += 8) {  // eight loads out before their stores
      int32_t v[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) v[u] = hb[(t + u) * n_c + c];
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        hb[(t + u) * n_c + c] = run;
        run += v[u];
      }
    }
    for (; t < tiles; ++t) {
      const int32_t v = hb[t * n_c + c];
      hb[t * n_c + c] = run;
      run += v;
    }
  }
  if (chunk == chunks - 1 && threadIdx.x == 0) ob[n_c] = carry + all;
}

// One block of `waves` waves per (tile, bh); wave s takes the s-th of
// `waves` contiguous ranges of the tile's entries.  Entries are visited in
// index order e = j*b + r, 64 per round; lanes holding the same code are
// ranked by lane order, so every bucket receives its keys in ascending j.
// With several waves each first counts its range's codes (LDS, [waves][n_c]);
// wave s's cursor for code c then starts at the tile's base for c plus the
// counts of the ranges before it, and the waves' round loops run side by side
// (a tile's 64 rounds in one wave were a chain of memory and LDS latencies).
__global__ __launch_bounds__(256) void index_scatter_kernel(
    const int32_t* __restrict__ k_codes, int64_t n, int b, int cstride, int n_c, int code_bits,
    int64_t tile_keys, int64_t tiles, const int32_t* __restrict__ base,
    int32_t* __restrict__ postings) {
  extern __shared__ int32_t cursors[];
  const int64_t tile = blockIdx.x;
  const int64_t bh = blockIdx.y;
  const int lane = threadIdx.x & 63;
  const int wave = static_cast<int>(threadIdx.x >> 6);
  const int waves = static_cast<int>(blockDim.x >> 6);
  const int32_t* bb = base + (bh * tiles + tile) * static_cast<int64_t>(n_c);
  const int64_t t0 = tile * tile_keys * b;
  int64_t t1 = (tile + 1) * tile_keys * b;
  if (t1 > n * b) t1 = n * b;
  const int32_t* kc = k_codes + bh * n * cstride;
  const int64_t per = (t1 - t0 + waves - 1) / waves;
  const int64_t e0 = min(t0 + wave * per, t1);
  const int64_t e1 = min(e0 + per, t1);
  int32_t* cursor = cursors + static_cast<int64_t>(wave) * n_c;
  if (waves == 1) {
    for (int c = lane; c < n_c; c += 64) cursor[c] = bb[c];
  } else {
    for (int x = threadIdx.x; x < waves * n_c; x += blockDim.x) cursors[x] = 0;
    __syncthreads();
    for (int64_t e = e0 + lane; e < e1; e += 64) {
      const int32_t c = kc[code_at(e, b, cstride)];
      if (static_cast<uint32_t>(c) < static_cast<uint32_t>(n_c)) atomicAdd(&cursor[c], 1);
    }
    __syncthreads();
    for (int c = threadIdx.x; c < n_c; c += blockDim.x) {
      int32_t run = bb[c];
      for (int w = 0; w < waves; ++w) {
        const int32_t cnt = cursors[static_cast<int64_t>(w) * n_c + c];
        cursors[static_cast<int64_t>(w) * n_c + c] = run;
        run += cnt;
      }
    }
  }
  __syncthreads();
  int32_t* post = postings + bh * n * b;
  const uint64_t below = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
  // The codes of kScatterBatch rounds are loaded before any is ranked, so a
  // wave waits for memory once per batch instead of once per round.  Indices
  // past the tile are clamped to its last entry and the code replaced after
  // the load (a guarded load is waited for where it is issued).
  for (int64_t b0 = e0; b0 < e1; b0 += 64 * kScatterBatch) {
    int32_t cb[kScatterBatch];
#pragma unroll
    for (int u = 0; u < kScatterBatch; ++u) {
      const int64_t e = b0 + 64 * u + lane;
      cb[u] = kc[code_at(e < e1 ? e : e1 - 1, b, cstride)];
    }
#pragma unroll
    for (int u = 0; u < kScatterBatch; ++u) {
      const int64_t r0 = b0 + 64 * u;
      if (r0 >= e1) break;  // uniform
      const int64_t e = r0 + lane;
      const int32_t c = e < e1 ? cb[u] : -1;
      const bool ok = static_cast<uint32_t>(c) < static_cast<uint32_t>(n_c);
      uint64_t peers = __ballot(ok);
      for (int bit = 0; bit < code_bits; ++bit) {
        const bool set = ((c >> bit) & 1) != 0;
        const uint64_t m = __ballot(set);
        peers &= set ? m : ~m;
      }
      int32_t pos = 0;
      if (ok) {
        const int rank = __popcll(peers & below);
        pos = cursor[c] + rank;
        post[pos] = static_cast<int32_t>(key_of(e, b));
      }
      __builtin_amdgcn_wave_barrier();
      if (ok && (peers & below) == 0ull) cursor[c] += __popcll(peers);
      __builtin_amdgcn_wave_barrier();
    }
  }
}

__global__ void fill_i32_kernel(int32_t* __restrict__ p, int64_t count, int32_t v) {
  const int64_t e = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (e < count) p[e] = v;
}

// Per-tile bucket counts [bh][tiles][n_c], then the per-chunk entry counts
// [bh][ceil(n_c / kScanThreads)].
size_t hist_entry_bytes(int64_t bh, int64_t n, int n_c) {
  const int64_t tiles = ceil_div(n, tile_keys_for(n));
  return align_up(sizeof(int32_t) * static_cast<size_t>(bh) * n_c * tiles, 256);
}
size_t hist_bytes(int64_t bh, int64_t n, int n_c);

// The index kernels over entries (j, r < b) of every (batch, head); `hist`
// is the workspace, `offsets` receives the bucket starts.
int run_index(const int32_t* codes, int64_t bh, int64_t n, int b, int cstride, int n_c,
              int32_t* offsets, int32_t* postings, int32_t* hist, hipStream_t st) {
  if (n * b >= (int64_t(1) << 31))
    return fail(SSA_ERR_UNSUPPORTED, "index: n * b = %lld entries per head exceed int32 positions",
                static_cast<long long>(n * b));
  const int64_t tk = tile_keys_for(n);
  const int64_t tiles = ceil_div(n, tk);
  int code_bits = 0;
  while ((1 << code_bits) < n_c) ++code_bits;
  index_hist_kernel<<<dim3(static_cast<unsigned>(tiles), static_cast<unsigned>(bh)), kHistThreads,
                      sizeof(int32_t) * n_c, st>>>(codes, n, b, cstride, n_c, tk, tiles, hist);
  int s = check_launch("index_hist_kernel");
  if (s) return s;
  const int chunks = static_cast<int>(ceil_div(n_c, kScanThreads));
  int32_t* sums = reinterpret_cast<int32_t*>(reinterpret_cast<char*>(hist) + hist_entry_bytes(bh, n, n_c));
  index_chunk_sum_kernel<<<dim3(static_cast<unsigned>(chunks), static_cast<unsigned>(bh)), kScanThreads, 0, st>>>(
      hist, n_c, tiles, chunks, sums);
  if ((s = check_launch("index_chunk_sum_kernel"))) return s;
  index_scan_kernel<<<dim3(static_cast<unsigned>(chunks), static_cast<unsigned>(bh)), kScanThreads, 0, st>>>(
      hist, n_c, tiles, chunks, sums, offsets);
  if ((s = check_launch("index_scan_kernel"))) return s;
  // waves per tile: as many cursor arrays as fit 64 KB of LDS, at most 4 (N_c =
  // 4096: 4 waves; 8192: 2; 16384 and more: 1, the single-wave kernel as before)
  int waves = 4;
  while (waves > 1 && sizeof(int32_t) * static_cast<size_t>(n_c) * waves > 64 * 1024) waves >>= 1;
  index_scatter_kernel<<<dim3(static_cast<unsigned>(tiles), static_cast<unsigned>(bh)), 64 * waves,
                         sizeof(int32_t) * n_c * waves, st>>>(codes, n, b, cstride, n_c, code_bits, tk,
                                                              tiles, hist, postings);
  return check_launch("index_scatter_kernel");
}

size_t hist_bytes(int64_t bh, int64_t n, int n_c) {
  return hist_entry_bytes(bh, n, n_c) +
         align_up(sizeof(int32_t) * static_cast<size_t>(bh) * static_cast<size_t>(ceil_div(n_c, kScanThreads)), 256);
}

}  // namespace

// Library-internal: the index of codes [bh][n][b] into offsets [bh][n_c + 1]
// and postings [bh][n * b], with index_ws_bytes(bh, n, n_c) bytes of `ws`.
size_t index_ws_bytes(int64_t bh, int64_t n, int n_c) { return hist_bytes(bh, n, n_c); }
int build_index_into(const int32_t* codes, int64_t bh, int64_t n, int b, int n_c, int32_t* offsets,
                     int32_t* postings, void* ws, hipStream_t st) {
  return run_index(codes, bh, n, b, b, n_c, offsets, postings, static_cast<int32_t*>(ws), st);
}

}  // namespace ssa

using namespace ssa;

extern "C" size_t ssa_index_workspace_bytes(int64_t batch, int64_t n, int h_kv, int b, int n_c) {
  (void)b;
  if (batch < 0 || n < 0 || h_kv <= 0 || n_c <= 0) return 0;
  return hist_bytes(batch * h_kv, n, n_c);
}

extern "C" int ssa_build_index(const int32_t* k_codes, int64_t batch, int64_t n, int h_kv, int b,
                               int n_c, int32_t* offsets, int32_t* postings, void* workspace,
                               size_t workspace_bytes, void* stream) {
  if (batch < 0 || n < 0 || h_kv <= 0 || b <= 0 || n_c <= 0)
    return fail(SSA_ERR_INVALID_ARGUMENT, "build_index: bad shape");
  if (n_c > 16384) return fail(SSA_ERR_UNSUPPORTED, "build_index: num_codebook %d > 16384", n_c);
  if (n * b >= (int64_t(1) << 31))
    return fail(SSA_ERR_UNSUPPORTED, "build_index: n*b must be < 2^31");
  const size_t need = ssa_index_workspace_bytes(batch, n, h_kv, b, n_c);
  if (workspace_bytes < need)
    return fail(SSA_ERR_WORKSPACE, "build_index: workspace %zu < %zu bytes", workspace_bytes, need);
  if (batch == 0) return SSA_OK;
  if (!offsets || (n > 0 && (!k_codes || !postings || !workspace)))
    return fail(SSA_ERR_INVALID_ARGUMENT, "build_index: null pointer");
  hipStream_t st = as_stream(stream);
  const int64_t bh = batch * h_kv;
  if (n == 0) {
    const int64_t count = bh * (n_c + 1);
    fill_i32_kernel<<<dim3(static_cast<unsigned>(ceil_div(count, 256))), 256, 0, st>>>(offsets, count, 0);
    return check_launch("fill_i32_kernel");
  }
  return run_index(k_codes, bh, n, b, b, n_c, offsets, postings, static_cast<int32_t*>(workspace), st);
}

namespace ssa {
namespace {

// Smallest code of each query row: min over q_codes[row][0 .. a).  Rows that
// share their smallest code share that bucket, and with it much of their
// candidate set; grouping by it measured 2.77 ms for c3's stage (d) against
// 2.85-2.94 ms grouped by the best code q_codes[row][0].
__global__ void row_min_code_kernel(const int32_t* __restrict__ q_codes, int64_t rows, int a,
                                    int32_t* __restrict__ mins) {
  const int64_t row = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (row >= rows) return;
  const int32_t* c = q_codes + row * a;
  int32_t m = c[0];
  for (int t = 1; t < a; ++t) m = min(m, c[t]);
  mins[row] = m;
}

size_t query_order_hist_offsets_bytes(int64_t bh, int64_t n, int n_c) {
  return hist_bytes(bh, n, n_c) + align_up(sizeof(int32_t) * static_cast<size_t>(bh) * (n_c + 1), 256);
}

}  // namespace
}  // namespace ssa

using namespace ssa;

extern "C" size_t ssa_query_order_workspace_bytes(int64_t batch, int64_t n, int h_kv, int n_c) {
  if (batch < 0 || n < 0 || h_kv <= 0 || n_c <= 0) return 0;
  return query_order_hist_offsets_bytes(batch * h_kv, n, n_c) +
         align_up(sizeof(int32_t) * static_cast<size_t>(batch * h_kv * n), 256);
}

extern "C" int ssa_query_order(const int32_t* q_codes, int64_t batch, int64_t n, int h_kv, int a,
                               int n_c, int32_t* order, void* workspace, size_t workspace_bytes,
                               void* stream) {
  if (batch < 0 || n < 0 || h_kv <= 0 || a <= 0 || n_c <= 0)
    return fail(SSA_ERR_INVALID_ARGUMENT, "query_order: bad shape");
  if (n_c > 16384) return fail(SSA_ERR_UNSUPPORTED, "query_order: num_codebook %d > 16384", n_c);
  if (n * a >= (int64_t(1) << 31))
    return fail(SSA_ERR_UNSUPPORTED, "query_order: n*a must be < 2^31");
  const size_t need = ssa_query_order_workspace_bytes(batch, n, h_kv, n_c);
  if (workspace_bytes < need)
    return fail(SSA_ERR_WORKSPACE, "query_order: workspace %zu < %zu bytes", workspace_bytes, need);
  if (batch == 0 || n == 0) return SSA_OK;
  if (!q_codes || !order || !workspace) return fail(SSA_ERR_INVALID_ARGUMENT, "query_order: null pointer");
  const int64_t bh = batch * h_kv;
  int32_t* hist = static_cast<int32_t*>(workspace);
  int32_t* offsets = reinterpret_cast<int32_t*>(static_cast<char*>(workspace) + hist_bytes(bh, n, n_c));
  int32_t* mins = reinterpret_cast<int32_t*>(static_cast<char*>(workspace) +
                                             query_order_hist_offsets_bytes(bh, n, n_c));
  hipStream_t st = as_stream(stream);
  const int64_t rows = bh * n;
  row_min_code_kernel<<<dim3(static_cast<unsigned>(ceil_div(rows, 256))), 256, 0, st>>>(q_codes, rows, a, mins);
  if (int s = check_launch("row_min_code_kernel")) return s;
  return run_index(mins, bh, n, 1, 1, n_c, offsets, order, hist, st);
}
