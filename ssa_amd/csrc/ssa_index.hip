// Stage (b): inverted index code -> keys, deterministic and stable.
//
// No reference counterpart: the reference materialises the [n, h, n] mask by
// broadcast compare (ssa/router.py:241-257).  The index reproduces the same
// key sets per code, and its postings ascend inside each bucket, so offsets and
// postings are bit-identical with the CPU oracle.
//
// Three kernels per (batch, kv-head) pair "bh", keys cut into tiles of
// `tile_keys` keys (tile_keys*b entries):
//   1. index_hist    : per-tile LDS histogram of codes -> hist[bh][c][tile]
//   2. index_scan    : exclusive scan of hist in (code, tile) order -> base
//                      positions; offsets[bh][c] = base[c][0]
//   3. index_scatter : one wave per tile walks its entries in order; lanes that
//                      share a code rank themselves by ballot (lowest lane =
//                      lowest key first) and advance an LDS cursor per code.
#include "ssa_common.h"

namespace ssa {
namespace {

constexpr int kHistThreads = 256;
constexpr int kScanThreads = 1024;

int64_t tile_keys_for(int64_t n) {
  int64_t tk = ceil_div(n, 64);
  tk = ceil_div(tk, 64) * 64;
  return tk < 1024 ? 1024 : tk;
}

__global__ __launch_bounds__(kHistThreads) void index_hist_kernel(
    const int32_t* __restrict__ k_codes, int64_t n, int b, int n_c, int64_t tile_keys,
    int64_t tiles, int32_t* __restrict__ hist) {
  extern __shared__ int32_t lds_hist[];
  const int64_t tile = blockIdx.x;
  const int64_t bh = blockIdx.y;
  for (int c = threadIdx.x; c < n_c; c += kHistThreads) lds_hist[c] = 0;
  __syncthreads();
  const int64_t e0 = tile * tile_keys * b;
  int64_t e1 = (tile + 1) * tile_keys * b;
  if (e1 > n * b) e1 = n * b;
  const int32_t* kc = k_codes + bh * n * b;
  for (int64_t e = e0 + threadIdx.x; e < e1; e += kHistThreads) {
    const int32_t c = kc[e];
    if (static_cast<uint32_t>(c) < static_cast<uint32_t>(n_c)) atomicAdd(&lds_hist[c], 1);
  }
  __syncthreads();
  int32_t* hb = hist + bh * static_cast<int64_t>(n_c) * tiles;
  for (int c = threadIdx.x; c < n_c; c += kHistThreads) hb[static_cast<int64_t>(c) * tiles + tile] = lds_hist[c];
}

// Exclusive scan over hist[bh][0 .. n_c*tiles) in place; writes offsets.
__global__ __launch_bounds__(kScanThreads) void index_scan_kernel(int32_t* __restrict__ hist,
                                                                  int n_c, int64_t tiles,
                                                                  int32_t* __restrict__ offsets) {
  __shared__ int32_t part[kScanThreads];
  const int64_t bh = blockIdx.x;
  const int64_t total = static_cast<int64_t>(n_c) * tiles;
  int32_t* hb = hist + bh * total;
  const int64_t per = ceil_div(total, kScanThreads);
  const int64_t s0 = threadIdx.x * per;
  int64_t s1 = s0 + per;
  if (s1 > total) s1 = total;
  int32_t local = 0;
  for (int64_t e = s0; e < s1; ++e) local += hb[e];
  part[threadIdx.x] = local;
  __syncthreads();
  // Hillis-Steele inclusive scan of the per-thread sums.
  for (int off = 1; off < kScanThreads; off <<= 1) {
    const int32_t v = (static_cast<int>(threadIdx.x) >= off) ? part[threadIdx.x - off] : 0;
    __syncthreads();
    part[threadIdx.x] += v;
    __syncthreads();
  }
  int32_t run = part[threadIdx.x] - local;
  for (int64_t e = s0; e < s1; ++e) {
    const int32_t v = hb[e];
    hb[e] = run;
    run += v;
  }
  __syncthreads();
  int32_t* ob = offsets + bh * (n_c + 1);
  for (int c = threadIdx.x; c < n_c; c += kScanThreads) ob[c] = hb[static_cast<int64_t>(c) * tiles];
  if (threadIdx.x == kScanThreads - 1) ob[n_c] = part[kScanThreads - 1];
}

// One wave per (tile, bh).  Entries are visited in index order e = j*b + r, 64
// per round; lanes holding the same code are ranked by lane order, so every
// bucket receives its keys in ascending j.
__global__ __launch_bounds__(64) void index_scatter_kernel(
    const int32_t* __restrict__ k_codes, int64_t n, int b, int n_c, int code_bits,
    int64_t tile_keys, int64_t tiles, const int32_t* __restrict__ base,
    int32_t* __restrict__ postings) {
  extern __shared__ int32_t cursor[];
  const int64_t tile = blockIdx.x;
  const int64_t bh = blockIdx.y;
  const int lane = threadIdx.x;
  const int32_t* bb = base + bh * static_cast<int64_t>(n_c) * tiles;
  for (int c = lane; c < n_c; c += 64) cursor[c] = bb[static_cast<int64_t>(c) * tiles + tile];
  __syncthreads();
  const int64_t e0 = tile * tile_keys * b;
  int64_t e1 = (tile + 1) * tile_keys * b;
  if (e1 > n * b) e1 = n * b;
  const int32_t* kc = k_codes + bh * n * b;
  int32_t* post = postings + bh * n * b;
  const uint64_t below = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
  for (int64_t r0 = e0; r0 < e1; r0 += 64) {
    const int64_t e = r0 + lane;
    int32_t c = -1;
    if (e < e1) c = kc[e];
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
      post[pos] = static_cast<int32_t>(e / b);
    }
    __builtin_amdgcn_wave_barrier();
    if (ok && (peers & below) == 0ull) cursor[c] += __popcll(peers);
    __builtin_amdgcn_wave_barrier();
  }
}

__global__ void fill_i32_kernel(int32_t* __restrict__ p, int64_t count, int32_t v) {
  const int64_t e = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (e < count) p[e] = v;
}

}  // namespace
}  // namespace ssa

using namespace ssa;

extern "C" size_t ssa_index_workspace_bytes(int64_t batch, int64_t n, int h_kv, int b, int n_c) {
  (void)b;
  if (batch < 0 || n < 0 || h_kv <= 0 || n_c <= 0) return 0;
  const int64_t tiles = ceil_div(n, tile_keys_for(n));
  return align_up(sizeof(int32_t) * static_cast<size_t>(batch * h_kv) * n_c * tiles, 256);
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
  const int64_t tk = tile_keys_for(n);
  const int64_t tiles = ceil_div(n, tk);
  int32_t* hist = static_cast<int32_t*>(workspace);
  int code_bits = 0;
  while ((1 << code_bits) < n_c) ++code_bits;
  index_hist_kernel<<<dim3(static_cast<unsigned>(tiles), static_cast<unsigned>(bh)), kHistThreads,
                      sizeof(int32_t) * n_c, st>>>(k_codes, n, b, n_c, tk, tiles, hist);
  int s = check_launch("index_hist_kernel");
  if (s) return s;
  index_scan_kernel<<<dim3(static_cast<unsigned>(bh)), kScanThreads, 0, st>>>(hist, n_c, tiles,
                                                                               offsets);
  if ((s = check_launch("index_scan_kernel"))) return s;
  index_scatter_kernel<<<dim3(static_cast<unsigned>(tiles), static_cast<unsigned>(bh)), 64,
                         sizeof(int32_t) * n_c, st>>>(k_codes, n, b, n_c, code_bits, tk, tiles,
                                                      hist, postings);
  return check_launch("index_scatter_kernel");
}
