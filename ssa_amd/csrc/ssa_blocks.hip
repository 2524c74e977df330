// Key blocks per query block (block-granular variant of the selections).
//
// ssa/triton_kernel.py:226-294 (convert_indices_to_blocks) maps a router's
// token selections [n, h_kv, top_k] to the n_k_blocks key blocks that the
// queries of each block of `block_size` positions reference most often:
//   * key j lies in block j / block_size;
//   * query rows past n (the padding of the last query block) count as top_k
//     references to block 0 each, as the reference's zero padding does;
//   * blocks are ranked by reference count; equal counts go to the lower block
//     id (the reference's torch.topk leaves that order unspecified).
//
// One block of 256 threads per (query block, KV head, batch): an LDS histogram
// over the nbk key blocks, then a bitonic sort of (count, ~id) keys in LDS.

#include "ssa_common.h"

namespace ssa {
namespace {

constexpr int kBlkThreads = 256;
constexpr int kMaxKeyBlocks = 8192;  // LDS: 4 bytes of count + 8 of sort key per block

struct BlkParams {
  const void* idx;
  int idx_i64, top_k;
  int64_t idx_sb, idx_sn, idx_sh;
  int64_t n, nbq, nbk;
  int h_kv, lg, sort_n, n_k_blocks;
  void* out;
  int out_i64;
  int64_t o_sb, o_sq, o_sh;
  int32_t* err;
};

__global__ __launch_bounds__(kBlkThreads) void block_indices_kernel(BlkParams p) {
  extern __shared__ __align__(16) unsigned char smem_raw[];
  uint64_t* keys = reinterpret_cast<uint64_t*>(smem_raw);                   // [sort_n]
  uint32_t* cnt = reinterpret_cast<uint32_t*>(keys + p.sort_n);            // [nbk]
  const int64_t bq = blockIdx.x;
  const int h = static_cast<int>(blockIdx.y);
  const int64_t bb = blockIdx.z;
  const int tid = threadIdx.x;
  for (int64_t c = tid; c < p.nbk; c += kBlkThreads) cnt[c] = 0u;
  __syncthreads();

  const int64_t bs = int64_t(1) << p.lg;
  const int64_t r0 = bq * bs;
  const int64_t real = (r0 + bs <= p.n) ? bs : p.n - r0;  // query rows of this block inside [0, n)
  const int64_t entries = real * p.top_k;
  for (int64_t e = tid; e < entries; e += kBlkThreads) {
    const int64_t r = r0 + e / p.top_k;
    const int t = static_cast<int>(e % p.top_k);
    const int64_t at = bb * p.idx_sb + r * p.idx_sn + static_cast<int64_t>(h) * p.idx_sh + t;
    const int64_t j = p.idx_i64 ? static_cast<const int64_t*>(p.idx)[at]
                                : static_cast<int64_t>(static_cast<const int32_t*>(p.idx)[at]);
    if (j < 0 || j >= p.n) {
      if (p.err) p.err[0] = 1;
      continue;
    }
    atomicAdd(&cnt[j >> p.lg], 1u);
  }
  if (tid == 0 && real < bs) atomicAdd(&cnt[0], static_cast<uint32_t>((bs - real) * p.top_k));
  __syncthreads();

  // keys: count high, ~id low, so descending key order is (count desc, id asc);
  // the padding entries (zero) sort last
  for (int64_t c = tid; c < p.sort_n; c += kBlkThreads)
    keys[c] = (c < p.nbk) ? ((static_cast<uint64_t>(cnt[c]) << 32) | (0xFFFFFFFFull - static_cast<uint64_t>(c)))
                          : 0ull;
  __syncthreads();
  for (int size = 2; size <= p.sort_n; size <<= 1) {
    for (int stride = size >> 1; stride > 0; stride >>= 1) {
      for (int t = tid; t < p.sort_n / 2; t += kBlkThreads) {
        const int i = 2 * t - (t & (stride - 1));  // lower element of pair t
        const int j = i + stride;
        const bool desc = (i & size) == 0;
        const uint64_t a = keys[i], b = keys[j];
        if ((a < b) == desc) {
          keys[i] = b;
          keys[j] = a;
        }
      }
      __syncthreads();
    }
  }
  const int64_t obase = bb * p.o_sb + bq * p.o_sq + static_cast<int64_t>(h) * p.o_sh;
  for (int t = tid; t < p.n_k_blocks; t += kBlkThreads) {
    const uint32_t id = 0xFFFFFFFFu - static_cast<uint32_t>(keys[t] & 0xFFFFFFFFull);
    if (p.out_i64) static_cast<int64_t*>(p.out)[obase + t] = id;
    else static_cast<int32_t*>(p.out)[obase + t] = static_cast<int32_t>(id);
  }
}

}  // namespace
}  // namespace ssa

using namespace ssa;

extern "C" int ssa_block_indices(const void* idx, int idx_dtype, int64_t batch, int64_t n, int h_kv, int top_k,
                                 int64_t idx_sb, int64_t idx_sn, int64_t idx_sh, int block_size,
                                 int n_k_blocks, void* out, int out_dtype, int64_t o_sb, int64_t o_sq,
                                 int64_t o_sh, int32_t* error_flag, void* stream) {
  if (idx_dtype != SSA_INDEX_I32 && idx_dtype != SSA_INDEX_I64)
    return fail(SSA_ERR_INVALID_ARGUMENT, "block_indices: idx dtype %d", idx_dtype);
  if (out_dtype != SSA_INDEX_I32 && out_dtype != SSA_INDEX_I64)
    return fail(SSA_ERR_INVALID_ARGUMENT, "block_indices: out dtype %d", out_dtype);
  if (batch < 0 || n < 0 || h_kv <= 0 || top_k < 0)
    return fail(SSA_ERR_INVALID_ARGUMENT, "block_indices: bad shape");
  if (block_size < 2 || block_size > 256 || (block_size & (block_size - 1)) != 0)
    return fail(SSA_ERR_INVALID_ARGUMENT, "block_indices: block_size %d (need a power of 2 in [2, 256])",
                block_size);
  const int64_t nbk = (n + block_size - 1) / block_size;
  if (nbk > kMaxKeyBlocks)
    return fail(SSA_ERR_UNSUPPORTED, "block_indices: %lld key blocks > %d", static_cast<long long>(nbk),
                kMaxKeyBlocks);
  if (n_k_blocks < 0 || n_k_blocks > nbk)
    return fail(SSA_ERR_INVALID_ARGUMENT, "block_indices: n_k_blocks %d outside [0, %lld]", n_k_blocks,
                static_cast<long long>(nbk));
  if (batch == 0 || n == 0 || n_k_blocks == 0) return SSA_OK;
  if (!out || (top_k > 0 && !idx)) return fail(SSA_ERR_INVALID_ARGUMENT, "block_indices: null pointer");
  if (batch > 65535) return fail(SSA_ERR_UNSUPPORTED, "block_indices: batch > 65535");
  BlkParams p{};
  p.idx = idx;
  p.idx_i64 = (idx_dtype == SSA_INDEX_I64);
  p.top_k = top_k;
  p.idx_sb = idx_sb; p.idx_sn = idx_sn; p.idx_sh = idx_sh;
  p.n = n;
  p.nbq = nbk;
  p.nbk = nbk;
  p.h_kv = h_kv;
  while ((1 << p.lg) < block_size) ++p.lg;
  p.sort_n = 2;
  while (p.sort_n < nbk) p.sort_n <<= 1;
  p.n_k_blocks = n_k_blocks;
  p.out = out;
  p.out_i64 = (out_dtype == SSA_INDEX_I64);
  p.o_sb = o_sb; p.o_sq = o_sq; p.o_sh = o_sh;
  p.err = error_flag;
  const size_t smem = sizeof(uint64_t) * static_cast<size_t>(p.sort_n) + sizeof(uint32_t) * static_cast<size_t>(nbk);
  if (int s = reserve_lds(reinterpret_cast<const void*>(block_indices_kernel), smem, "block_indices")) return s;
  block_indices_kernel<<<dim3(static_cast<unsigned>(nbk), static_cast<unsigned>(h_kv), static_cast<unsigned>(batch)),
                         kBlkThreads, smem, as_stream(stream)>>>(p);
  return check_launch("block_indices_kernel");
}
