// Incremental decoding: one step for m new tokens against a key/value cache
// (ssa_design.md:225-234: "maintained incrementally, avoiding re-scanning the
// full KV cache on each step").
//
// The cache holds K and V [batch][max_len][h_kv][d], the key codes
// [batch][h_kv][max_len][b] and two inverted indices per (batch, kv head):
//   * the main index over keys 0 .. n_base - 1, built by ssa_build_index when
//     the caller last rebuilt it;
//   * a tail index over keys n_base .. n0 + m - 1, rebuilt by every step from
//     the tail's codes alone: one block per (batch, kv head) histograms the
//     tail postings over the n_c buckets in LDS, scans, and scatters (the
//     selection unions buckets through a bitmap, so the order inside a bucket
//     does not matter).  Its cost grows with the tail, not with the cache.
// A step appends the new K/V rows and codes, routes the new rows against the
// codebook prepared once (ssa_decode_prepare), rebuilds the tail index,
// selects each new query's keys from both indices and attends them: six
// launches for a few rows, none of them over the whole cache.  The caller
// rebuilds the main index (and empties the tail) whenever the tail has grown
// past its capacity.

#include "ssa_common.h"
#include "ssa_internal.h"

namespace ssa {
namespace {

constexpr int kDecThreads = 256;

// One cache append of append_rows_kernel: the m new rows of x [batch][m][h][d]
// (byte strides) into the cache [batch][max_len][h][d] at n0 .. n0 + m - 1.
struct RowAppend {
  const unsigned char* src;
  unsigned char* dst;
  int64_t s_sb, s_sn, s_sh, d_sb, d_sn, d_sh;
};

// Appends K (blockIdx.y = 0) and V (blockIdx.y = 1), 16 bytes per thread (rows
// are 16-byte aligned; d * esize is a multiple of 16).
__global__ __launch_bounds__(kDecThreads) void append_rows_kernel(RowAppend k, RowAppend v, int64_t batch,
                                                                  int64_t m, int h, int row_bytes, int64_t n0) {
  const RowAppend& a = blockIdx.y ? v : k;
  const int per_row = row_bytes / 16;
  const int64_t t = static_cast<int64_t>(blockIdx.x) * kDecThreads + threadIdx.x;
  const int64_t total = batch * m * h * per_row;
  if (t >= total) return;
  const int piece = static_cast<int>(t % per_row);
  const int64_t row = t / per_row;
  const int hh = static_cast<int>(row % h);
  const int64_t bi = row / h;
  const int64_t i = bi % m;
  const int64_t b = bi / m;
  const uint4 x = *reinterpret_cast<const uint4*>(a.src + b * a.s_sb + i * a.s_sn + hh * a.s_sh + 16 * piece);
  *reinterpret_cast<uint4*>(a.dst + b * a.d_sb + (n0 + i) * a.d_sn + hh * a.d_sh + 16 * piece) = x;
}

// Tail index of one (batch, kv head) over keys n_base .. n0 + m - 1: the
// cached codes of keys n_base .. n0 - 1 and the step's new codes new_codes
// [batch * h][m][b], which the block also appends to the code cache
// [batch * h][max_len][b] at n0.  offsets [n_c + 1] (bucket c =
// postings[offsets[c] .. offsets[c+1]), holding key - n_base); codes outside
// [0, n_c) are skipped.
__global__ __launch_bounds__(kDecThreads) void tail_index_kernel(
    const int32_t* __restrict__ new_codes, int32_t* __restrict__ codes, int64_t max_len, int b,
    int64_t n_base, int64_t n0, int64_t m, int n_c, int32_t* __restrict__ offsets,
    int32_t* __restrict__ postings, int64_t tail_cap) {
  extern __shared__ __align__(16) unsigned char smem_raw[];
  uint32_t* cnt = reinterpret_cast<uint32_t*>(smem_raw);  // [n_c], then the cursors
  __shared__ uint32_t s_wsum[kDecThreads / 64];
  const int64_t bh = blockIdx.x;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int32_t* cb = codes + bh * max_len * b + n_base * b;
  const int32_t* nb = new_codes + bh * m * b;
  const int64_t old_entries = (n0 - n_base) * b;
  const int64_t entries = old_entries + m * b;
  const auto code_at = [&](int64_t e) { return e < old_entries ? cb[e] : nb[e - old_entries]; };
  int32_t* dst = codes + bh * max_len * b + n0 * b;
  strided_batches<4, kDecThreads>(m * b, tid, [&](int64_t e) { return nb[e]; },
                                  [&](int64_t e, int32_t c) { dst[e] = c; });
  for (int c = tid; c < n_c; c += kDecThreads) cnt[c] = 0u;
  __syncthreads();
  strided_batches<8, kDecThreads>(entries, tid, code_at, [&](int64_t, int32_t c) {
    if (static_cast<uint32_t>(c) < static_cast<uint32_t>(n_c)) atomicAdd(&cnt[c], 1u);
  });
  __syncthreads();
  // exclusive scan: thread t owns codes [t * per, (t + 1) * per)
  const int per = (n_c + kDecThreads - 1) / kDecThreads;
  const int c0 = tid * per;
  uint32_t mine = 0;
  for (int c = c0; c < c0 + per && c < n_c; ++c) mine += cnt[c];
  uint32_t incl = mine;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const uint32_t y = __shfl_up(incl, o);
    if (lane >= o) incl += y;
  }
  if (lane == 63) s_wsum[wave] = incl;
  __syncthreads();
  uint32_t base = 0;
  for (int w = 0; w < wave; ++w) base += s_wsum[w];
  uint32_t run = base + incl - mine;
  int32_t* off = offsets + bh * (n_c + 1);
  for (int c = c0; c < c0 + per && c < n_c; ++c) {
    const uint32_t x = cnt[c];
    off[c] = static_cast<int32_t>(run);
    cnt[c] = run;  // becomes the bucket's cursor
    run += x;
  }
  if (tid == kDecThreads - 1) off[n_c] = static_cast<int32_t>(run);
  __syncthreads();
  int32_t* post = postings + bh * tail_cap;
  strided_batches<8, kDecThreads>(entries, tid, code_at, [&](int64_t e, int32_t c) {
    if (static_cast<uint32_t>(c) < static_cast<uint32_t>(n_c)) {
      const uint32_t slot = atomicAdd(&cnt[c], 1u);
      if (slot < static_cast<uint64_t>(tail_cap)) post[slot] = static_cast<int32_t>(e / b);
    }
  });
}

int esize_of(int dtype) { return dtype == SSA_DTYPE_F32 ? 4 : 2; }

struct DecWs {
  int32_t* q_codes;  // [batch][h_kv][m][a]
  int32_t* k_codes;  // [batch][h_kv][m][b]
  int32_t* idx;      // [batch][m][h_kv][top_k]
  void* route;       // routing vectors and flags
};

size_t dec_ws_bytes(int64_t batch, int64_t m, int h_kv, int d_s, int n_c, int a, int b, int top_k) {
  const int64_t rows = batch * h_kv * m;
  return align_up(sizeof(int32_t) * static_cast<size_t>(rows * a), 256) +
         align_up(sizeof(int32_t) * static_cast<size_t>(rows * b), 256) +
         align_up(sizeof(int32_t) * static_cast<size_t>(rows * top_k), 256) +
         route_prepped_ws_bytes(batch, m, h_kv, d_s, n_c);
}

DecWs carve_dec(void* ws, int64_t batch, int64_t m, int h_kv, int a, int b, int top_k) {
  const int64_t rows = batch * h_kv * m;
  char* c = static_cast<char*>(ws);
  DecWs w{};
  w.q_codes = reinterpret_cast<int32_t*>(c);
  c += align_up(sizeof(int32_t) * static_cast<size_t>(rows * a), 256);
  w.k_codes = reinterpret_cast<int32_t*>(c);
  c += align_up(sizeof(int32_t) * static_cast<size_t>(rows * b), 256);
  w.idx = reinterpret_cast<int32_t*>(c);
  c += align_up(sizeof(int32_t) * static_cast<size_t>(rows * top_k), 256);
  w.route = c;
  return w;
}

}  // namespace
}  // namespace ssa

using namespace ssa;

extern "C" size_t ssa_decode_prepare_bytes(int h_kv, int n_c, int d_s) {
  if (h_kv <= 0 || n_c <= 0 || d_s <= 0) return 0;
  return decode_prep_bytes(h_kv, n_c, d_s);
}

extern "C" int ssa_decode_prepare(const float* codebook, int h_kv, int n_c, int d_s, void* prep,
                                  size_t prep_bytes, void* stream) {
  if (h_kv <= 0 || n_c <= 0 || d_s <= 0 || d_s > 32)
    return fail(SSA_ERR_INVALID_ARGUMENT, "decode_prepare: bad shape (d_s <= 32)");
  if (!codebook || !prep) return fail(SSA_ERR_INVALID_ARGUMENT, "decode_prepare: null pointer");
  if (prep_bytes < decode_prep_bytes(h_kv, n_c, d_s))
    return fail(SSA_ERR_WORKSPACE, "decode_prepare: %zu < %zu bytes", prep_bytes,
                decode_prep_bytes(h_kv, n_c, d_s));
  return decode_prep(codebook, h_kv, n_c, d_s, prep, as_stream(stream));
}

extern "C" size_t ssa_decode_workspace_bytes(int64_t batch, int64_t m, int h_kv, int d_s, int n_c,
                                             int a, int b, int top_k) {
  if (batch < 0 || m < 0 || h_kv <= 0 || d_s <= 0 || n_c <= 0 || a <= 0 || b <= 0 || top_k <= 0) return 0;
  return dec_ws_bytes(batch, m, h_kv, d_s, n_c, a, b, top_k);
}

extern "C" int ssa_decode_step(
    const void* q, const void* k, const void* v, int dtype, int64_t batch, int64_t m, int h_q,
    int h_kv, int d, int64_t q_sb, int64_t q_sn, int64_t q_sh, int64_t k_sb, int64_t k_sn,
    int64_t k_sh, int64_t v_sb, int64_t v_sn, int64_t v_sh, void* k_cache, void* v_cache,
    int64_t max_len, int64_t kc_sb, int64_t kc_sn, int64_t kc_sh, int64_t vc_sb, int64_t vc_sn,
    int64_t vc_sh, int64_t n0, const float* w_qr, const float* w_kr, const void* prep, int d_s,
    int n_c, int a, int b, float temperature, int32_t* k_codes, const int32_t* offsets,
    const int32_t* postings, int64_t n_base, int32_t* tail_offsets, int32_t* tail_postings,
    int64_t tail_cap, int top_k, float score_div, float scale_div, int causal, int32_t* indices,
    void* out, int out_dtype, int64_t o_sb, int64_t o_sn, int64_t o_sh, void* workspace,
    size_t workspace_bytes, void* stream) {
  if (dtype != SSA_DTYPE_F32 && dtype != SSA_DTYPE_BF16)
    return fail(SSA_ERR_UNSUPPORTED, "decode_step: dtype %d not supported (f32, bf16)", dtype);
  if (batch < 0 || m < 0 || h_q <= 0 || h_kv <= 0 || d <= 0 || a <= 0 || b <= 0 || n_c <= 0 ||
      top_k <= 0 || h_q % h_kv != 0)
    return fail(SSA_ERR_INVALID_ARGUMENT, "decode_step: bad shape");
  if (n0 < 0 || n0 + m > max_len)
    return fail(SSA_ERR_INVALID_ARGUMENT, "decode_step: %lld + %lld tokens exceed the cache (%lld)",
                static_cast<long long>(n0), static_cast<long long>(m), static_cast<long long>(max_len));
  if (n_base < 0 || n_base > n0)
    return fail(SSA_ERR_INVALID_ARGUMENT, "decode_step: the main index covers %lld keys, more than "
                "the %lld cached", static_cast<long long>(n_base), static_cast<long long>(n0));
  if ((n0 + m - n_base) * b > tail_cap)
    return fail(SSA_ERR_WORKSPACE, "decode_step: the tail of %lld keys needs %lld postings > tail_cap "
                "%lld; rebuild the main index", static_cast<long long>(n0 + m - n_base),
                static_cast<long long>((n0 + m - n_base) * b), static_cast<long long>(tail_cap));
  if ((d * esize_of(dtype)) % 16 != 0)
    return fail(SSA_ERR_UNSUPPORTED, "decode_step: rows must be a multiple of 16 bytes");
  {
    const int64_t vec = 16 / esize_of(dtype);
    const auto al = [](const void* ptr) { return reinterpret_cast<uintptr_t>(ptr) % 16 == 0; };
    if (k_sb % vec || k_sn % vec || k_sh % vec || v_sb % vec || v_sn % vec || v_sh % vec ||
        kc_sb % vec || kc_sn % vec || kc_sh % vec || vc_sb % vec || vc_sn % vec || vc_sh % vec ||
        !al(k) || !al(v) || !al(k_cache) || !al(v_cache))
      return fail(SSA_ERR_UNSUPPORTED, "decode_step: k/v rows and cache rows must be 16-byte aligned");
  }
  if (workspace_bytes < dec_ws_bytes(batch, m, h_kv, d_s, n_c, a, b, top_k))
    return fail(SSA_ERR_WORKSPACE, "decode_step: workspace %zu < %zu bytes", workspace_bytes,
                dec_ws_bytes(batch, m, h_kv, d_s, n_c, a, b, top_k));
  const size_t tail_lds = sizeof(uint32_t) * static_cast<size_t>(n_c);
  if (tail_lds > 64 * 1024)
    return fail(SSA_ERR_UNSUPPORTED, "decode_step: n_c %d > 16384", n_c);
  if (batch == 0 || m == 0) return SSA_OK;
  if (!q || !k || !v || !k_cache || !v_cache || !w_qr || !w_kr || !prep || !k_codes || !offsets ||
      !postings || !tail_offsets || !tail_postings || !out || !workspace)
    return fail(SSA_ERR_INVALID_ARGUMENT, "decode_step: null pointer");
  hipStream_t st = as_stream(stream);
  const int es = esize_of(dtype);
  const int64_t n = n0 + m;
  DecWs w = carve_dec(workspace, batch, m, h_kv, a, b, top_k);
  int32_t* idx = indices ? indices : w.idx;

  // 1. append the new K and V rows
  {
    const int64_t total = batch * m * h_kv * (d * es / 16);
    const dim3 grid(static_cast<unsigned>(ceil_div(total, kDecThreads)), 2);
    const RowAppend ka{static_cast<const unsigned char*>(k), static_cast<unsigned char*>(k_cache),
                       k_sb * es, k_sn * es, k_sh * es, kc_sb * es, kc_sn * es, kc_sh * es};
    const RowAppend va{static_cast<const unsigned char*>(v), static_cast<unsigned char*>(v_cache),
                       v_sb * es, v_sn * es, v_sh * es, vc_sb * es, vc_sn * es, vc_sh * es};
    append_rows_kernel<<<grid, kDecThreads, 0, st>>>(ka, va, batch, m, h_kv, d * es, n0);
    if (int s = check_launch("append_rows_kernel")) return s;
  }
  // 2. route the new queries and keys
  if (int s = route_codes_prepped(q, k, dtype, batch, m, h_q, h_kv, d, q_sb, q_sn, q_sh, k_sb, k_sn, k_sh,
                                  w_qr, w_kr, prep, d_s, n_c, a, b, temperature, w.q_codes, w.k_codes,
                                  w.route, st))
    return s;
  // 3. append the new key codes and rebuild the tail index (one launch)
  {
    if (int s = reserve_lds(reinterpret_cast<const void*>(tail_index_kernel), tail_lds, "tail_index")) return s;
    tail_index_kernel<<<dim3(static_cast<unsigned>(batch * h_kv)), kDecThreads, tail_lds, st>>>(
        w.k_codes, k_codes, max_len, b, n_base, n0, m, n_c, tail_offsets, tail_postings, tail_cap);
    if (int s = check_launch("tail_index_kernel")) return s;
  }
  // 4. select the new rows' keys from both indices (index order, one block per row)
  if (int s = select_entry(q, k_cache, dtype, batch, n, m, n0, h_q, h_kv, d, q_sb, q_sn, q_sh, kc_sb,
                           kc_sn, kc_sh, w.q_codes, a, offsets, postings, n_c, b, top_k, SSA_MASK_CAUSAL,
                           nullptr, 0, 0, score_div, 0, nullptr, idx, SSA_INDEX_I32, nullptr, nullptr, 0,
                           stream, n_base * b, tail_offsets, tail_postings, tail_cap, n_base))
    return s;
  // 5. attention of the new rows over the whole cache
  return attention_entry(q, k_cache, v_cache, dtype, batch, n, m, n0, h_q, h_kv, d, q_sb, q_sn, q_sh, kc_sb,
                         kc_sn, kc_sh, vc_sb, vc_sn, vc_sh, idx, SSA_INDEX_I32, top_k,
                         m * h_kv * static_cast<int64_t>(top_k), h_kv * static_cast<int64_t>(top_k), top_k,
                         scale_div, causal, nullptr, out, out_dtype, o_sb, o_sn, o_sh, nullptr, stream, 0, 0);
}
