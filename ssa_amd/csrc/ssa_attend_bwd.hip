// Stage (d) backward: gradients of the gathered exact attention.
//
// The reference gets them from autograd through gather -> einsum -> / scale ->
// softmax -> einsum (ssa/attention.py:64-113).  With s_t = q . k_t / scale,
// p = softmax(s) over the slots of a (query, head) row, o = sum_t p_t v_t and
// D = dO . o:
//   dv[idx_t] += p_t dO
//   ds_t       = p_t (dO . v_t - D)
//   dq        += ds_t k_t / scale
//   dk[idx_t] += ds_t q / scale
// Slots repeat with duplicated indices and then contribute once per slot, as
// the reference's gather does; dropped slots (causal cut, index outside [0, n))
// contribute nothing.
//
// One wave per (batch, kv head, query) row, as in the forward: lane l holds
// dimensions l, l + 64, ... of the g query heads' q, dO and dq in registers.
// Pass 1 recomputes each head's running max and sum over the slots; pass 2
// recomputes p, forms ds and accumulates dq in registers, and adds the row's
// g-head sums for dk[idx_t] and dv[idx_t] with fp32 atomics (many rows select
// the same key).  All arithmetic is fp32; dq, dk and dv are fp32 buffers.
#include "ssa_common.h"
#include "ssa_internal.h"
#include "ssa_rows.h"

namespace ssa {
namespace {

constexpr int kBwdWaves = 4;

struct BwdParams {
  const void* q;
  const void* k;
  const void* v;
  const void* o;
  const void* dout;
  int64_t n;
  int h_q, h_kv, g, d;
  int64_t q_sb, q_sn, q_sh, k_sb, k_sn, k_sh, v_sb, v_sn, v_sh;
  int64_t o_sb, o_sn, o_sh, do_sb, do_sn, do_sh;
  int o_bf16, do_bf16;  // o and dO storage (bf16 or fp32), independent of q/k/v
  const void* idx;
  int idx_i64, top_k;
  int64_t idx_sb, idx_sn, idx_sh;
  float inv_scale;      // 1 / scale_div
  float qk_scale_log2;  // log2(e) / scale_div
  int causal;
  float* dq;  // [B][n][h_q][d]
  float* dk;  // [B][n][h_kv][d]
  float* dv;  // [B][n][h_kv][d]
  int32_t* err;
  int64_t rows;
  const int32_t* order;  // nullable [B*h_kv][n]
  // Dense key prefixes (nullable; matrix-core path): X per row [B*h_kv][n] as
  // the selection writes it, and per (row, head) the softmax reference, the
  // reciprocal sum and D = dO . o that the row kernel found ([rows][g][4]).
  // The row kernel then skips indices below X; prefix_attention_bwd_kernel
  // handles them for blocks of neighbouring rows.
  const int32_t* pfx;
  float* pstats;
  // Bucket mode (nullable [rows], with pfx): the candidate slots' dk and dv
  // come from bucket_attention_bwd_kernel, so the row kernel adds them only
  // for rows marked -1 here (rows without filler that got no key bitmap).
  const int32_t* rowmap;
  // Nullable [rows][g][2]: the forward's softmax reference and 1 / sum per
  // (row, head); a row whose entry is not NaN skips the row kernel's pass 1.
  const float* stats_in;
  // prefix_attention_bwd_kernel adds dq only (the prefix keys' dk and dv come
  // from bucket_attention_bwd_kernel's prefix mode)
  int pfx_dq_only;
};

__device__ __forceinline__ float ld_any(const void* p, int64_t off, int is_bf16) {
  return is_bf16 ? bf16_bits_to_f32(static_cast<const uint16_t*>(p)[off])
                 : static_cast<const float*>(p)[off];
}

// Sum over the 64 lanes; every lane receives it (same value on every lane).
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
  return v;
}

__global__ void zero_f32_kernel(float* __restrict__ p, int64_t count) {
  const int64_t e = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (e < count) p[e] = 0.0f;
}

template <typename T, int GMAX, int R>
__global__ __launch_bounds__(64 * kBwdWaves) void sparse_attention_bwd_kernel(BwdParams p) {
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const int64_t lrow = static_cast<int64_t>(blockIdx.x) * kBwdWaves + wave;
  if (lrow >= p.rows) return;
  const int64_t bh = lrow / p.n;
  int64_t i = lrow - bh * p.n;
  if (p.order) {
    const int64_t oi = p.order[lrow];
    if (oi < 0 || oi >= p.n) {
      if (lane == 0 && p.err) p.err[0] = 1;
      return;
    }
    i = oi;
  }
  const int h = static_cast<int>(bh % p.h_kv);
  const int64_t bb = bh / p.h_kv;
  const int g = p.g;
  const T* kb = static_cast<const T*>(p.k) + bb * p.k_sb + h * p.k_sh;
  const T* vb = static_cast<const T*>(p.v) + bb * p.v_sb + h * p.v_sh;

  float qv[GMAX][R], dov[GMAX][R], dqv[GMAX][R], dd[GMAX], mx[GMAX], sm[GMAX];
#pragma unroll
  for (int j = 0; j < GMAX; ++j) {
    const int hq = h * g + (j < g ? j : 0);
    float od = 0.0f;
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int dim = lane + 64 * r;
      const bool ok = j < g && dim < p.d;
      qv[j][r] = ok ? ld(static_cast<const T*>(p.q) + bb * p.q_sb + i * p.q_sn + hq * p.q_sh + dim) : 0.0f;
      dov[j][r] = ok ? ld_any(p.dout, bb * p.do_sb + i * p.do_sn + hq * p.do_sh + dim, p.do_bf16) : 0.0f;
      const float ov = ok ? ld_any(p.o, bb * p.o_sb + i * p.o_sn + hq * p.o_sh + dim, p.o_bf16) : 0.0f;
      od = fma_rn(dov[j][r], ov, od);
      dqv[j][r] = 0.0f;
    }
    dd[j] = wave_sum(od);
    mx[j] = -INFINITY;
    sm[j] = 0.0f;
  }

  const unsigned char* ib = static_cast<const unsigned char*>(p.idx) +
                            (bb * p.idx_sb + i * p.idx_sn + h * p.idx_sh) * (p.idx_i64 ? 8 : 4);
  auto key_at = [&](int t, bool* ok) -> int64_t {
    const int64_t key = p.idx_i64 ? reinterpret_cast<const int64_t*>(ib)[t]
                                  : static_cast<int64_t>(reinterpret_cast<const int32_t*>(ib)[t]);
    const bool in_range = key >= 0 && key < p.n;
    if (!in_range && lane == 0 && p.err) p.err[0] = 1;
    *ok = in_range && !(p.causal && key > i);
    return key;
  };

  // ---- pass 1: per-head max and sum of exp over the row's slots
  for (int t = 0; t < p.top_k; ++t) {
    bool ok;
    const int64_t key = key_at(t, &ok);
    if (!ok) continue;  // uniform: every lane read the same index
    float kv[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int dim = lane + 64 * r;
      kv[r] = dim < p.d ? ld(kb + key * p.k_sn + dim) : 0.0f;
    }
#pragma unroll
    for (int j = 0; j < GMAX; ++j) {
      if (j < g) {
        float part = 0.0f;
#pragma unroll
        for (int r = 0; r < R; ++r) part = fma_rn(qv[j][r], kv[r], part);
        const float s = wave_sum(part) * p.inv_scale;
        const float mn = fmaxf(mx[j], s);
        sm[j] = sm[j] * expf(mx[j] - mn) + expf(s - mn);
        mx[j] = mn;
      }
    }
  }

  // ---- pass 2: p, ds; dq in registers, dk and dv by atomics
  float* dkb = p.dk + (bb * p.n * p.h_kv + h) * p.d;
  float* dvb = p.dv + (bb * p.n * p.h_kv + h) * p.d;
  const int64_t krow = static_cast<int64_t>(p.h_kv) * p.d;
  float inv_sum[GMAX];
#pragma unroll
  for (int j = 0; j < GMAX; ++j) inv_sum[j] = sm[j] > 0.0f ? 1.0f / sm[j] : 0.0f;
  for (int t = 0; t < p.top_k; ++t) {
    bool ok;
    const int64_t key = key_at(t, &ok);
    if (!ok) continue;
    float kv[R], vv[R], dk_acc[R], dv_acc[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int dim = lane + 64 * r;
      kv[r] = dim < p.d ? ld(kb + key * p.k_sn + dim) : 0.0f;
      vv[r] = dim < p.d ? ld(vb + key * p.v_sn + dim) : 0.0f;
      dk_acc[r] = 0.0f;
      dv_acc[r] = 0.0f;
    }
#pragma unroll
    for (int j = 0; j < GMAX; ++j) {
      if (j < g) {
        float part = 0.0f, pdv = 0.0f;
#pragma unroll
        for (int r = 0; r < R; ++r) {
          part = fma_rn(qv[j][r], kv[r], part);
          pdv = fma_rn(dov[j][r], vv[r], pdv);
        }
        const float s = wave_sum(part) * p.inv_scale;
        const float dp = wave_sum(pdv);
        const float pr = expf(s - mx[j]) * inv_sum[j];
        const float ds = pr * (dp - dd[j]);
#pragma unroll
        for (int r = 0; r < R; ++r) {
          dqv[j][r] = fma_rn(ds, kv[r], dqv[j][r]);
          dk_acc[r] = fma_rn(ds, qv[j][r], dk_acc[r]);
          dv_acc[r] = fma_rn(pr, dov[j][r], dv_acc[r]);
        }
      }
    }
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int dim = lane + 64 * r;
      if (dim < p.d) {
        unsafeAtomicAdd(dkb + key * krow + dim, dk_acc[r] * p.inv_scale);
        unsafeAtomicAdd(dvb + key * krow + dim, dv_acc[r]);
      }
    }
  }

  float* dqb = p.dq + ((bb * p.n + i) * p.h_q + h * g) * p.d;
#pragma unroll
  for (int j = 0; j < GMAX; ++j) {
    if (j < g) {
#pragma unroll
      for (int r = 0; r < R; ++r) {
        const int dim = lane + 64 * r;
        if (dim < p.d) dqb[j * p.d + dim] = dqv[j][r] * p.inv_scale;
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Matrix-core backward (bf16 q/k/v/dO, d = 64 or 128, g <= 8).  One wave per
// (batch, kv head, query) row, 32-key chunks gathered whole into the wave's LDS
// as in the forward kernel (buffer loads straight to LDS, XOR-swizzled rows):
//   pass 1   S^T = K Q^T (MFMA) per chunk, running max and sum of exp2 per head;
//   pass 2   S^T again and dP^T = V dO^T (MFMA, same layout: lane (q4, c16) holds
//            keys 16t + 4 q4 + e of head c16), p = exp2(s - m) / l,
//            ds = p (dP - D);
//            dQ^T += K^T dS^T like the forward's O^T += V^T P^T (A = K^T from
//            transposing LDS reads, B = dS split into bf16 hi (rows < g) and lo
//            (rows 8 + r));
//            dV_chunk = P^T dO and dK_chunk = dS^T Q: P and dS go through LDS to
//            [key][head], A = [hi | lo] over heads (k = 0..7 hi, 8..15 lo), B =
//            dO / Q rows by head (stored transposed in LDS once per row), and the
//            16 x 16 result tiles go to dv / dk with fp32 atomics.
// The hi/lo splits keep about 16 mantissa bits of p and ds; q, k, v and dO are
// exact in bf16.
constexpr int kBwMfWaves = 2;

// DKDV = false: dq only, for the rows whose dk and dv the bucket kernel adds
// (rowmap != -1); DKDV = true: every row, or in bucket mode only rowmap == -1.
template <int D, bool DKDV>
__global__ __launch_bounds__(64 * kBwMfWaves, 2) void sparse_attention_bwd_mfma_kernel(BwdParams p) {
  using S = MfShape<D>;
  constexpr int KB = S::KB, NT = S::NT;
  constexpr int TW = DKDV ? kBwMfWaves : 1;  // the dk / dv staging exists only in the DKDV build
  __shared__ __align__(16) unsigned char kv_lds[kBwMfWaves][2][kMfChunk * S::ROW];
  __shared__ __align__(16) float tr_lds[TW][kMfChunk][16];      // P or dS as [key][head]
  __shared__ __align__(16) uint16_t hd_lds[TW][2][D][8];        // Q, dO as [dim][head] (bf16)

  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const int q4 = lane >> 4, c16 = lane & 15;
  const int64_t lrow = static_cast<int64_t>(blockIdx.x) * kBwMfWaves + wave;
  if (lrow >= p.rows) return;  // wave-uniform; the kernel has no block barrier
  const int64_t bh = lrow / p.n;
  int64_t i = lrow - bh * p.n;
  if (p.order) {
    const int64_t oi = p.order[lrow];
    if (oi < 0 || oi >= p.n) {
      if (lane == 0 && p.err) p.err[0] = 1;
      return;
    }
    i = oi;
  }
  if (p.rowmap && DKDV != (p.rowmap[bh * p.n + i] == -1)) return;  // the other build takes this row
  const int h = static_cast<int>(bh % p.h_kv);
  const int64_t bb = bh / p.h_kv;
  const int g = p.g;
  const bool col_ok = c16 < g;

  // q and dO fragments (B operands of S^T and dP^T): head c16, dims kb*32 + q4*8 + 0..7
  const int hq = h * g + (col_ok ? c16 : 0);
  const uint16_t* qh = static_cast<const uint16_t*>(p.q) + bb * p.q_sb + i * p.q_sn + static_cast<int64_t>(hq) * p.q_sh;
  const uint16_t* dh = static_cast<const uint16_t*>(p.dout) + bb * p.do_sb + i * p.do_sn + static_cast<int64_t>(hq) * p.do_sh;
  bf16x8_t qf[KB], df[KB];
  // o of head hq at the same dims, in 16-byte loads that all go out before
  // the first use (one branch on o's type around all of them)
  float ov[KB][8];
  {
    const int64_t oo = bb * p.o_sb + i * p.o_sn + static_cast<int64_t>(hq) * p.o_sh + q4 * 8;
    if (p.o_bf16) {
      const uint16_t* ob = static_cast<const uint16_t*>(p.o) + oo;
      uint4 w[KB];
#pragma unroll
      for (int kb = 0; kb < KB; ++kb) w[kb] = col_ok ? *reinterpret_cast<const uint4*>(ob + kb * 32) : make_uint4(0u, 0u, 0u, 0u);
#pragma unroll
      for (int kb = 0; kb < KB; ++kb) {
        const uint32_t ww[4] = {w[kb].x, w[kb].y, w[kb].z, w[kb].w};
#pragma unroll
        for (int e = 0; e < 8; ++e) ov[kb][e] = __uint_as_float((e & 1) ? (ww[e >> 1] & 0xFFFF0000u) : (ww[e >> 1] << 16));
      }
    } else {
      const float* of = static_cast<const float*>(p.o) + oo;
      float4 w[KB][2];
#pragma unroll
      for (int kb = 0; kb < KB; ++kb)
#pragma unroll
        for (int x = 0; x < 2; ++x)
          w[kb][x] = col_ok ? *reinterpret_cast<const float4*>(of + kb * 32 + 4 * x) : make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
      for (int kb = 0; kb < KB; ++kb) {
        ov[kb][0] = w[kb][0].x, ov[kb][1] = w[kb][0].y, ov[kb][2] = w[kb][0].z, ov[kb][3] = w[kb][0].w;
        ov[kb][4] = w[kb][1].x, ov[kb][5] = w[kb][1].y, ov[kb][6] = w[kb][1].z, ov[kb][7] = w[kb][1].w;
      }
    }
  }
  float dpart = 0.0f;  // this lane's share of D = dO . o for head c16
#pragma unroll
  for (int kb = 0; kb < KB; ++kb) {
    qf[kb] = col_ok ? *reinterpret_cast<const bf16x8_t*>(qh + kb * 32 + q4 * 8) : bf16x8_t{};
    df[kb] = col_ok ? *reinterpret_cast<const bf16x8_t*>(dh + kb * 32 + q4 * 8) : bf16x8_t{};
    const uint4 qu = __builtin_bit_cast(uint4, qf[kb]), du = __builtin_bit_cast(uint4, df[kb]);
    const uint32_t qw[4] = {qu.x, qu.y, qu.z, qu.w}, dw[4] = {du.x, du.y, du.z, du.w};
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const int dim = kb * 32 + q4 * 8 + e;
      const uint16_t qv = static_cast<uint16_t>((e & 1) ? (qw[e >> 1] >> 16) : (qw[e >> 1] & 0xFFFFu));
      const uint16_t dv = static_cast<uint16_t>((e & 1) ? (dw[e >> 1] >> 16) : (dw[e >> 1] & 0xFFFFu));
      if (col_ok) dpart = fma_rn(bf16_bits_to_f32(dv), ov[kb][e], dpart);
      if (DKDV && c16 < 8) {  // head slots 0..7 of the [dim][head] copies (zero past g)
        hd_lds[DKDV ? wave : 0][0][dim][c16] = col_ok ? qv : static_cast<uint16_t>(0);
        hd_lds[DKDV ? wave : 0][1][dim][c16] = col_ok ? dv : static_cast<uint16_t>(0);
      }
    }
  }
  dpart += __shfl_xor(dpart, 16);
  dpart += __shfl_xor(dpart, 32);
  const float dcol = dpart;  // D of head c16 (lanes of column c16)

  const uint16_t* kbase = static_cast<const uint16_t*>(p.k) + bb * p.k_sb + static_cast<int64_t>(h) * p.k_sh;
  const uint16_t* vbase = static_cast<const uint16_t*>(p.v) + bb * p.v_sb + static_cast<int64_t>(h) * p.v_sh;
  const unsigned char* ib = static_cast<const unsigned char*>(p.idx) +
                            (bb * p.idx_sb + i * p.idx_sn + h * p.idx_sh) * (p.idx_i64 ? 8 : 4);
  unsigned char* kl = kv_lds[wave][0];
  unsigned char* vl = kv_lds[wave][1];
  const uint32_t ksn2 = 2u * static_cast<uint32_t>(p.k_sn), vsn2 = 2u * static_cast<uint32_t>(p.v_sn);
  const int kbytes = static_cast<int>((p.n - 1) * p.k_sn * 2 + 2 * D);
  const int vbytes = static_cast<int>((p.n - 1) * p.v_sn * 2 + 2 * D);
  const __amdgpu_buffer_rsrc_t krs = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(kbase), 0, kbytes, kBufferWord3);
  const __amdgpu_buffer_rsrc_t vrs = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(vbase), 0, vbytes, kBufferWord3);
  uint32_t seg16[S::SWZ_PERIOD];
  row_seg16<D>(lane, seg16);
  const int kswz = mf_swz<D>(c16);
  // key of chunk slot `lane` (lanes < 32), -1 past top_k, -2 out of range (flagged)
  // (loading and checking apart: a batch of loads goes out before a check waits)
  // (two dword loads with no branch on the index type: the low word, and the
  // high word or, for int32 entries, the same word again)
  auto slot_at = [&](int ch, int l) { return l < kMfChunk && ch * kMfChunk + l < p.top_k; };
  const int ewords = p.idx_i64 ? 2 : 1;
  auto raw_at = [&](int ch, int l) -> uint64_t {
    const int slot = slot_at(ch, l) ? ch * kMfChunk + l : 0;
    const uint32_t* w = reinterpret_cast<const uint32_t*>(ib) + slot * ewords;
    return (static_cast<uint64_t>(w[ewords - 1]) << 32) | w[0];
  };
  auto key_at = [&](int ch, int l, uint64_t raw) -> int {
    if (!slot_at(ch, l)) return -1;
    const int64_t j = p.idx_i64 ? static_cast<int64_t>(raw)
                                : static_cast<int64_t>(static_cast<int32_t>(static_cast<uint32_t>(raw)));
    if (j < 0 || j >= p.n) {
      if (p.err) p.err[0] = 1;
      return -2;
    }
    return static_cast<int>(j);
  };
  auto load_idx = [&](int ch) { return key_at(ch, lane, raw_at(ch, lane)); };
  auto chunk_ok = [&](int j) { return j >= 0 && !(p.causal && j > i); };
  auto read_k = [&](const unsigned char* l, bf16x8_t (&f)[2][KB]) {
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int kb = 0; kb < KB; ++kb)
        f[t][kb] = *(lds_bf16x8_ptr)(l + (16 * t + c16) * S::ROW + (((kb * 4 + q4) ^ kswz) << 4));
  };
  // valid bit of the lane's score x = 4t + e (key slot 16t + 4 q4 + e)
  auto valid = [&](uint64_t okb, int x) { return ((okb >> (4 * q4 + 16 * (x >> 2) + (x & 3))) & 1ull) != 0; };
  const int nchunks = (p.top_k + kMfChunk - 1) / kMfChunk;

  // ---- pass 1: running max (log2 domain) and sum per head over the row's
  // slots, unless the forward left them (a NaN entry: it did not)
  float m_run = -INFINITY, l_run = 0.0f;
  const float* fst = p.stats_in ? p.stats_in + (bh * p.n + i) * g * 2 : nullptr;
  const bool have_st = fst != nullptr && !__builtin_isnan(fst[0]);
  if (!have_st) {
    const int j0 = nchunks > 0 ? load_idx(0) : -1;
    uint64_t okn = __ballot(chunk_ok(j0));
    if (nchunks > 0) row_issue<D>(krs, kl, chunk_ok(j0) ? j0 : -1, lane, ksn2, seg16);
    uint64_t jn_raw = nchunks > 1 ? raw_at(1, lane) : 0;  // checked after the next wait
    for (int ch = 0; ch < nchunks; ++ch) {
      __builtin_amdgcn_s_waitcnt(kWaitVm0);
      bf16x8_t kf[2][KB];
      read_k(kl, kf);
      __builtin_amdgcn_s_waitcnt(kWaitLgkm0);
      const uint64_t okb = okn;
      if (ch + 1 < nchunks) {
        const int jn = key_at(ch + 1, lane, jn_raw);
        okn = __ballot(chunk_ok(jn));
        row_issue<D>(krs, kl, chunk_ok(jn) ? jn : -1, lane, ksn2, seg16);
        if (ch + 2 < nchunks) jn_raw = raw_at(ch + 2, lane);
      }
      float sc[8];
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        floatx4_t sv = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int kb = 0; kb < KB; ++kb) sv = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kf[t][kb], qf[kb], sv, 0, 0, 0);
#pragma unroll
        for (int e = 0; e < 4; ++e) sc[4 * t + e] = valid(okb, 4 * t + e) ? sv[e] * p.qk_scale_log2 : -INFINITY;
      }
      float mx = sc[0];
#pragma unroll
      for (int x = 1; x < 8; ++x) mx = fmaxf(mx, sc[x]);
      mx = fmaxf(mx, __shfl_xor(mx, 16));
      mx = fmaxf(mx, __shfl_xor(mx, 32));
      const float mnew = fmaxf(m_run, mx);
      const float mref = (mnew == -INFINITY) ? 0.0f : mnew;
      float ps = 0.0f;
#pragma unroll
      for (int x = 0; x < 8; ++x) ps += exp2f(sc[x] - mref);
      l_run = l_run * exp2f(m_run - mref) + ps;
      m_run = mnew;
    }
  }
  float l_tot = l_run + __shfl_xor(l_run, 16);
  l_tot += __shfl_xor(l_tot, 32);
  float inv_l = (l_tot > 0.0f && col_ok) ? 1.0f / l_tot : 0.0f;  // 0: no slot, or an unused column
  float mref = (m_run == -INFINITY) ? 0.0f : m_run;
  if (have_st) {
    mref = col_ok ? fst[2 * c16] : 0.0f;
    inv_l = col_ok ? fst[2 * c16 + 1] : 0.0f;
  }
  // the prefix keys [0, X) go to prefix_attention_bwd_kernel, which needs the
  // row's softmax reference, 1/sum and D
  const int xpre = p.pfx ? min(max(p.pfx[bh * p.n + i], 0),
                               static_cast<int>(min(static_cast<int64_t>(p.top_k), p.n)))
                         : 0;
  if (p.pfx && q4 == 0 && col_ok) {
    float* ps = p.pstats + ((bh * p.n + i) * g + c16) * 4;
    ps[0] = mref;
    ps[1] = inv_l;
    ps[2] = dcol;
  }
  auto chunk_ok2 = [&](int j) { return j >= xpre && chunk_ok(j); };
  const bool row_dkdv = !p.rowmap || p.rowmap[bh * p.n + i] == -1;

  // ---- pass 2
  const bool hi_row = c16 < g;
  const bool lo_row = c16 >= 8 && c16 < 8 + g;
  floatx4_t dqacc[NT];
#pragma unroll
  for (int t = 0; t < NT; ++t) dqacc[t] = floatx4_t{0.f, 0.f, 0.f, 0.f};
  float* dkb = p.dk + (bb * p.n * p.h_kv + h) * p.d;
  float* dvb = p.dv + (bb * p.n * p.h_kv + h) * p.d;
  const int64_t krow = static_cast<int64_t>(p.h_kv) * p.d;
  float* tr = &tr_lds[DKDV ? wave : 0][0][0];
  // A operand over heads from the [key][head] copy: k = 0..7 bf16 hi of heads
  // 0..7 (lanes q4 = 0), 8..15 their lo (q4 = 1), 16..31 zero
  auto heads_operand = [&](int t) -> bf16x8_t {
    if (q4 >= 2) return bf16x8_t{};
    const float4 a = *reinterpret_cast<const float4*>(tr + (16 * t + c16) * 16);
    const float4 b = *reinterpret_cast<const float4*>(tr + (16 * t + c16) * 16 + 4);
    const float v[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
    uint32_t w[4];
#pragma unroll
    for (int x = 0; x < 4; ++x) {
      const uint32_t hi = pack_bf16x2(v[2 * x], v[2 * x + 1]);
      const uint32_t lo = pack_bf16x2(v[2 * x] - __uint_as_float(hi << 16), v[2 * x + 1] - __uint_as_float(hi & 0xFFFF0000u));
      w[x] = q4 == 0 ? hi : lo;
    }
    return __builtin_bit_cast(bf16x8_t, make_uint4(w[0], w[1], w[2], w[3]));
  };
  // B operand by head from the [dim][head] copy of Q (which = 0) or dO (1):
  // k = 8 q4 + e holds head e for q4 < 2 (hi and lo rows of A meet the same
  // head row), zero for q4 >= 2; column c16 = dim 16 dt + c16
  auto head_rows = [&](int which, int dt) -> bf16x8_t {
    if (q4 >= 2) return bf16x8_t{};
    return *reinterpret_cast<const bf16x8_t*>(&hd_lds[DKDV ? wave : 0][which][16 * dt + c16][0]);
  };
  // only the chunks with a slot to differentiate (a chunk without one adds
  // nothing to dQ, dK or dV)
  // The next live chunk's index entries (jn_raw, for chunk un) fly with the
  // current chunk's gathers and are checked after the wait those need anyway.
  LiveChunks lc;
  if (xpre > 0) lc.build(nchunks, lane, raw_at, key_at, chunk_ok2);
  else lc.all_live(nchunks);
  int u = lc.next(-1);
  int un = nchunks;
  int jc = -1;
  uint64_t jn_raw = 0;
  uint64_t okn = 0;
  if (u < nchunks) {
    jc = lc.get(u, lane, load_idx);
    okn = __ballot(chunk_ok2(jc));
    row_issue<D>(krs, kl, chunk_ok2(jc) ? jc : -1, lane, ksn2, seg16);
    row_issue<D>(vrs, vl, chunk_ok2(jc) ? jc : -1, lane, vsn2, seg16);
    un = lc.next(u);
    if (un < nchunks) jn_raw = raw_at(un, lane);
  }
  while (u < nchunks) {
    __builtin_amdgcn_s_waitcnt(kWaitVm0);
    bf16x8_t kf[2][KB], vf[2][KB], kt[NT];
    read_k(kl, kf);
    read_k(vl, vf);
#pragma unroll
    for (int t = 0; t < NT; ++t) kt[t] = rows_transposed<D>(kl, t, q4, c16);
    __builtin_amdgcn_s_waitcnt(kWaitLgkm0);
    const uint64_t okb = okn;
    const int jcur = jc;
    u = un;
    if (u < nchunks) {
      const int jn = key_at(u, lane, jn_raw);
      okn = __ballot(chunk_ok2(jn));
      row_issue<D>(krs, kl, chunk_ok2(jn) ? jn : -1, lane, ksn2, seg16);
      row_issue<D>(vrs, vl, chunk_ok2(jn) ? jn : -1, lane, vsn2, seg16);
      jc = jn;
      un = lc.next(u);
      if (un < nchunks) jn_raw = raw_at(un, lane);
    }
    float pr[8], ds[8];
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      floatx4_t sv = {0.f, 0.f, 0.f, 0.f}, dv = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int kb = 0; kb < KB; ++kb) {
        sv = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kf[t][kb], qf[kb], sv, 0, 0, 0);
        dv = __builtin_amdgcn_mfma_f32_16x16x32_bf16(vf[t][kb], df[kb], dv, 0, 0, 0);
      }
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int x = 4 * t + e;
        pr[x] = valid(okb, x) ? exp2f(sv[e] * p.qk_scale_log2 - mref) * inv_l : 0.0f;
        ds[x] = pr[x] * (dv[e] - dcol);
      }
    }
    // dQ^T += K^T dS^T (B: rows c16 < g dS_hi of head c16, rows 8 + r dS_lo of head r)
    uint32_t db[4];
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      const uint32_t hi = pack_bf16x2(ds[2 * w], ds[2 * w + 1]);
      const uint32_t lo = pack_bf16x2(ds[2 * w] - __uint_as_float(hi << 16), ds[2 * w + 1] - __uint_as_float(hi & 0xFFFF0000u));
      const uint32_t lo_in = dpp_from_minus8(lo);
      db[w] = hi_row ? hi : (lo_row ? lo_in : 0u);
    }
    const bf16x8_t dsb = __builtin_bit_cast(bf16x8_t, make_uint4(db[0], db[1], db[2], db[3]));
#pragma unroll
    for (int t = 0; t < NT; ++t) dqacc[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kt[t], dsb, dqacc[t], 0, 0, 0);

    // dV and dK tiles; P then dS pass through tr as [key][head]
    if (!DKDV || !row_dkdv) continue;
#pragma unroll
    for (int pass = 0; pass < 2; ++pass) {
      const float* src = pass == 0 ? pr : ds;
#pragma unroll
      for (int x = 0; x < 8; ++x) tr[(16 * (x >> 2) + 4 * q4 + (x & 3)) * 16 + c16] = src[x];
      __builtin_amdgcn_s_waitcnt(kWaitLgkm0);
      __builtin_amdgcn_wave_barrier();
      const bf16x8_t a0 = heads_operand(0), a1 = heads_operand(1);
      __builtin_amdgcn_s_waitcnt(kWaitLgkm0);
      __builtin_amdgcn_wave_barrier();  // tr is rewritten by the next pass
      float* dst = pass == 0 ? dvb : dkb;
      const float mul = pass == 0 ? 1.0f : p.inv_scale;
      const int which = pass == 0 ? 1 : 0;  // P^T dO, then dS^T Q
#pragma unroll
      for (int dt = 0; dt < NT; ++dt) {
        const bf16x8_t bop = head_rows(which, dt);
#pragma unroll
        for (int t = 0; t < 2; ++t) {
          const floatx4_t c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(t == 0 ? a0 : a1, bop, floatx4_t{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const int slot = 16 * t + 4 * q4 + e;
            const int j = __shfl(jcur, slot);
            if ((okb >> slot) & 1ull) unsafeAtomicAdd(dst + j * krow + 16 * dt + c16, c[e] * mul);
          }
        }
      }
    }
  }

  // dQ: hi row + lo row, / scale; lanes c16 < g hold dims 16t + 4 q4 + e of head c16
#pragma unroll
  for (int t = 0; t < NT; ++t)
#pragma unroll
    for (int e = 0; e < 4; ++e) dqacc[t][e] += dpp_from_plus8(dqacc[t][e]);
  if (!hi_row) return;
  float* dqb = p.dq + ((bb * p.n + i) * p.h_q + h * g + c16) * p.d + 4 * q4;
#pragma unroll
  for (int t = 0; t < NT; ++t)
    *reinterpret_cast<float4*>(dqb + 16 * t) =
        make_float4(dqacc[t][0] * p.inv_scale, dqacc[t][1] * p.inv_scale, dqacc[t][2] * p.inv_scale,
                    dqacc[t][3] * p.inv_scale);
}

// ---------------------------------------------------------------------------
// Dense key prefixes (after the matrix-core row kernel, which skipped them):
// one block per kPbWaves neighbouring rows of one (batch, kv head), wave w
// taking row r0 + w.  The keys [0, max X) stream through LDS in 32-key chunks
// (loads shared by the block); per chunk each wave forms its row's p and ds
// with the row kernel's MFMA layout and the stats the row kernel left
// (softmax reference, 1/sum, D), masked to keys below its X (and its position
// when causal), and adds dQ^T += K^T dS^T in registers.  P and dS of all the
// block's query vectors then meet in LDS as [key][query vector], and
// dV = P^T dO, dK = dS^T Q come from MFMAs that sum over the block's query
// vectors (A = P^T or dS^T split into bf16 hi and lo, B = dO or Q as
// [dim][query vector] in LDS): one fp32 atomic per (key, dim) and block instead
// of one per row.
constexpr int kPbWaves = 8;

// Rows per wave: the dq-only build packs 8 / g rows into a wave's 8 query
// vector columns (column c: row c / g, head c % g; the low parts of dS then
// fill columns 8 .. 15), so the block's K/V chunks and each MFMA serve 8 / g
// rows instead of one; the full build keeps one row per wave.
__host__ __device__ inline int pb_rows_per_wave(int g, bool dq) { return dq && g < 8 ? 8 / g : 1; }

// DQ: dq only (the bucket kernel's prefix mode adds dk and dv): 4 waves per
// block and no [key][query vector] staging, for 4 blocks per CU (at most 128
// registers at d = 128, a few of them in scratch).
template <int D, bool DQ>
__global__ __launch_bounds__(64 * (DQ ? 4 : kPbWaves)) __attribute__((amdgpu_waves_per_eu(DQ ? 4 : 1, 8))) void
prefix_attention_bwd_kernel(BwdParams p) {
  using S = MfShape<D>;
  constexpr int KB = S::KB, NT = S::NT;
  constexpr int W = DQ ? 4 : kPbWaves;  // rows (waves) per block
  constexpr int QV = DQ ? 1 : 8 * W;    // query vectors per block at most (g <= 8)
  constexpr int LPW = (S::NLD + W - 1) / W;  // chunk loads per wave and tensor
  __shared__ __align__(16) unsigned char kv[2][2][kMfChunk * S::ROW];  // [buffer][K, V]
  __shared__ __align__(16) float pall[2][kMfChunk][QV];                // P, dS as [key][qv]
  __shared__ __align__(16) uint16_t qall[2][DQ ? 1 : D][QV];           // Q, dO as [dim][qv] (bf16)
  __shared__ int s_xmax;

  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int tid = threadIdx.x, lane = tid & 63;
  const int q4 = lane >> 4, c16 = lane & 15;
  const int g = p.g;
  const int rpw = pb_rows_per_wave(g, DQ);  // rows per wave
  const int qvw = rpw * g;                  // query vector columns per wave (<= 8)
  const int64_t tiles = ceil_div(p.n, static_cast<int64_t>(W) * rpw);
  const int64_t nblk = (p.rows / p.n) * tiles;
  const int64_t blk = xcd_block(blockIdx.x, xcd_per(nblk));
  if (blk >= nblk) return;
  const int64_t bh = blk / tiles;
  const bool col_ok = c16 < qvw;
  const int rr = col_ok ? c16 / g : 0, hh = col_ok ? c16 - rr * g : 0;  // this column's row in the wave, head
  const int64_t i = ((blk - bh * tiles) * W + wave) * rpw + rr;  // this column's row
  const bool row_ok = i < p.n;
  const int h = static_cast<int>(bh % p.h_kv);
  const int64_t bb = bh / p.h_kv;
  const int xcap = static_cast<int>(min(static_cast<int64_t>(p.top_k), p.n));
  const int xrow = (row_ok && col_ok) ? min(max(p.pfx[bh * p.n + i], 0), xcap) : 0;

  // the block's Q and dO as [dim][qv], zero for unused query vectors (whose P
  // and dS columns stay zero too: the reductions run over whole 32-column blocks)
  if (!DQ) {
    for (int e = tid; e < 2 * D * QV; e += 64 * W) reinterpret_cast<uint16_t*>(qall)[e] = 0;
    for (int e = tid; e < 2 * kMfChunk * QV; e += 64 * W) reinterpret_cast<float*>(pall)[e] = 0.0f;
  }
  if (tid == 0) s_xmax = 0;
  __syncthreads();
  {
    int xm = xrow;  // the wave's largest X (lanes 0..15 cover its columns)
#pragma unroll
    for (int o = 1; o < 16; o <<= 1) xm = max(xm, __shfl_xor(xm, o));
    if (lane == 0) atomicMax(&s_xmax, xm);
  }
  const int hq = h * g + hh;
  const uint16_t* qh = static_cast<const uint16_t*>(p.q) + bb * p.q_sb + (row_ok ? i : 0) * p.q_sn +
                       static_cast<int64_t>(hq) * p.q_sh;
  const uint16_t* dh = static_cast<const uint16_t*>(p.dout) + bb * p.do_sb + (row_ok ? i : 0) * p.do_sn +
                       static_cast<int64_t>(hq) * p.do_sh;
  bf16x8_t qf[KB], df[KB];
  const bool have = row_ok && col_ok && xrow > 0;
#pragma unroll
  for (int kb = 0; kb < KB; ++kb) {
    qf[kb] = have ? *reinterpret_cast<const bf16x8_t*>(qh + kb * 32 + q4 * 8) : bf16x8_t{};
    df[kb] = have ? *reinterpret_cast<const bf16x8_t*>(dh + kb * 32 + q4 * 8) : bf16x8_t{};
    if (have) {
      const uint4 qu = __builtin_bit_cast(uint4, qf[kb]), du = __builtin_bit_cast(uint4, df[kb]);
      const uint32_t qw[4] = {qu.x, qu.y, qu.z, qu.w}, dw[4] = {du.x, du.y, du.z, du.w};
#pragma unroll
      for (int e = 0; e < 8 && !DQ; ++e) {
        const int dim = kb * 32 + q4 * 8 + e;
        qall[0][DQ ? 0 : dim][DQ ? 0 : wave * g + c16] =
            static_cast<uint16_t>((e & 1) ? (qw[e >> 1] >> 16) : (qw[e >> 1] & 0xFFFFu));
        qall[1][DQ ? 0 : dim][DQ ? 0 : wave * g + c16] =
            static_cast<uint16_t>((e & 1) ? (dw[e >> 1] >> 16) : (dw[e >> 1] & 0xFFFFu));
      }
    }
  }
  float mref = 0.0f, inv_l = 0.0f, dcol = 0.0f;
  if (have) {
    const float* ps = p.pstats + ((bh * p.n + i) * g + hh) * 4;
    mref = ps[0];
    inv_l = ps[1];
    dcol = ps[2];
  }
  __syncthreads();
  const int xmax = s_xmax;
  if (xmax == 0) return;

  const uint16_t* kbase = static_cast<const uint16_t*>(p.k) + bb * p.k_sb + static_cast<int64_t>(h) * p.k_sh;
  const uint16_t* vbase = static_cast<const uint16_t*>(p.v) + bb * p.v_sb + static_cast<int64_t>(h) * p.v_sh;
  const uint32_t ksn2 = 2u * static_cast<uint32_t>(p.k_sn), vsn2 = 2u * static_cast<uint32_t>(p.v_sn);
  const int kbytes = static_cast<int>((p.n - 1) * p.k_sn * 2 + 2 * D);
  const int vbytes = static_cast<int>((p.n - 1) * p.v_sn * 2 + 2 * D);
  const __amdgpu_buffer_rsrc_t krs = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(kbase), 0, kbytes, kBufferWord3);
  const __amdgpu_buffer_rsrc_t vrs = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(vbase), 0, vbytes, kBufferWord3);
  uint32_t seg16[S::SWZ_PERIOD];
  row_seg16<D>(lane, seg16);
  const int kswz = mf_swz<D>(c16);
  // this wave's loads of chunk ch: loads r = wave + W * t (< NLD) of K and V
  auto issue = [&](int ch) {
#pragma unroll
    for (int t = 0; t < LPW; ++t) {
      const int r = wave + W * t;
      if (r < S::NLD) {
        const int j = ch * kMfChunk + S::KPI * r + lane / S::SEGS;
        const uint32_t sg = seg16[r % S::SWZ_PERIOD];
        const uint32_t ko = j < xmax ? __umul24(static_cast<uint32_t>(j), ksn2) + sg : kOobOffset;
        const uint32_t vo = j < xmax ? __umul24(static_cast<uint32_t>(j), vsn2) + sg : kOobOffset;
        __builtin_amdgcn_raw_ptr_buffer_load_lds(krs, (lds_void_ptr)(kv[ch & 1][0] + r * 1024), 16, static_cast<int>(ko), 0, 0, 0);
        __builtin_amdgcn_raw_ptr_buffer_load_lds(vrs, (lds_void_ptr)(kv[ch & 1][1] + r * 1024), 16, static_cast<int>(vo), 0, 0, 0);
      }
    }
  };
  const int ilim = p.causal ? static_cast<int>(min(i, static_cast<int64_t>(0x7FFFFFFF))) : 0x7FFFFFFF;
  const bool hi_row = c16 < qvw;
  const bool lo_row = c16 >= 8 && c16 < 8 + qvw;
  floatx4_t dqacc[NT];
#pragma unroll
  for (int t = 0; t < NT; ++t) dqacc[t] = floatx4_t{0.f, 0.f, 0.f, 0.f};
  float* dkb = p.dk + (bb * p.n * p.h_kv + h) * p.d;
  float* dvb = p.dv + (bb * p.n * p.h_kv + h) * p.d;
  const int64_t krow = static_cast<int64_t>(p.h_kv) * p.d;
  const int nqv = W * g;
  const int kblocks = (nqv + 31) / 32;
  const int nch = (xmax + kMfChunk - 1) / kMfChunk;
  issue(0);
  for (int u = 0; u < nch; ++u) {
    __builtin_amdgcn_s_waitcnt(kWaitVm0);
    // chunk u is in LDS for every wave; every wave is done with chunk u - 1 and pall
    __syncthreads();
    if (u + 1 < nch) issue(u + 1);
    const unsigned char* kl = kv[u & 1][0];
    const unsigned char* vl = kv[u & 1][1];
    bf16x8_t kf[2][KB], vf[2][KB], kt[NT];
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int kb = 0; kb < KB; ++kb) {
        kf[t][kb] = *(lds_bf16x8_ptr)(kl + (16 * t + c16) * S::ROW + (((kb * 4 + q4) ^ kswz) << 4));
        vf[t][kb] = *(lds_bf16x8_ptr)(vl + (16 * t + c16) * S::ROW + (((kb * 4 + q4) ^ kswz) << 4));
      }
#pragma unroll
    for (int t = 0; t < NT; ++t) kt[t] = rows_transposed<D>(kl, t, q4, c16);
    float pr[8], ds[8];
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      floatx4_t sv = {0.f, 0.f, 0.f, 0.f}, dv = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int kb = 0; kb < KB; ++kb) {
        sv = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kf[t][kb], qf[kb], sv, 0, 0, 0);
        dv = __builtin_amdgcn_mfma_f32_16x16x32_bf16(vf[t][kb], df[kb], dv, 0, 0, 0);
      }
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int x = 4 * t + e;
        const int j = u * kMfChunk + 16 * t + 4 * q4 + e;
        const bool ok = have && j < xrow && j <= ilim;
        pr[x] = ok ? exp2f(sv[e] * p.qk_scale_log2 - mref) * inv_l : 0.0f;
        ds[x] = pr[x] * (dv[e] - dcol);
      }
    }
    // dQ^T += K^T dS^T (B: rows c16 < g dS_hi of head c16, rows 8 + r dS_lo of head r)
    uint32_t db[4];
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      const uint32_t hi = pack_bf16x2(ds[2 * w], ds[2 * w + 1]);
      const uint32_t lo = pack_bf16x2(ds[2 * w] - __uint_as_float(hi << 16), ds[2 * w + 1] - __uint_as_float(hi & 0xFFFF0000u));
      const uint32_t lo_in = dpp_from_minus8(lo);
      db[w] = hi_row ? hi : (lo_row ? lo_in : 0u);
    }
    const bf16x8_t dsb = __builtin_bit_cast(bf16x8_t, make_uint4(db[0], db[1], db[2], db[3]));
#pragma unroll
    for (int t = 0; t < NT; ++t) dqacc[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kt[t], dsb, dqacc[t], 0, 0, 0);
    if (DQ) continue;
    // P and dS of this row's heads into [key][qv]
    if (col_ok) {
#pragma unroll
      for (int x = 0; x < 8; ++x) {
        const int key = 16 * (x >> 2) + 4 * q4 + (x & 3);
        pall[0][key][DQ ? 0 : wave * g + c16] = pr[x];
        pall[1][key][DQ ? 0 : wave * g + c16] = ds[x];
      }
    }
    __syncthreads();
    // dV = P^T dO (pass 0) and dK = dS^T Q (pass 1), summed over the block's
    // query vectors: item (pass, dt) by wave item % W
    for (int item = wave; item < 2 * NT; item += W) {
      const int pass = item / NT, dt = item - pass * NT;
      const int which = pass == 0 ? 1 : 0;  // B: dO for dV, Q for dK
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        floatx4_t c = {0.f, 0.f, 0.f, 0.f};
        for (int kq = 0; kq < kblocks; ++kq) {
          const float* src = &pall[pass][16 * t + c16][DQ ? 0 : 32 * kq + 8 * q4];
          const float4 a = *reinterpret_cast<const float4*>(src);
          const float4 b = *reinterpret_cast<const float4*>(src + 4);
          const float v[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
          uint32_t hw[4], lw[4];
#pragma unroll
          for (int x = 0; x < 4; ++x) {
            hw[x] = pack_bf16x2(v[2 * x], v[2 * x + 1]);
            lw[x] = pack_bf16x2(v[2 * x] - __uint_as_float(hw[x] << 16), v[2 * x + 1] - __uint_as_float(hw[x] & 0xFFFF0000u));
          }
          const bf16x8_t ah = __builtin_bit_cast(bf16x8_t, make_uint4(hw[0], hw[1], hw[2], hw[3]));
          const bf16x8_t al = __builtin_bit_cast(bf16x8_t, make_uint4(lw[0], lw[1], lw[2], lw[3]));
          const bf16x8_t bop =
              *reinterpret_cast<const bf16x8_t*>(&qall[which][DQ ? 0 : 16 * dt + c16][DQ ? 0 : 32 * kq + 8 * q4]);
          c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ah, bop, c, 0, 0, 0);
          c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(al, bop, c, 0, 0, 0);
        }
        float* dst = pass == 0 ? dvb : dkb;
        const float mul = pass == 0 ? 1.0f : p.inv_scale;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int j = u * kMfChunk + 16 * t + 4 * q4 + e;
          if (j < xmax) unsafeAtomicAdd(dst + j * krow + 16 * dt + c16, c[e] * mul);
        }
      }
    }
  }
  // dQ of the prefix: hi row + lo row, / scale, added to the row kernel's part
#pragma unroll
  for (int t = 0; t < NT; ++t)
#pragma unroll
    for (int e = 0; e < 4; ++e) dqacc[t][e] += dpp_from_plus8(dqacc[t][e]);
  if (!have || !hi_row) return;
  float* dqb = p.dq + ((bb * p.n + i) * p.h_q + h * g + hh) * p.d + 4 * q4;
#pragma unroll
  for (int t = 0; t < NT; ++t) {
    float4 cur = *reinterpret_cast<float4*>(dqb + 16 * t);
    cur.x += dqacc[t][0] * p.inv_scale;
    cur.y += dqacc[t][1] * p.inv_scale;
    cur.z += dqacc[t][2] * p.inv_scale;
    cur.w += dqacc[t][3] * p.inv_scale;
    *reinterpret_cast<float4*>(dqb + 16 * t) = cur;
  }
}

// ---------------------------------------------------------------------------
// Bucket mode: dk and dv of the candidate slots, by codebook bucket.
//
// A row's candidates are the keys that share one of its a query codes (inside
// the routing window), so the (query row, candidate key) pairs of one kv head
// are the union over buckets c of R_c x K_c: R_c the rows holding code c (an
// index of q_codes built like stage (b)'s) and K_c the keys holding it (stage
// (b)'s index).  A pair sharing several codes counts in the bucket of the
// smallest shared code.  The pairs a row selected, at or above its dense
// prefix X, are
//   * for a row with filler (X > 0): every candidate at or above X;
//   * for a row without filler (X = 0: at least top_k candidates): the ones
//     its indices hold, read from a per-row key bitmap (bucket_rowmap_kernel);
//     rows past the bitmap capacity keep the row kernel's atomics.
// One block per (bucket, 32-key chunk) "item": K and V of the chunk stay in
// LDS while the bucket's rows stream through in chunks of 16 query vectors
// (row, head), staged one chunk ahead.  Wave w takes keys 16 (w & 1) ... + 15
// and dims (w >> 1) D/2 ... + D/2 - 1: S = Q K^T and dP = dO V^T on the matrix
// cores (A = the query vectors' Q / dO rows, B = the chunk's K / V rows),
// p = exp2(s - m) / l and ds = p (dP - D) from the row kernel's stats, and
// dV^T += dO^T P, dK^T += Q^T dS in registers (B = P or dS split into bf16 hi
// and lo, k = 8 q4 + e <-> query vector 4 q4 + (e & 3); A = dO^T or Q^T from
// transposing LDS reads of the staged rows, the same four query vectors
// twice).  One fp32 atomic per (key, dim) and item at the end.  Every LDS read
// of a chunk precedes the next chunk's LDS-bound loads, so no read waits for
// them.
constexpr int kBkKeys = 32;    // keys per item
constexpr int kBkQv = 16;      // query vectors per row chunk
constexpr int kBkMaxA = 32;    // query codes per row (bucket mode)
constexpr int kBkMaxB = 8;     // key codes per key (bucket mode)
constexpr int kBkHash = 512;   // LDS hash of the item's codes below c (at most 32 x 7)
constexpr int kBkThreads = 256;

struct BucketParams {
  const int32_t* kpost;   // [bh][n * b] key index postings
  const int32_t* kcodes;  // [bh][n][b]
  const int4* desc;       // [bh][max_items] (bucket_desc_kernel)
  const int2* meta;       // [bh][n * a]: (row position, w) per query posting, w as bucket_meta_kernel
  const int32_t* qcodes;  // [bh][n][a]
  const uint32_t* bits;   // [capacity][words]: key bitmaps of rows without filler
  int64_t words, max_items;
  int a, b, gp_log2, router_causal;
};

// items[bh][c] = sum over c' < c of ceil(|K_c'| / kBkKeys); one block per bh.
__global__ __launch_bounds__(1024) void bucket_items_kernel(const int32_t* __restrict__ koff, int n_c,
                                                            int32_t* __restrict__ items) {
  __shared__ int32_t wsum[16];
  __shared__ int32_t carry;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int32_t* o = koff + static_cast<int64_t>(blockIdx.x) * (n_c + 1);
  int32_t* it = items + static_cast<int64_t>(blockIdx.x) * (n_c + 1);
  if (tid == 0) carry = 0;
  __syncthreads();
  for (int base = 0; base < n_c; base += 1024) {
    const int c = base + tid;
    const int cnt = c < n_c ? (o[c + 1] - o[c] + kBkKeys - 1) / kBkKeys : 0;
    int x = cnt;
#pragma unroll
    for (int s = 1; s < 64; s <<= 1) {
      const int y = __shfl_up(x, s);
      if (lane >= s) x += y;
    }
    if (lane == 63) wsum[wave] = x;
    __syncthreads();
    if (tid == 0) {
      int run = carry;
      for (int w = 0; w < 16; ++w) {
        const int t = wsum[w];
        wsum[w] = run;
        run += t;
      }
      carry = run;
    }
    __syncthreads();
    if (c < n_c) it[c] = wsum[wave] + x - cnt;
    __syncthreads();
  }
  if (tid == 0) it[n_c] = carry;
}

// Per item slot of (bh, max_items): int4 (c | nk << 16, k0, rs, r1) -- the
// bucket, its postings k0 .. k0 + nk - 1, and its rows rs .. r1 - 1 in the
// query index (rows below the chunk's lowest key dropped when a mask is
// causal) -- or c = -1 past the bh's items.
__global__ void bucket_desc_kernel(const int32_t* __restrict__ koff, const int32_t* __restrict__ kpost,
                                   const int32_t* __restrict__ qoff, const int32_t* __restrict__ qpost,
                                   const int32_t* __restrict__ items, int n_c, int64_t n, int a, int b,
                                   int64_t max_items, int causal_any, int4* __restrict__ desc) {
  const int64_t item = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  const int64_t bh = blockIdx.y;
  if (item >= max_items) return;
  const int64_t ob = bh * (n_c + 1);
  const int32_t* it = items + ob;
  int4 out = make_int4(-1, 0, 0, 0);
  if (item < it[n_c]) {
    int lo = 0, hi = n_c;  // it[lo] <= item < it[hi]
    while (hi - lo > 1) {
      const int mid = (lo + hi) >> 1;
      if (it[mid] <= item) lo = mid;
      else hi = mid;
    }
    const int k0 = koff[ob + lo] + static_cast<int>(item - it[lo]) * kBkKeys;
    const int nk = min(kBkKeys, koff[ob + lo + 1] - k0);
    int rs = qoff[ob + lo];
    const int r1 = qoff[ob + lo + 1];
    if (causal_any) {
      const int kmin = kpost[bh * n * b + k0];
      const int32_t* qp = qpost + bh * n * a;
      int h2 = r1;
      while (rs < h2) {
        const int mid = (rs + h2) >> 1;
        if (qp[mid] < kmin) rs = mid + 1;
        else h2 = mid;
      }
    }
    out = make_int4(lo | (nk << 16), k0, rs, r1);
  }
  desc[bh * max_items + item] = out;
}

// Rows without filler (X <= 0) get a slot of `bits` holding the keys of their
// indices; rowmap = slot, -1 past the capacity (the row kernel keeps those
// rows' dk and dv), -2 for rows with filler.  One wave per 64 rows, one
// counter atomic per wave.
__global__ __launch_bounds__(256) void bucket_rowmap_kernel(BwdParams p, int32_t* __restrict__ ctr,
                                                            int32_t* __restrict__ rowmap,
                                                            uint32_t* __restrict__ bits, int64_t cap,
                                                            int64_t words) {
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int64_t r0 = (static_cast<int64_t>(blockIdx.x) * 4 + wave) * 64;
  if (r0 >= p.rows) return;
  const int64_t r = r0 + lane;
  const bool in = r < p.rows;
  const bool need = in && p.pfx[r] <= 0;
  const uint64_t bal = __ballot(need);
  int base = 0;
  if (lane == 0 && bal) base = atomicAdd(ctr, static_cast<int>(__popcll(bal)));
  base = __shfl(base, 0);
  const int id = base + static_cast<int>(__builtin_amdgcn_mbcnt_hi(static_cast<uint32_t>(bal >> 32),
                                                                   __builtin_amdgcn_mbcnt_lo(static_cast<uint32_t>(bal), 0u)));
  if (in) rowmap[r] = need ? (id < cap ? id : -1) : -2;
  for (uint64_t todo = bal; todo; todo &= todo - 1) {
    const int rid = __shfl(id, __builtin_ctzll(todo));
    if (rid >= cap) break;  // ids ascend with the lane
    uint32_t* bm = bits + static_cast<int64_t>(rid) * words;
    for (int64_t w = lane; w < words; w += 64) bm[w] = 0u;
  }
  __threadfence();  // the cleared words reach memory before the ORs below
  for (uint64_t todo = bal; todo; todo &= todo - 1) {
    const int l = __builtin_ctzll(todo);
    const int rid = __shfl(id, l);
    if (rid >= cap) break;
    uint32_t* bm = bits + static_cast<int64_t>(rid) * words;
    const int64_t rr = r0 + l;
    const int64_t bh = rr / p.n, i = rr - bh * p.n;
    const int h = static_cast<int>(bh % p.h_kv);
    const int64_t bb = bh / p.h_kv;
    const int ewords = p.idx_i64 ? 2 : 1;
    const uint32_t* iw = reinterpret_cast<const uint32_t*>(p.idx) + (bb * p.idx_sb + i * p.idx_sn + h * p.idx_sh) * ewords;
    // eight index loads per lane at a time, all out before the first OR (two
    // dword loads each, with no branch on the index type; slots past top_k
    // reload the last slot, top_k >= 1 here)
    for (int s0 = 0; s0 < p.top_k; s0 += 64 * 8) {
      uint32_t lo8[8], hi8[8];
#pragma unroll
      for (int t = 0; t < 8; ++t) {
        const int sl = min(s0 + 64 * t + lane, p.top_k - 1);
        lo8[t] = iw[sl * ewords];
        hi8[t] = iw[sl * ewords + ewords - 1];
      }
#pragma unroll
      for (int t = 0; t < 8; ++t) {
        const int64_t j = p.idx_i64 ? static_cast<int64_t>((static_cast<uint64_t>(hi8[t]) << 32) | lo8[t])
                                    : static_cast<int64_t>(static_cast<int32_t>(lo8[t]));
        if (s0 + 64 * t + lane < p.top_k && j >= 0 && j < p.n) atomicOr(bm + (j >> 5), 1u << (j & 31));
      }
    }
  }
}

// meta[e] = (row position i, w) per query posting e: w = X for a row with
// filler, -2 - bitmap slot for a row without, -1 for a row the row kernel keeps.
__global__ void bucket_meta_kernel(const int32_t* __restrict__ qpost, int64_t per_bh, int64_t total, int64_t n,
                                   const int32_t* __restrict__ pfx, const int32_t* __restrict__ rowmap,
                                   int2* __restrict__ meta) {
  const int64_t e = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (e >= total) return;
  const int i = qpost[e];
  const int64_t r = (e / per_bh) * n + i;
  const int x = pfx[r];
  int w = x;
  if (x <= 0) {
    const int id = rowmap[r];
    w = id >= 0 ? -2 - id : -1;
  }
  meta[e] = make_int2(i, w);
}

// Prefix mode: the keys [0, X) of the rows with filler.  Rows are indexed by
// X (a counting sort of clamp(X, 0, top_k)), so the rows whose prefix reaches
// past key 32 kc are one suffix of that index; an item is 32 consecutive keys
// and up to kBkPfxRows of those rows.
constexpr int kBkPfxRows = 256;

__global__ void bucket_xcodes_kernel(const int32_t* __restrict__ pfx, int64_t rows, int top_k,
                                     int32_t* __restrict__ xc) {
  const int64_t r = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (r < rows) xc[r] = min(max(pfx[r], 0), top_k);
}

// pitems[bh][kc] = sum over kc' < kc of ceil(R_kc' / kBkPfxRows), R_kc the rows
// with X > 32 kc (xoff: [bh][top_k + 2]); kchunks key chunks; one block per bh.
__global__ __launch_bounds__(1024) void prefix_items_kernel(const int32_t* __restrict__ xoff, int top_k,
                                                            int kchunks, int32_t* __restrict__ pitems) {
  __shared__ int32_t wsum[16];
  __shared__ int32_t carry;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int32_t* o = xoff + static_cast<int64_t>(blockIdx.x) * (top_k + 2);
  int32_t* it = pitems + static_cast<int64_t>(blockIdx.x) * (kchunks + 1);
  if (tid == 0) carry = 0;
  __syncthreads();
  for (int base = 0; base < kchunks; base += 1024) {
    const int kc = base + tid;
    const int rk = kc < kchunks ? o[top_k + 1] - o[min(kBkKeys * kc + 1, top_k + 1)] : 0;
    const int cnt = (rk + kBkPfxRows - 1) / kBkPfxRows;
    int x = cnt;
#pragma unroll
    for (int s = 1; s < 64; s <<= 1) {
      const int y = __shfl_up(x, s);
      if (lane >= s) x += y;
    }
    if (lane == 63) wsum[wave] = x;
    __syncthreads();
    if (tid == 0) {
      int run = carry;
      for (int w = 0; w < 16; ++w) {
        const int t = wsum[w];
        wsum[w] = run;
        run += t;
      }
      carry = run;
    }
    __syncthreads();
    if (kc < kchunks) it[kc] = wsum[wave] + x - cnt;
    __syncthreads();
  }
  if (tid == 0) it[kchunks] = carry;
}

// Per prefix item slot: int4 (nk << 16, k0, rs, r1) -- keys k0 .. k0 + nk - 1
// and rows rs .. r1 - 1 of the X index -- or -1 past the bh's items.
__global__ void prefix_desc_kernel(const int32_t* __restrict__ xoff, const int32_t* __restrict__ pitems,
                                   int top_k, int kchunks, int kmax, int64_t max_items, int4* __restrict__ desc) {
  const int64_t item = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  const int64_t bh = blockIdx.y;
  if (item >= max_items) return;
  const int32_t* it = pitems + bh * (kchunks + 1);
  const int32_t* o = xoff + bh * (top_k + 2);
  int4 out = make_int4(-1, 0, 0, 0);
  if (item < it[kchunks]) {
    int lo = 0, hi = kchunks;  // it[lo] <= item < it[hi]
    while (hi - lo > 1) {
      const int mid = (lo + hi) >> 1;
      if (it[mid] <= item) lo = mid;
      else hi = mid;
    }
    const int k0 = kBkKeys * lo;
    const int nk = min(kBkKeys, kmax - k0);
    const int rs = o[min(k0 + 1, top_k + 1)] + static_cast<int>(item - it[lo]) * kBkPfxRows;
    const int r1 = min(rs + kBkPfxRows, o[top_k + 1]);
    out = make_int4(nk << 16, k0, rs, r1);
  }
  desc[bh * max_items + item] = out;
}

// 4 bf16 of the staged rows 4 q4 + e (e = 0..3) at column 16 dt + c16 (the
// first half of rows_transposed: a 16-row buffer).
template <int D>
__device__ __forceinline__ uint2 rows_transposed16(const unsigned char* l, int dt, int q4, int c16) {
  const int vkey = 4 * q4 + (c16 >> 2);
  const int off = vkey * MfShape<D>::ROW + (((2 * dt + ((c16 & 3) >> 1)) ^ mf_swz<D>(vkey)) << 4) + (c16 & 1) * 8;
  return __builtin_bit_cast(uint2, __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4i16_ptr)(l + off)));
}

__device__ __forceinline__ int bk_hash(int code) {
  return static_cast<int>((static_cast<uint32_t>(code) * 2654435761u) >> 23) & (kBkHash - 1);
}

template <int D, bool PFX>
// At least 3 waves per SIMD (3 blocks per CU, which the LDS also allows): at
// d = 128 the candidate build then keeps a few loop-invariant values in
// scratch, and still runs the c3 backward 1.4 ms faster than at 2 waves.
__global__ __launch_bounds__(kBkThreads) __attribute__((amdgpu_waves_per_eu(3, 8))) void
bucket_attention_bwd_kernel(BwdParams p, BucketParams bp) {
  using S = MfShape<D>;
  constexpr int KB = S::KB;
  constexpr int DT = D / 32;             // 16-dim tiles per wave (half of the dims)
  constexpr int QLD = kBkQv / S::KPI;    // wave-wide loads per staged tensor
  __shared__ __align__(16) unsigned char kvs[2][kBkKeys * S::ROW];     // K, V of the item's keys
  __shared__ __align__(16) unsigned char qds[2][2][kBkQv * S::ROW];    // [buffer][Q, dO] query vectors
  __shared__ __align__(16) float s_st[2][kBkQv][4];                    // softmax reference, 1/sum, D
  __shared__ int2 s_meta[2][kBkQv];                                    // (i, w) per row of a chunk
  __shared__ uint32_t s_bw[2][kBkQv][kBkKeys];                         // bitmap word per (row, key)
  __shared__ uint32_t s_dup[2][kBkQv];   // keys sharing a code below c with the row
  __shared__ uint32_t s_mask[kBkQv];     // pairs counted here, per row
  __shared__ int32_t s_j[kBkKeys];
  __shared__ int32_t s_kc[kBkKeys][kBkMaxB];
  __shared__ int32_t s_hk[kBkHash];      // codes below c of the item's keys ...
  __shared__ uint32_t s_hm[kBkHash];     // ... and the keys holding each

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int q4 = lane >> 4, c16 = lane & 15;
  const int64_t bh = blockIdx.y;
  const int4 ds = bp.desc[bh * bp.max_items + blockIdx.x];
  if (ds.x < 0) return;
  const int c = ds.x & 0xFFFF, nk = ds.x >> 16, k0 = ds.y, rs = ds.z, r1 = ds.w;
  const int g = p.g, gpl = bp.gp_log2, rpc = kBkQv >> gpl;
  const int nrc = (r1 - rs + rpc - 1) / rpc;
  if (nrc <= 0) return;
  const int32_t* kp = PFX ? nullptr : bp.kpost + bh * p.n * bp.b;
  const int2* meta = bp.meta + bh * p.n * bp.a;
  // key of item slot t (< nk): the bucket's posting, or prefix key k0 + t
  auto key_at = [&](int t) -> int { return PFX ? k0 + t : kp[k0 + t]; };
  const int h = static_cast<int>(bh % p.h_kv);
  const int64_t bb = bh / p.h_kv;

  if (tid < kBkKeys) {
    const int j = tid < nk ? key_at(tid) : -1;
    s_j[tid] = j;
    if constexpr (!PFX) {
      const int32_t* kcj = bp.kcodes + (bh * p.n + (j >= 0 ? j : 0)) * bp.b;
      int cv[kBkMaxB];
#pragma unroll
      for (int x = 0; x < kBkMaxB; ++x) cv[x] = kcj[x < bp.b ? x : 0];  // all loads in flight together
#pragma unroll
      for (int x = 0; x < kBkMaxB; ++x) s_kc[tid][x] = (j >= 0 && x < bp.b) ? cv[x] : 0x7FFFFFFF;
    }
  }
  for (int e = tid; e < kBkHash; e += kBkThreads) {
    s_hk[e] = -1;
    s_hm[e] = 0u;
  }
  if (tid < kBkQv) s_dup[0][tid] = 0u;
  // K and V of the chunk (32-bit buffer offsets, zeros past the chunk)
  const uint16_t* kbase = static_cast<const uint16_t*>(p.k) + bb * p.k_sb + static_cast<int64_t>(h) * p.k_sh;
  const uint16_t* vbase = static_cast<const uint16_t*>(p.v) + bb * p.v_sb + static_cast<int64_t>(h) * p.v_sh;
  const uint32_t ksn2 = 2u * static_cast<uint32_t>(p.k_sn), vsn2 = 2u * static_cast<uint32_t>(p.v_sn);
  const __amdgpu_buffer_rsrc_t krs = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint16_t*>(kbase), 0, static_cast<int>((p.n - 1) * p.k_sn * 2 + 2 * D), kBufferWord3);
  const __amdgpu_buffer_rsrc_t vrs = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint16_t*>(vbase), 0, static_cast<int>((p.n - 1) * p.v_sn * 2 + 2 * D), kBufferWord3);
  // this lane's segment offset in every load the wave issues: loads r = wave
  // + 4x (prologue) and r = wave (rows) share r mod SWZ_PERIOD (2 or 4)
  const uint32_t sgw = static_cast<uint32_t>(
      ((lane % S::SEGS) ^ mf_swz<D>(S::KPI * (wave % S::SWZ_PERIOD) + lane / S::SEGS)) << 4);
  constexpr int KVL = (S::NLD + kBkThreads / 64 - 1) / (kBkThreads / 64);  // K/V loads per wave
  int jl[KVL];
#pragma unroll
  for (int x = 0; x < KVL; ++x) {
    const int slot = S::KPI * (wave + x * (kBkThreads / 64)) + lane / S::SEGS;
    jl[x] = (wave + x * (kBkThreads / 64) < S::NLD && slot < nk) ? key_at(slot) : -1;
  }
#pragma unroll
  for (int x = 0; x < KVL; ++x) {
    const int r = wave + x * (kBkThreads / 64);
    if (r >= S::NLD) break;
    const int j = jl[x];
    const uint32_t sg = sgw;
    const uint32_t ko = j >= 0 ? __umul24(static_cast<uint32_t>(j), ksn2) + sg : kOobOffset;
    const uint32_t vo = j >= 0 ? __umul24(static_cast<uint32_t>(j), vsn2) + sg : kOobOffset;
    __builtin_amdgcn_raw_ptr_buffer_load_lds(krs, (lds_void_ptr)(kvs[0] + r * 1024), 16, static_cast<int>(ko), 0, 0, 0);
    __builtin_amdgcn_raw_ptr_buffer_load_lds(vrs, (lds_void_ptr)(kvs[1] + r * 1024), 16, static_cast<int>(vo), 0, 0, 0);
  }
  // Q and dO of the head group (offsets checked below 2^31 on the host)
  const uint16_t* qbase = static_cast<const uint16_t*>(p.q) + bb * p.q_sb + static_cast<int64_t>(h * g) * p.q_sh;
  const uint16_t* dbase = static_cast<const uint16_t*>(p.dout) + bb * p.do_sb + static_cast<int64_t>(h * g) * p.do_sh;
  const __amdgpu_buffer_rsrc_t qrs = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint16_t*>(qbase), 0, static_cast<int>(((p.n - 1) * p.q_sn + (g - 1) * p.q_sh) * 2 + 2 * D), kBufferWord3);
  const __amdgpu_buffer_rsrc_t drs = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint16_t*>(dbase), 0, static_cast<int>(((p.n - 1) * p.do_sn + (g - 1) * p.do_sh) * 2 + 2 * D), kBufferWord3);
  const int gmask = (1 << gpl) - 1;

  // the query vectors of chunk rows s_meta[bf] into qds[bf]
  auto stage_rows = [&](int bf) {
    if (wave < QLD) {
      const int qv = S::KPI * wave + lane / S::SEGS;
      const int rho = qv >> gpl, hh = qv & gmask;
      const int i = s_meta[bf][rho].x;
      const bool ok = rho < rpc && i >= 0 && hh < g;
      const uint32_t sg = sgw;
      const uint32_t qo = ok ? static_cast<uint32_t>((i * p.q_sn + hh * p.q_sh) * 2) + sg : kOobOffset;
      const uint32_t dof = ok ? static_cast<uint32_t>((i * p.do_sn + hh * p.do_sh) * 2) + sg : kOobOffset;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(qrs, (lds_void_ptr)(qds[bf][0] + wave * 1024), 16, static_cast<int>(qo), 0, 0, 0);
      __builtin_amdgcn_raw_ptr_buffer_load_lds(drs, (lds_void_ptr)(qds[bf][1] + wave * 1024), 16, static_cast<int>(dof), 0, 0, 0);
    }
  };
  // stats, query codes and bitmap words of chunk rows s_meta[bf], into registers
  float4 st_r = make_float4(0.f, 0.f, 0.f, 0.f);
  int qc_r[2] = {-1, -1};
  uint32_t bw_r[2] = {0u, 0u};
  auto load_rows = [&](int bf) {
    // (the candidate build makes the thread index opaque per call: its per-lane
    // address terms are recomputed here instead of hoisted out of the row loop
    // and spilled)
    int tidv = tid;
    if constexpr (!PFX) asm volatile("" : "+v"(tidv));
    if (tidv < kBkQv) {
      const int rho = tidv >> gpl, hh = tidv & gmask;
      const int i = s_meta[bf][rho].x;
      st_r = (rho < rpc && i >= 0 && hh < g)
                 ? *reinterpret_cast<const float4*>(p.pstats + ((bh * p.n + i) * g + hh) * 4)
                 : make_float4(0.f, 0.f, 0.f, 0.f);
    }
    if constexpr (PFX) return;
#pragma unroll
    for (int x = 0; x < 2; ++x) {
      const int e = tidv + kBkThreads * x;
      const int rho = e / bp.a, aa = e - rho * bp.a;
      qc_r[x] = -1;
      if (rho < rpc) {
        const int i = s_meta[bf][rho].x;
        if (i >= 0) {
          qc_r[x] = bp.qcodes[(bh * p.n + i) * bp.a + aa];
        }
      }
      const int rk = e >> 5, kappa = e & 31;
      bw_r[x] = 0u;
      if (rk < rpc) {
        const int w = s_meta[bf][rk].y;
        const int j = s_j[kappa];
        if (w <= -2 && j >= 0) bw_r[x] = bp.bits[static_cast<int64_t>(-2 - w) * bp.words + (j >> 5)];
      }
    }
  };
  // ... into LDS; a row code below c names the item's keys that share it
  auto store_rows = [&](int bf) {
    if (tid < kBkQv) *reinterpret_cast<float4*>(&s_st[bf][tid][0]) = st_r;
    if constexpr (PFX) return;
    int tidv = tid;  // (opaque, as in load_rows)
    asm volatile("" : "+v"(tidv));
#pragma unroll
    for (int x = 0; x < 2; ++x) {
      const int e = tidv + kBkThreads * x;
      const int rk = e >> 5;
      if (rk < rpc) s_bw[bf][rk][e & 31] = bw_r[x];
      const int code = qc_r[x];
      if (code >= 0 && code < c) {  // (code -1: no such row)
        int slot = bk_hash(code);
        uint32_t m = 0u;
        for (int probe = 0; probe < kBkHash; ++probe) {
          const int k2 = s_hk[slot];
          if (k2 == code) {
            m = s_hm[slot];
            break;
          }
          if (k2 == -1) break;
          slot = (slot + 1) & (kBkHash - 1);
        }
        if (m) atomicOr(&s_dup[bf][e / bp.a], m);
      }
    }
  };
  // which (row, key) pairs of chunk bf this item counts -> s_mask
  auto make_mask = [&](int bf) {
    int tidv = tid;  // (opaque in the candidate build, as in load_rows)
    if constexpr (!PFX) asm volatile("" : "+v"(tidv));
#pragma unroll
    for (int x = 0; x < 2; ++x) {
      if (x == 1 && rpc * kBkKeys <= kBkThreads) break;
      const int pr = tidv + kBkThreads * x;
      const int rho = pr >> 5, kappa = pr & 31;
      bool ok = false;
      if (rho < rpc) {
        const int2 m = s_meta[bf][rho];
        const int j = s_j[kappa];
        if constexpr (PFX) {
          ok = m.x >= 0 && j >= 0 && j < m.y && !(p.causal && j > m.x);  // the row's prefix [0, X)
        } else if (m.x >= 0 && j >= 0 && m.y != -1 && !(p.causal && j > m.x) &&
                   !((s_dup[bf][rho] >> kappa) & 1u)) {
          if (m.y > 0) ok = j >= m.y && !(bp.router_causal && j > m.x);
          else ok = ((s_bw[bf][rho][kappa] >> (j & 31)) & 1u) != 0;
        }
      }
      const uint64_t bal = __ballot(ok);
      const int rb = 2 * wave + 8 * x;
      if (lane == 0) {
        if (rb < rpc) s_mask[rb] = static_cast<uint32_t>(bal);
        if (rb + 1 < rpc) s_mask[rb + 1] = static_cast<uint32_t>(bal >> 32);
      }
    }
  };

  int2 m_next = make_int2(-1, -1);
  if (tid < kBkQv) {
    const int e0 = rs + tid, e1 = rs + rpc + tid;
    s_meta[0][tid] = (tid < rpc && e0 < r1) ? meta[e0] : make_int2(-1, -1);
    m_next = (tid < rpc && e1 < r1) ? meta[e1] : make_int2(-1, -1);
  }
  __syncthreads();
  // the item's codes below c -> keys holding them
  if constexpr (!PFX) {
    const int kappa = tid >> 3, y = tid & 7;
    const int code = s_kc[kappa][y];
    if (code < c) {
      int slot = bk_hash(code);
      for (int probe = 0; probe < kBkHash; ++probe) {
        const int prev = atomicCAS(&s_hk[slot], -1, code);
        if (prev == -1 || prev == code) {
          atomicOr(&s_hm[slot], 1u << kappa);
          break;
        }
        slot = (slot + 1) & (kBkHash - 1);
      }
    }
  }
  load_rows(0);
  stage_rows(0);
  __syncthreads();  // the hash is complete
  store_rows(0);
  if (tid < kBkQv) s_meta[1][tid] = m_next;
  __builtin_amdgcn_s_waitcnt(kWaitVm0);
  __syncthreads();

  const int t = wave & 1, dh = wave >> 1;
  const bool keys_here = 16 * t < nk;
  const int kswz = mf_swz<D>(16 * t + c16);
  // K / V fragments of the wave's keys, read from kvs at each use (not held in registers)
  const unsigned char* krow = kvs[0] + (16 * t + c16) * S::ROW;
  const unsigned char* vrow = kvs[1] + (16 * t + c16) * S::ROW;
  const int qswz = mf_swz<D>(c16);
  floatx4_t accv[DT], acck[DT];
#pragma unroll
  for (int dd = 0; dd < DT; ++dd) {
    accv[dd] = floatx4_t{0.f, 0.f, 0.f, 0.f};
    acck[dd] = floatx4_t{0.f, 0.f, 0.f, 0.f};
  }
  const uint32_t keybit = 1u << (16 * t + c16);

  for (int u = 0; u < nrc; ++u) {
    const int bf = u & 1, nb = bf ^ 1;
    make_mask(bf);
    if (tid < kBkQv) s_dup[nb][tid] = 0u;
    __syncthreads();  // s_mask of chunk u
    // every LDS read of chunk u, before chunk u + 1's LDS-bound loads
    uint32_t hm = 0;
    for (int rho = 0; rho < rpc; ++rho) hm |= s_mask[rho];
    const bool act = keys_here && ((hm >> (16 * t)) & 0xFFFFu) != 0;
    bf16x8_t qa[KB], da[KB];
    uint2 ad[DT], aq[DT];
    float3 stv[4];  // softmax reference, 1/sum, D (the stats' fourth float is unused)
    bool okv[4];
    if (act) {
      const unsigned char* ql = qds[bf][0];
      const unsigned char* dl = qds[bf][1];
#pragma unroll
      for (int kb = 0; kb < KB; ++kb) {
        qa[kb] = *(lds_bf16x8_ptr)(ql + c16 * S::ROW + (((kb * 4 + q4) ^ qswz) << 4));
        da[kb] = *(lds_bf16x8_ptr)(dl + c16 * S::ROW + (((kb * 4 + q4) ^ qswz) << 4));
      }
#pragma unroll
      for (int dd = 0; dd < DT; ++dd) {
        ad[dd] = rows_transposed16<D>(dl, DT * dh + dd, q4, c16);
        aq[dd] = rows_transposed16<D>(ql, DT * dh + dd, q4, c16);
      }
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int qv = 4 * q4 + e;
        stv[e] = make_float3(s_st[bf][qv][0], s_st[bf][qv][1], s_st[bf][qv][2]);
        okv[e] = (qv & gmask) < g && (s_mask[qv >> gpl] & keybit) != 0;
      }
    }
    if (u + 1 < nrc) load_rows(nb);
    if (u + 2 < nrc && tid < kBkQv) {
      const int e2 = rs + (u + 2) * rpc + tid;
      m_next = (tid < rpc && e2 < r1) ? meta[e2] : make_int2(-1, -1);
    }
    if (u + 1 < nrc) stage_rows(nb);
    if (act) {
      floatx4_t sv = {0.f, 0.f, 0.f, 0.f}, dv = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int kb = 0; kb < KB; ++kb) {
        const bf16x8_t kf = *(lds_bf16x8_ptr)(krow + (((kb * 4 + q4) ^ kswz) << 4));
        const bf16x8_t vf = *(lds_bf16x8_ptr)(vrow + (((kb * 4 + q4) ^ kswz) << 4));
        sv = __builtin_amdgcn_mfma_f32_16x16x32_bf16(qa[kb], kf, sv, 0, 0, 0);
        dv = __builtin_amdgcn_mfma_f32_16x16x32_bf16(da[kb], vf, dv, 0, 0, 0);
      }
      // lane (q4, c16): query vectors 4 q4 + e against key 16 t + c16
      float pv[4], dsv[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        pv[e] = okv[e] ? exp2f(sv[e] * p.qk_scale_log2 - stv[e].x) * stv[e].y : 0.0f;
        dsv[e] = pv[e] * (dv[e] - stv[e].z);
      }
      uint32_t bpw[4], bdw[4];
#pragma unroll
      for (int w = 0; w < 2; ++w) {
        const uint32_t ph = pack_bf16x2(pv[2 * w], pv[2 * w + 1]);
        const uint32_t qh = pack_bf16x2(dsv[2 * w], dsv[2 * w + 1]);
        bpw[w] = ph;
        bpw[2 + w] = pack_bf16x2(pv[2 * w] - __uint_as_float(ph << 16), pv[2 * w + 1] - __uint_as_float(ph & 0xFFFF0000u));
        bdw[w] = qh;
        bdw[2 + w] = pack_bf16x2(dsv[2 * w] - __uint_as_float(qh << 16), dsv[2 * w + 1] - __uint_as_float(qh & 0xFFFF0000u));
      }
      const bf16x8_t bpv = __builtin_bit_cast(bf16x8_t, make_uint4(bpw[0], bpw[1], bpw[2], bpw[3]));
      const bf16x8_t bds = __builtin_bit_cast(bf16x8_t, make_uint4(bdw[0], bdw[1], bdw[2], bdw[3]));
#pragma unroll
      for (int dd = 0; dd < DT; ++dd) {
        accv[dd] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
            __builtin_bit_cast(bf16x8_t, make_uint4(ad[dd].x, ad[dd].y, ad[dd].x, ad[dd].y)), bpv, accv[dd], 0, 0, 0);
        acck[dd] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
            __builtin_bit_cast(bf16x8_t, make_uint4(aq[dd].x, aq[dd].y, aq[dd].x, aq[dd].y)), bds, acck[dd], 0, 0, 0);
      }
    }
    if (u + 1 < nrc) store_rows(nb);
    if (u + 2 < nrc && tid < kBkQv) s_meta[bf][tid] = m_next;
    __builtin_amdgcn_s_waitcnt(kWaitVm0);
    __syncthreads();  // chunk u + 1 staged; every wave is done with chunk u
  }

  // dV^T, dK^T tiles: lane (q4, c16) holds dims 16 dt + 4 q4 + e of key 16 t + c16.
  // They pass through LDS (the row buffers are free now) as [key][dim] so that
  // each atomic instruction adds D/2 consecutive floats of one key row.
  if (!keys_here) return;
  constexpr int HD = D / 2;
  float* tw = reinterpret_cast<float*>(&qds[0][0][0]) + wave * 16 * HD;
  const int64_t grow = static_cast<int64_t>(p.h_kv) * p.d;  // floats between consecutive keys of dk / dv
  const int64_t kbase0 = (bb * p.n * p.h_kv + h) * p.d + dh * HD;
#pragma unroll
  for (int pass = 0; pass < 2; ++pass) {
    const float mul = pass == 0 ? 1.0f : p.inv_scale;
#pragma unroll
    for (int dd = 0; dd < DT; ++dd)
#pragma unroll
      for (int e = 0; e < 4; ++e)
        tw[c16 * HD + 16 * dd + 4 * q4 + e] = (pass == 0 ? accv[dd][e] : acck[dd][e]) * mul;
    __builtin_amdgcn_s_waitcnt(kWaitLgkm0);
    __builtin_amdgcn_wave_barrier();
    float* dst = (pass == 0 ? p.dv : p.dk) + kbase0;
    for (int kk = 0; kk < 16; ++kk) {
      const int j = s_j[16 * t + kk];
      if (j >= 0 && lane < HD) unsafeAtomicAdd(dst + j * grow + lane, tw[kk * HD + lane]);
    }
    __builtin_amdgcn_s_waitcnt(kWaitLgkm0);
    __builtin_amdgcn_wave_barrier();  // tw is rewritten by the next pass
  }
}

template <typename T, int GMAX>
int launch_bwd_g(const BwdParams& p, hipStream_t st) {
  const dim3 grid(static_cast<unsigned>(ceil_div(p.rows, kBwdWaves)));
  const dim3 block(64 * kBwdWaves);
  if (p.d <= 64)
    sparse_attention_bwd_kernel<T, GMAX, 1><<<grid, block, 0, st>>>(p);
  else if (p.d <= 128)
    sparse_attention_bwd_kernel<T, GMAX, 2><<<grid, block, 0, st>>>(p);
  else
    sparse_attention_bwd_kernel<T, GMAX, 4><<<grid, block, 0, st>>>(p);
  return check_launch("sparse_attention_bwd_kernel");
}

// The matrix-core kernel: bf16 inputs and output gradient, d = 64 or 128,
// g <= 8, q, dO and o rows 16-byte aligned (strides in multiples of 8
// elements), and K/V rows addressable by 32-bit buffer offsets (rows below
// 2^31 bytes, n and byte strides below 2^24).
bool bwd_mfma_ok(const BwdParams& p, const void* q, const void* dout) {
  const auto fits = [&](int64_t sn) {
    return sn >= 0 && 2 * sn < (int64_t(1) << 24) && (p.n - 1) * sn * 2 + 2 * p.d < (int64_t(1) << 31);
  };
  const bool aligned = (p.q_sb % 8 == 0) && (p.q_sn % 8 == 0) && (p.q_sh % 8 == 0) &&
                       (p.do_sb % 8 == 0) && (p.do_sn % 8 == 0) && (p.do_sh % 8 == 0) &&
                       (p.o_sb % 8 == 0) && (p.o_sn % 8 == 0) && (p.o_sh % 8 == 0) &&
                       (reinterpret_cast<uintptr_t>(q) % 16 == 0) && (reinterpret_cast<uintptr_t>(dout) % 16 == 0) &&
                       (reinterpret_cast<uintptr_t>(p.o) % 16 == 0);
  return p.do_bf16 && (p.d == 64 || p.d == 128) && p.g <= 8 && aligned && p.n < (int64_t(1) << 24) &&
         fits(p.k_sn) && fits(p.v_sn);
}

template <typename T>
int launch_bwd(const BwdParams& p, hipStream_t st) {
  if constexpr (sizeof(T) == 2) {
    if (bwd_mfma_ok(p, p.q, p.dout)) {
      const dim3 grid(static_cast<unsigned>(ceil_div(p.rows, kBwMfWaves)));
      if (p.rowmap) {  // bucket mode: dq only for most rows, the full kernel for rowmap == -1
        if (p.d == 64)
          sparse_attention_bwd_mfma_kernel<64, false><<<grid, 64 * kBwMfWaves, 0, st>>>(p);
        else
          sparse_attention_bwd_mfma_kernel<128, false><<<grid, 64 * kBwMfWaves, 0, st>>>(p);
        if (int s = check_launch("sparse_attention_bwd_mfma_kernel")) return s;
      }
      if (p.d == 64)
        sparse_attention_bwd_mfma_kernel<64, true><<<grid, 64 * kBwMfWaves, 0, st>>>(p);
      else
        sparse_attention_bwd_mfma_kernel<128, true><<<grid, 64 * kBwMfWaves, 0, st>>>(p);
      if (int s = check_launch("sparse_attention_bwd_mfma_kernel")) return s;
      if (!p.pfx) return SSA_OK;
      const int w = p.pfx_dq_only ? 4 : kPbWaves;
      const int64_t brows = static_cast<int64_t>(w) * pb_rows_per_wave(p.g, p.pfx_dq_only != 0);  // rows per block
      const dim3 pgrid(static_cast<unsigned>(kXcds * xcd_per((p.rows / p.n) * ceil_div(p.n, brows))));
      if (p.pfx_dq_only) {
        if (p.d == 64)
          prefix_attention_bwd_kernel<64, true><<<pgrid, 64 * w, 0, st>>>(p);
        else
          prefix_attention_bwd_kernel<128, true><<<pgrid, 64 * w, 0, st>>>(p);
      } else if (p.d == 64) {
        prefix_attention_bwd_kernel<64, false><<<pgrid, 64 * w, 0, st>>>(p);
      } else {
        prefix_attention_bwd_kernel<128, false><<<pgrid, 64 * w, 0, st>>>(p);
      }
      return check_launch("prefix_attention_bwd_kernel");
    }
  }
  if (p.g <= 4) return launch_bwd_g<T, 4>(p, st);
  if (p.g <= 8) return launch_bwd_g<T, 8>(p, st);
  return launch_bwd_g<T, 16>(p, st);
}

}  // namespace
}  // namespace ssa

using namespace ssa;

namespace ssa {
namespace {
// Per (row, head) softmax stats for the dense-prefix pass: 4 floats.
size_t bwd_ws_bytes(int dtype, int dout_dtype, int64_t batch, int64_t n, int h_q, int h_kv, int d) {
  if (dtype != SSA_DTYPE_BF16 || dout_dtype != SSA_DTYPE_BF16 || (d != 64 && d != 128) || h_kv <= 0 ||
      h_q % h_kv != 0 || h_q / h_kv > 8 || batch <= 0 || n <= 0)
    return 0;
  return sizeof(float) * 4 * static_cast<size_t>(batch * n * h_q);
}

// Bucket-mode workspace after the stats: query index (offsets, postings and
// its build scratch), item starts, a counter, rowmap, posting meta, then the
// key bitmaps (words per row each).
struct BucketWs {
  int32_t* qoff;
  int32_t* qpost;
  void* hist;
  int32_t* items;
  int4* desc;
  int32_t* ctr;
  int32_t* rowmap;
  int2* meta;
  // prefix mode: X per row (clamped), its index, item starts and descriptors,
  // posting meta (row, X)
  int32_t* xcodes;
  int32_t* xoff;
  int32_t* xpost;
  int32_t* pitems;
  int4* pdesc;
  int2* pmeta;
  uint32_t* bits;
  int64_t cap;  // bitmaps that fit
};

// Items (bucket, 32-key chunk) per bh at most: sum over c of ceil(|K_c| / 32).
int64_t bucket_max_items(int64_t n, int b, int n_c) { return ceil_div(n * b, kBkKeys) + n_c; }
// Prefix mode (X index of top_k + 1 codes): key chunks and items per bh at most.
bool prefix_mode_ok(int top_k) { return top_k + 1 <= 16384; }
int prefix_kchunks(int64_t n, int top_k) { return static_cast<int>(ceil_div(min(static_cast<int64_t>(top_k), n), kBkKeys)); }
int64_t prefix_max_items(int64_t n, int top_k) { return prefix_kchunks(n, top_k) * (ceil_div(n, kBkPfxRows) + 1); }

size_t bucket_fixed_bytes(int64_t batch, int64_t n, int h_kv, int a, int b, int n_c, int top_k) {
  const int64_t bh = batch * h_kv;
  const int xn = prefix_mode_ok(top_k) ? top_k + 1 : 1;
  const size_t hist = index_ws_bytes(bh, n, n_c) > index_ws_bytes(bh, n, xn) ? index_ws_bytes(bh, n, n_c)
                                                                              : index_ws_bytes(bh, n, xn);
  return align_up(sizeof(int32_t) * static_cast<size_t>(bh * (n_c + 1)), 256) +
         align_up(sizeof(int32_t) * static_cast<size_t>(bh * n * a), 256) + align_up(hist, 256) +
         align_up(sizeof(int32_t) * static_cast<size_t>(bh * (n_c + 1)), 256) +
         align_up(sizeof(int4) * static_cast<size_t>(bh * bucket_max_items(n, b, n_c)), 256) + 256 +
         align_up(sizeof(int32_t) * static_cast<size_t>(bh * n), 256) +
         align_up(sizeof(int2) * static_cast<size_t>(bh * n * a), 256) +
         align_up(sizeof(int32_t) * static_cast<size_t>(bh * n), 256) +
         align_up(sizeof(int32_t) * static_cast<size_t>(bh * (xn + 1)), 256) +
         align_up(sizeof(int32_t) * static_cast<size_t>(bh * n), 256) +
         align_up(sizeof(int32_t) * static_cast<size_t>(bh * (prefix_kchunks(n, top_k) + 1)), 256) +
         align_up(sizeof(int4) * static_cast<size_t>(bh * prefix_max_items(n, top_k)), 256) +
         align_up(sizeof(int2) * static_cast<size_t>(bh * n), 256);
}

int64_t bucket_words(int64_t n) { return ceil_div(n, 32); }

BucketWs carve_bucket_ws(void* base, size_t bytes, int64_t batch, int64_t n, int h_kv, int a, int b, int n_c,
                         int top_k) {
  const int64_t bh = batch * h_kv;
  char* c = static_cast<char*>(base);
  BucketWs w{};
  auto take = [&](size_t sz) {
    char* r = c;
    c += align_up(sz, 256);
    return r;
  };
  w.qoff = reinterpret_cast<int32_t*>(take(sizeof(int32_t) * static_cast<size_t>(bh * (n_c + 1))));
  w.qpost = reinterpret_cast<int32_t*>(take(sizeof(int32_t) * static_cast<size_t>(bh * n * a)));
  const int xn = prefix_mode_ok(top_k) ? top_k + 1 : 1;
  w.hist = take(index_ws_bytes(bh, n, n_c) > index_ws_bytes(bh, n, xn) ? index_ws_bytes(bh, n, n_c)
                                                                       : index_ws_bytes(bh, n, xn));
  w.items = reinterpret_cast<int32_t*>(take(sizeof(int32_t) * static_cast<size_t>(bh * (n_c + 1))));
  w.desc = reinterpret_cast<int4*>(take(sizeof(int4) * static_cast<size_t>(bh * bucket_max_items(n, b, n_c))));
  w.ctr = reinterpret_cast<int32_t*>(take(256));
  w.rowmap = reinterpret_cast<int32_t*>(take(sizeof(int32_t) * static_cast<size_t>(bh * n)));
  w.meta = reinterpret_cast<int2*>(take(sizeof(int2) * static_cast<size_t>(bh * n * a)));
  w.xcodes = reinterpret_cast<int32_t*>(take(sizeof(int32_t) * static_cast<size_t>(bh * n)));
  w.xoff = reinterpret_cast<int32_t*>(take(sizeof(int32_t) * static_cast<size_t>(bh * (xn + 1))));
  w.xpost = reinterpret_cast<int32_t*>(take(sizeof(int32_t) * static_cast<size_t>(bh * n)));
  w.pitems = reinterpret_cast<int32_t*>(take(sizeof(int32_t) * static_cast<size_t>(bh * (prefix_kchunks(n, top_k) + 1))));
  w.pdesc = reinterpret_cast<int4*>(take(sizeof(int4) * static_cast<size_t>(bh * prefix_max_items(n, top_k))));
  w.pmeta = reinterpret_cast<int2*>(take(sizeof(int2) * static_cast<size_t>(bh * n)));
  w.bits = reinterpret_cast<uint32_t*>(c);
  const size_t used = static_cast<size_t>(c - static_cast<char*>(base));
  const size_t row_bytes = sizeof(uint32_t) * static_cast<size_t>(bucket_words(n));
  w.cap = bytes > used ? static_cast<int64_t>((bytes - used) / row_bytes) : 0;
  if (w.cap > bh * n) w.cap = bh * n;
  return w;
}

// Checks and fills the parameters shared by both backward entry points.
// Returns SSA_OK with `empty` set when there is nothing to compute.
int bwd_setup(const void* q, const void* k, const void* v, int dtype, int64_t batch, int64_t n, int h_q,
              int h_kv, int d, int64_t q_sb, int64_t q_sn, int64_t q_sh, int64_t k_sb, int64_t k_sn,
              int64_t k_sh, int64_t v_sb, int64_t v_sn, int64_t v_sh, const void* idx, int idx_dtype,
              int top_k, int64_t idx_sb, int64_t idx_sn, int64_t idx_sh, float scale_div, int causal,
              const int32_t* row_order, const void* out, int out_dtype, int64_t o_sb, int64_t o_sn,
              int64_t o_sh, const void* dout, int dout_dtype, int64_t do_sb, int64_t do_sn, int64_t do_sh,
              float* dq, float* dk, float* dv, int32_t* error_flag, BwdParams& p, bool& empty) {
  empty = false;
  if (dtype != SSA_DTYPE_F32 && dtype != SSA_DTYPE_BF16)
    return fail(SSA_ERR_UNSUPPORTED, "sparse_attention_backward: dtype %d not supported (f32, bf16)", dtype);
  if ((out_dtype != SSA_DTYPE_F32 && out_dtype != SSA_DTYPE_BF16) ||
      (dout_dtype != SSA_DTYPE_F32 && dout_dtype != SSA_DTYPE_BF16))
    return fail(SSA_ERR_UNSUPPORTED, "sparse_attention_backward: out/dout dtype not supported");
  if (idx_dtype != SSA_INDEX_I32 && idx_dtype != SSA_INDEX_I64)
    return fail(SSA_ERR_INVALID_ARGUMENT, "sparse_attention_backward: idx dtype %d", idx_dtype);
  if (batch < 0 || n < 0 || h_q <= 0 || h_kv <= 0 || top_k < 0)
    return fail(SSA_ERR_INVALID_ARGUMENT, "sparse_attention_backward: bad shape");
  if (h_q % h_kv != 0)
    return fail(SSA_ERR_INVALID_ARGUMENT, "num_q_heads must be divisible by num_kv_heads");
  if (h_q / h_kv > 16)
    return fail(SSA_ERR_UNSUPPORTED, "sparse_attention_backward: group size %d > 16", h_q / h_kv);
  if (d < 1 || d > 256)
    return fail(SSA_ERR_UNSUPPORTED, "sparse_attention_backward: head_dim %d (need 1..256)", d);
  if (!(scale_div > 0.0f) && !(scale_div < 0.0f))
    return fail(SSA_ERR_INVALID_ARGUMENT, "sparse_attention_backward: scale must be non-zero");
  if (batch == 0 || n == 0) {
    empty = true;
    return SSA_OK;
  }
  if (!q || !k || !v || !out || !dout || !dq || !dk || !dv || (top_k > 0 && !idx))
    return fail(SSA_ERR_INVALID_ARGUMENT, "sparse_attention_backward: null pointer");
  p = BwdParams{};
  p.q = q; p.k = k; p.v = v; p.o = out; p.dout = dout;
  p.n = n; p.h_q = h_q; p.h_kv = h_kv; p.g = h_q / h_kv; p.d = d;
  p.q_sb = q_sb; p.q_sn = q_sn; p.q_sh = q_sh;
  p.k_sb = k_sb; p.k_sn = k_sn; p.k_sh = k_sh;
  p.v_sb = v_sb; p.v_sn = v_sn; p.v_sh = v_sh;
  p.o_sb = o_sb; p.o_sn = o_sn; p.o_sh = o_sh;
  p.do_sb = do_sb; p.do_sn = do_sn; p.do_sh = do_sh;
  p.o_bf16 = out_dtype == SSA_DTYPE_BF16;
  p.do_bf16 = dout_dtype == SSA_DTYPE_BF16;
  p.idx = idx; p.idx_i64 = idx_dtype == SSA_INDEX_I64; p.top_k = top_k;
  p.idx_sb = idx_sb; p.idx_sn = idx_sn; p.idx_sh = idx_sh;
  p.inv_scale = 1.0f / scale_div;
  p.qk_scale_log2 = static_cast<float>(1.4426950408889634 / static_cast<double>(scale_div));
  p.causal = causal ? 1 : 0;
  p.dq = dq; p.dk = dk; p.dv = dv;
  p.err = error_flag;
  p.rows = batch * h_kv * n;
  p.order = row_order;
  if (p.rows >= (int64_t(1) << 31))
    return fail(SSA_ERR_UNSUPPORTED, "sparse_attention_backward: too many rows");
  return SSA_OK;
}

// dk and dv accumulate; dq rows are written whole by the row that owns them.
int zero_dkdv(const BwdParams& p, int64_t batch, hipStream_t st) {
  const int64_t kv_elems = batch * p.n * p.h_kv * p.d;
  zero_f32_kernel<<<dim3(static_cast<unsigned>(ceil_div(kv_elems, 256))), 256, 0, st>>>(p.dk, kv_elems);
  zero_f32_kernel<<<dim3(static_cast<unsigned>(ceil_div(kv_elems, 256))), 256, 0, st>>>(p.dv, kv_elems);
  return check_launch("zero_f32_kernel");
}

// The plain path (row kernel, then the dense-prefix pass when p.pfx is set).
int run_bwd(BwdParams& p, int dtype, int64_t batch, const int32_t* row_prefix, void* workspace,
            size_t workspace_bytes, int dout_dtype, hipStream_t st) {
  if (row_prefix && workspace) {
    const size_t need = bwd_ws_bytes(dtype, dout_dtype, batch, p.n, p.h_q, p.h_kv, p.d);
    if (workspace_bytes < need)
      return fail(SSA_ERR_WORKSPACE, "sparse_attention_backward: workspace %zu < %zu bytes", workspace_bytes, need);
    if (need > 0 && dtype == SSA_DTYPE_BF16 && bwd_mfma_ok(p, p.q, p.dout)) {
      p.pfx = row_prefix;
      p.pstats = static_cast<float*>(workspace);
    }
  }
  if (int s = zero_dkdv(p, batch, st)) return s;
  if (dtype == SSA_DTYPE_BF16) return launch_bwd<uint16_t>(p, st);
  return launch_bwd<float>(p, st);
}

// Shapes the bucket path takes (else the routed entry runs the plain path).
bool bucket_ok(const BwdParams& p, int dtype, int dout_dtype, int a, int b, int n_c) {
  if (dtype != SSA_DTYPE_BF16 || dout_dtype != SSA_DTYPE_BF16 || !bwd_mfma_ok(p, p.q, p.dout)) return false;
  if (a < 1 || a > kBkMaxA || b < 1 || b > kBkMaxB || n_c < 1 || n_c > 16384) return false;
  if (p.n < p.top_k || p.top_k < 1) return false;  // rows padded past n hold key 0 repeatedly
  const auto fits = [&](int64_t sn, int64_t sh) {
    return sn >= 0 && sh >= 0 && ((p.n - 1) * sn + (p.g - 1) * sh) * 2 + 2 * p.d < (int64_t(1) << 31);
  };
  return fits(p.q_sn, p.q_sh) && fits(p.do_sn, p.do_sh) && p.n * a < (int64_t(1) << 31);
}
}  // namespace
}  // namespace ssa

extern "C" size_t ssa_sparse_attention_backward_workspace_bytes(int dtype, int dout_dtype, int64_t batch,
                                                                int64_t n, int h_q, int h_kv, int d) {
  return bwd_ws_bytes(dtype, dout_dtype, batch, n, h_q, h_kv, d);
}

extern "C" int ssa_sparse_attention_backward(
    const void* q, const void* k, const void* v, int dtype, int64_t batch, int64_t n, int h_q,
    int h_kv, int d, int64_t q_sb, int64_t q_sn, int64_t q_sh, int64_t k_sb, int64_t k_sn,
    int64_t k_sh, int64_t v_sb, int64_t v_sn, int64_t v_sh, const void* idx, int idx_dtype,
    int top_k, int64_t idx_sb, int64_t idx_sn, int64_t idx_sh, float scale_div, int causal,
    const int32_t* row_order, const void* out, int out_dtype, int64_t o_sb, int64_t o_sn,
    int64_t o_sh, const void* dout, int dout_dtype, int64_t do_sb, int64_t do_sn, int64_t do_sh,
    float* dq, float* dk, float* dv, int32_t* error_flag, const int32_t* row_prefix,
    const float* row_stats, void* workspace, size_t workspace_bytes, void* stream) {
  BwdParams p;
  bool empty = false;
  if (int s = bwd_setup(q, k, v, dtype, batch, n, h_q, h_kv, d, q_sb, q_sn, q_sh, k_sb, k_sn, k_sh, v_sb, v_sn,
                        v_sh, idx, idx_dtype, top_k, idx_sb, idx_sn, idx_sh, scale_div, causal, row_order, out,
                        out_dtype, o_sb, o_sn, o_sh, dout, dout_dtype, do_sb, do_sn, do_sh, dq, dk, dv,
                        error_flag, p, empty))
    return s;
  if (empty) return SSA_OK;
  p.stats_in = row_stats;
  return run_bwd(p, dtype, batch, row_prefix, workspace, workspace_bytes, dout_dtype, as_stream(stream));
}

extern "C" size_t ssa_sparse_attention_backward_routed_workspace_bytes(int dtype, int dout_dtype, int64_t batch,
                                                                       int64_t n, int h_q, int h_kv, int d,
                                                                       int top_k, int a, int b, int n_c,
                                                                       int64_t bitmap_rows) {
  const size_t stats = bwd_ws_bytes(dtype, dout_dtype, batch, n, h_q, h_kv, d);
  if (stats == 0 || a < 1 || a > kBkMaxA || b < 1 || b > kBkMaxB || n_c < 1 || n_c > 16384) return stats;
  const int64_t rows = batch * h_kv * n;
  const int64_t cap = bitmap_rows < 0 ? (rows + 1) / 2 : (bitmap_rows < rows ? bitmap_rows : rows);
  if (top_k < 1) return stats;
  return align_up(stats, 256) + bucket_fixed_bytes(batch, n, h_kv, a, b, n_c, top_k) +
         sizeof(uint32_t) * static_cast<size_t>(bucket_words(n)) * static_cast<size_t>(cap);
}

extern "C" int ssa_sparse_attention_backward_routed(
    const void* q, const void* k, const void* v, int dtype, int64_t batch, int64_t n, int h_q,
    int h_kv, int d, int64_t q_sb, int64_t q_sn, int64_t q_sh, int64_t k_sb, int64_t k_sn,
    int64_t k_sh, int64_t v_sb, int64_t v_sn, int64_t v_sh, const void* idx, int idx_dtype,
    int top_k, int64_t idx_sb, int64_t idx_sn, int64_t idx_sh, float scale_div, int causal,
    const int32_t* row_order, const void* out, int out_dtype, int64_t o_sb, int64_t o_sn,
    int64_t o_sh, const void* dout, int dout_dtype, int64_t do_sb, int64_t do_sn, int64_t do_sh,
    float* dq, float* dk, float* dv, int32_t* error_flag, const int32_t* row_prefix,
    const float* row_stats, const int32_t* q_codes, int a, const int32_t* k_codes, int b,
    const int32_t* offsets, const int32_t* postings, int n_c, int router_causal, void* workspace,
    size_t workspace_bytes, void* stream) {
  BwdParams p;
  bool empty = false;
  if (int s = bwd_setup(q, k, v, dtype, batch, n, h_q, h_kv, d, q_sb, q_sn, q_sh, k_sb, k_sn, k_sh, v_sb, v_sn,
                        v_sh, idx, idx_dtype, top_k, idx_sb, idx_sn, idx_sh, scale_div, causal, row_order, out,
                        out_dtype, o_sb, o_sn, o_sh, dout, dout_dtype, do_sb, do_sn, do_sh, dq, dk, dv,
                        error_flag, p, empty))
    return s;
  if (empty) return SSA_OK;
  p.stats_in = row_stats;
  if (!row_prefix || !q_codes || !k_codes || !offsets || !postings)
    return fail(SSA_ERR_INVALID_ARGUMENT, "sparse_attention_backward_routed: null routing pointer");
  hipStream_t st = as_stream(stream);
  if (!bucket_ok(p, dtype, dout_dtype, a, b, n_c))
    return run_bwd(p, dtype, batch, row_prefix, workspace, workspace_bytes, dout_dtype, st);
  const size_t stats = align_up(bwd_ws_bytes(dtype, dout_dtype, batch, n, h_q, h_kv, d), 256);
  const size_t need = stats + bucket_fixed_bytes(batch, n, h_kv, a, b, n_c, top_k);
  if (!workspace || workspace_bytes < need)
    return fail(SSA_ERR_WORKSPACE, "sparse_attention_backward_routed: workspace %zu < %zu bytes",
                workspace ? workspace_bytes : size_t(0), need);
  const int64_t bhn = batch * h_kv;
  BucketWs w = carve_bucket_ws(static_cast<char*>(workspace) + stats, workspace_bytes - stats, batch, n, h_kv, a, b,
                               n_c, top_k);
  p.pfx = row_prefix;
  p.pstats = static_cast<float*>(workspace);
  p.rowmap = w.rowmap;
  if (int s = zero_dkdv(p, batch, st)) return s;
  zero_f32_kernel<<<1, 64, 0, st>>>(reinterpret_cast<float*>(w.ctr), 64);
  // stats of a row that row_order never lists stay zero (1/sum = 0: no pair of it counts)
  const int64_t nstats = 4 * p.rows * p.g;
  zero_f32_kernel<<<dim3(static_cast<unsigned>(ceil_div(nstats, 256))), 256, 0, st>>>(p.pstats, nstats);
  if (int s = check_launch("zero_f32_kernel")) return s;
  if (int s = build_index_into(q_codes, bhn, n, a, n_c, w.qoff, w.qpost, w.hist, st)) return s;
  bucket_items_kernel<<<dim3(static_cast<unsigned>(bhn)), 1024, 0, st>>>(offsets, n_c, w.items);
  if (int s = check_launch("bucket_items_kernel")) return s;
  const int64_t max_items = bucket_max_items(n, b, n_c);
  bucket_desc_kernel<<<dim3(static_cast<unsigned>(ceil_div(max_items, 256)), static_cast<unsigned>(bhn)), 256, 0, st>>>(
      offsets, postings, w.qoff, w.qpost, w.items, n_c, n, a, b, max_items, (causal || router_causal) ? 1 : 0, w.desc);
  if (int s = check_launch("bucket_desc_kernel")) return s;
  const int64_t words = bucket_words(n);
  bucket_rowmap_kernel<<<dim3(static_cast<unsigned>(ceil_div(p.rows, 256))), 256, 0, st>>>(p, w.ctr, w.rowmap, w.bits,
                                                                                             w.cap, words);
  if (int s = check_launch("bucket_rowmap_kernel")) return s;
  const int64_t entries = bhn * n * a;
  bucket_meta_kernel<<<dim3(static_cast<unsigned>(ceil_div(entries, 256))), 256, 0, st>>>(
      w.qpost, n * a, entries, n, row_prefix, w.rowmap, w.meta);
  if (int s = check_launch("bucket_meta_kernel")) return s;
  // prefix mode: the X index, its items and meta; the prefix pass then adds dq only
  const bool pfx_mode = prefix_mode_ok(top_k);
  const int kchunks = prefix_kchunks(n, top_k);
  const int64_t pmax = prefix_max_items(n, top_k);
  if (pfx_mode && kchunks > 0) {
    bucket_xcodes_kernel<<<dim3(static_cast<unsigned>(ceil_div(p.rows, 256))), 256, 0, st>>>(row_prefix, p.rows, top_k,
                                                                                             w.xcodes);
    if (int s = check_launch("bucket_xcodes_kernel")) return s;
    if (int s = build_index_into(w.xcodes, bhn, n, 1, top_k + 1, w.xoff, w.xpost, w.hist, st)) return s;
    prefix_items_kernel<<<dim3(static_cast<unsigned>(bhn)), 1024, 0, st>>>(w.xoff, top_k, kchunks, w.pitems);
    if (int s = check_launch("prefix_items_kernel")) return s;
    prefix_desc_kernel<<<dim3(static_cast<unsigned>(ceil_div(pmax, 256)), static_cast<unsigned>(bhn)), 256, 0, st>>>(
        w.xoff, w.pitems, top_k, kchunks, static_cast<int>(min(static_cast<int64_t>(top_k), n)), pmax, w.pdesc);
    if (int s = check_launch("prefix_desc_kernel")) return s;
    bucket_meta_kernel<<<dim3(static_cast<unsigned>(ceil_div(p.rows, 256))), 256, 0, st>>>(
        w.xpost, n, p.rows, n, row_prefix, w.rowmap, w.pmeta);
    if (int s = check_launch("bucket_meta_kernel")) return s;
    p.pfx_dq_only = 1;
  }
  if (int s = launch_bwd<uint16_t>(p, st)) return s;  // row kernel (dq, stats, fallback rows) + prefix pass
  BucketParams bp{};
  bp.kpost = postings;
  bp.kcodes = k_codes;
  bp.desc = w.desc;
  bp.meta = w.meta;
  bp.qcodes = q_codes;
  bp.bits = w.bits;
  bp.words = words;
  bp.max_items = max_items;
  bp.a = a;
  bp.b = b;
  int gpl = 0;
  while ((1 << gpl) < p.g) ++gpl;
  bp.gp_log2 = gpl;
  bp.router_causal = router_causal ? 1 : 0;
  const dim3 grid(static_cast<unsigned>(max_items), static_cast<unsigned>(bhn));
  if (d == 64)
    bucket_attention_bwd_kernel<64, false><<<grid, kBkThreads, 0, st>>>(p, bp);
  else
    bucket_attention_bwd_kernel<128, false><<<grid, kBkThreads, 0, st>>>(p, bp);
  if (int s = check_launch("bucket_attention_bwd_kernel")) return s;
  if (!p.pfx_dq_only) return SSA_OK;
  BucketParams pp = bp;  // the prefix keys: X index rows, consecutive keys
  pp.desc = w.pdesc;
  pp.meta = w.pmeta;
  pp.a = 1;
  pp.max_items = pmax;
  const dim3 pgrid(static_cast<unsigned>(pmax), static_cast<unsigned>(bhn));
  if (d == 64)
    bucket_attention_bwd_kernel<64, true><<<pgrid, kBkThreads, 0, st>>>(p, pp);
  else
    bucket_attention_bwd_kernel<128, true><<<pgrid, kBkThreads, 0, st>>>(p, pp);
  return check_launch("bucket_attention_bwd_kernel");
}
