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

template <int D>
__global__ __launch_bounds__(64 * kBwMfWaves, 2) void sparse_attention_bwd_mfma_kernel(BwdParams p) {
  using S = MfShape<D>;
  constexpr int KB = S::KB, NT = S::NT;
  __shared__ __align__(16) unsigned char kv_lds[kBwMfWaves][2][kMfChunk * S::ROW];
  __shared__ __align__(16) float tr_lds[kBwMfWaves][kMfChunk][16];      // P or dS as [key][head]
  __shared__ __align__(16) uint16_t hd_lds[kBwMfWaves][2][D][8];        // Q, dO as [dim][head] (bf16)

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
  const int h = static_cast<int>(bh % p.h_kv);
  const int64_t bb = bh / p.h_kv;
  const int g = p.g;
  const bool col_ok = c16 < g;

  // q and dO fragments (B operands of S^T and dP^T): head c16, dims kb*32 + q4*8 + 0..7
  const int hq = h * g + (col_ok ? c16 : 0);
  const uint16_t* qh = static_cast<const uint16_t*>(p.q) + bb * p.q_sb + i * p.q_sn + static_cast<int64_t>(hq) * p.q_sh;
  const uint16_t* dh = static_cast<const uint16_t*>(p.dout) + bb * p.do_sb + i * p.do_sn + static_cast<int64_t>(hq) * p.do_sh;
  bf16x8_t qf[KB], df[KB];
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
      if (col_ok) dpart = fma_rn(bf16_bits_to_f32(dv), ld_any(p.o, bb * p.o_sb + i * p.o_sn + static_cast<int64_t>(hq) * p.o_sh + dim, p.o_bf16), dpart);
      if (c16 < 8) {  // head slots 0..7 of the [dim][head] copies (zero past g)
        hd_lds[wave][0][dim][c16] = col_ok ? qv : static_cast<uint16_t>(0);
        hd_lds[wave][1][dim][c16] = col_ok ? dv : static_cast<uint16_t>(0);
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
  auto load_idx = [&](int ch) -> int {
    const int slot = ch * kMfChunk + lane;
    if (lane >= kMfChunk || slot >= p.top_k) return -1;
    const int64_t j = p.idx_i64 ? reinterpret_cast<const int64_t*>(ib)[slot]
                                : static_cast<int64_t>(reinterpret_cast<const int32_t*>(ib)[slot]);
    if (j < 0 || j >= p.n) {
      if (p.err) p.err[0] = 1;
      return -2;
    }
    return static_cast<int>(j);
  };
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

  // ---- pass 1: running max (log2 domain) and sum per head over the row's slots
  float m_run = -INFINITY, l_run = 0.0f;
  {
    int jn = nchunks > 0 ? load_idx(0) : -1;
    uint64_t okn = __ballot(chunk_ok(jn));
    if (nchunks > 0) row_issue<D>(krs, kl, chunk_ok(jn) ? jn : -1, lane, ksn2, seg16);
    jn = nchunks > 1 ? load_idx(1) : -1;
    for (int ch = 0; ch < nchunks; ++ch) {
      __builtin_amdgcn_s_waitcnt(kWaitVm0);
      bf16x8_t kf[2][KB];
      read_k(kl, kf);
      __builtin_amdgcn_s_waitcnt(kWaitLgkm0);
      const uint64_t okb = okn;
      if (ch + 1 < nchunks) {
        okn = __ballot(chunk_ok(jn));
        row_issue<D>(krs, kl, chunk_ok(jn) ? jn : -1, lane, ksn2, seg16);
        jn = ch + 2 < nchunks ? load_idx(ch + 2) : -1;
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
  const float inv_l = (l_tot > 0.0f && col_ok) ? 1.0f / l_tot : 0.0f;  // 0: no slot, or an unused column
  const float mref = (m_run == -INFINITY) ? 0.0f : m_run;
  // the prefix keys [0, X) go to prefix_attention_bwd_kernel, which needs the
  // row's softmax reference, 1/sum and D
  const int xpre = p.pfx ? p.pfx[bh * p.n + i] : 0;
  if (p.pfx && q4 == 0 && col_ok) {
    float* ps = p.pstats + ((bh * p.n + i) * g + c16) * 4;
    ps[0] = mref;
    ps[1] = inv_l;
    ps[2] = dcol;
  }
  auto chunk_ok2 = [&](int j) { return j >= xpre && chunk_ok(j); };

  // ---- pass 2
  const bool hi_row = c16 < g;
  const bool lo_row = c16 >= 8 && c16 < 8 + g;
  floatx4_t dqacc[NT];
#pragma unroll
  for (int t = 0; t < NT; ++t) dqacc[t] = floatx4_t{0.f, 0.f, 0.f, 0.f};
  float* dkb = p.dk + (bb * p.n * p.h_kv + h) * p.d;
  float* dvb = p.dv + (bb * p.n * p.h_kv + h) * p.d;
  const int64_t krow = static_cast<int64_t>(p.h_kv) * p.d;
  float* tr = &tr_lds[wave][0][0];
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
    return *reinterpret_cast<const bf16x8_t*>(&hd_lds[wave][which][16 * dt + c16][0]);
  };
  int jc = nchunks > 0 ? load_idx(0) : -1;
  uint64_t okn = __ballot(chunk_ok2(jc));
  if (nchunks > 0) {
    row_issue<D>(krs, kl, chunk_ok2(jc) ? jc : -1, lane, ksn2, seg16);
    row_issue<D>(vrs, vl, chunk_ok2(jc) ? jc : -1, lane, vsn2, seg16);
  }
  int jn = nchunks > 1 ? load_idx(1) : -1;
  for (int ch = 0; ch < nchunks; ++ch) {
    __builtin_amdgcn_s_waitcnt(kWaitVm0);
    bf16x8_t kf[2][KB], vf[2][KB], kt[NT];
    read_k(kl, kf);
    read_k(vl, vf);
#pragma unroll
    for (int t = 0; t < NT; ++t) kt[t] = rows_transposed<D>(kl, t, q4, c16);
    __builtin_amdgcn_s_waitcnt(kWaitLgkm0);
    const uint64_t okb = okn;
    const int jcur = jc;
    if (ch + 1 < nchunks) {
      okn = __ballot(chunk_ok2(jn));
      row_issue<D>(krs, kl, chunk_ok2(jn) ? jn : -1, lane, ksn2, seg16);
      row_issue<D>(vrs, vl, chunk_ok2(jn) ? jn : -1, lane, vsn2, seg16);
      jc = jn;
      jn = ch + 2 < nchunks ? load_idx(ch + 2) : -1;
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

template <int D>
__global__ __launch_bounds__(64 * kPbWaves, 1) void prefix_attention_bwd_kernel(BwdParams p) {
  using S = MfShape<D>;
  constexpr int KB = S::KB, NT = S::NT;
  constexpr int QV = 8 * kPbWaves;      // query vectors per block at most (g <= 8)
  constexpr int LPW = (S::NLD + kPbWaves - 1) / kPbWaves;  // chunk loads per wave and tensor
  __shared__ __align__(16) unsigned char kv[2][2][kMfChunk * S::ROW];  // [buffer][K, V]
  __shared__ __align__(16) float pall[2][kMfChunk][QV];                // P, dS as [key][qv]
  __shared__ __align__(16) uint16_t qall[2][D][QV];                    // Q, dO as [dim][qv] (bf16)
  __shared__ int s_xmax;

  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int tid = threadIdx.x, lane = tid & 63;
  const int q4 = lane >> 4, c16 = lane & 15;
  const int g = p.g;
  const int64_t tiles = ceil_div(p.n, kPbWaves);
  const int64_t nblk = (p.rows / p.n) * tiles;
  const int64_t blk = xcd_block(blockIdx.x, xcd_per(nblk));
  if (blk >= nblk) return;
  const int64_t bh = blk / tiles;
  const int64_t i = (blk - bh * tiles) * kPbWaves + wave;  // this wave's row
  const bool row_ok = i < p.n;
  const int h = static_cast<int>(bh % p.h_kv);
  const int64_t bb = bh / p.h_kv;
  const bool col_ok = c16 < g;
  const int xcap = static_cast<int>(min(static_cast<int64_t>(p.top_k), p.n));
  const int xrow = row_ok ? min(max(p.pfx[bh * p.n + i], 0), xcap) : 0;

  // the block's Q and dO as [dim][qv], zero for unused query vectors (whose P
  // and dS columns stay zero too: the reductions run over whole 32-column blocks)
  for (int e = tid; e < 2 * D * QV; e += 64 * kPbWaves) reinterpret_cast<uint16_t*>(qall)[e] = 0;
  for (int e = tid; e < 2 * kMfChunk * QV; e += 64 * kPbWaves) reinterpret_cast<float*>(pall)[e] = 0.0f;
  if (tid == 0) s_xmax = 0;
  __syncthreads();
  if (lane == 0) atomicMax(&s_xmax, xrow);
  const int hq = h * g + (col_ok ? c16 : 0);
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
      for (int e = 0; e < 8; ++e) {
        const int dim = kb * 32 + q4 * 8 + e;
        qall[0][dim][wave * g + c16] = static_cast<uint16_t>((e & 1) ? (qw[e >> 1] >> 16) : (qw[e >> 1] & 0xFFFFu));
        qall[1][dim][wave * g + c16] = static_cast<uint16_t>((e & 1) ? (dw[e >> 1] >> 16) : (dw[e >> 1] & 0xFFFFu));
      }
    }
  }
  float mref = 0.0f, inv_l = 0.0f, dcol = 0.0f;
  if (have) {
    const float* ps = p.pstats + ((bh * p.n + i) * g + c16) * 4;
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
  // this wave's loads of chunk ch: loads r = wave + kPbWaves * t (< NLD) of K and V
  auto issue = [&](int ch) {
#pragma unroll
    for (int t = 0; t < LPW; ++t) {
      const int r = wave + kPbWaves * t;
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
  const bool hi_row = c16 < g;
  const bool lo_row = c16 >= 8 && c16 < 8 + g;
  floatx4_t dqacc[NT];
#pragma unroll
  for (int t = 0; t < NT; ++t) dqacc[t] = floatx4_t{0.f, 0.f, 0.f, 0.f};
  float* dkb = p.dk + (bb * p.n * p.h_kv + h) * p.d;
  float* dvb = p.dv + (bb * p.n * p.h_kv + h) * p.d;
  const int64_t krow = static_cast<int64_t>(p.h_kv) * p.d;
  const int nqv = kPbWaves * g;
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
    // P and dS of this row's heads into [key][qv]
    if (col_ok) {
#pragma unroll
      for (int x = 0; x < 8; ++x) {
        const int key = 16 * (x >> 2) + 4 * q4 + (x & 3);
        pall[0][key][wave * g + c16] = pr[x];
        pall[1][key][wave * g + c16] = ds[x];
      }
    }
    __syncthreads();
    // dV = P^T dO (pass 0) and dK = dS^T Q (pass 1), summed over the block's
    // query vectors: item (pass, dt) by wave item % kPbWaves
    for (int item = wave; item < 2 * NT; item += kPbWaves) {
      const int pass = item / NT, dt = item - pass * NT;
      const int which = pass == 0 ? 1 : 0;  // B: dO for dV, Q for dK
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        floatx4_t c = {0.f, 0.f, 0.f, 0.f};
        for (int kq = 0; kq < kblocks; ++kq) {
          const float* src = &pall[pass][16 * t + c16][32 * kq + 8 * q4];
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
          const bf16x8_t bop = *reinterpret_cast<const bf16x8_t*>(&qall[which][16 * dt + c16][32 * kq + 8 * q4]);
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
  float* dqb = p.dq + ((bb * p.n + i) * p.h_q + h * g + c16) * p.d + 4 * q4;
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
// g <= 8, q and dO rows 16-byte aligned, and K/V rows addressable by 32-bit
// buffer offsets (rows below 2^31 bytes, n and byte strides below 2^24).
bool bwd_mfma_ok(const BwdParams& p, const void* q, const void* dout) {
  const auto fits = [&](int64_t sn) {
    return sn >= 0 && 2 * sn < (int64_t(1) << 24) && (p.n - 1) * sn * 2 + 2 * p.d < (int64_t(1) << 31);
  };
  const bool aligned = (p.q_sb % 8 == 0) && (p.q_sn % 8 == 0) && (p.q_sh % 8 == 0) &&
                       (p.do_sb % 8 == 0) && (p.do_sn % 8 == 0) && (p.do_sh % 8 == 0) &&
                       (reinterpret_cast<uintptr_t>(q) % 16 == 0) && (reinterpret_cast<uintptr_t>(dout) % 16 == 0);
  return p.do_bf16 && (p.d == 64 || p.d == 128) && p.g <= 8 && aligned && p.n < (int64_t(1) << 24) &&
         fits(p.k_sn) && fits(p.v_sn);
}

template <typename T>
int launch_bwd(const BwdParams& p, hipStream_t st) {
  if constexpr (sizeof(T) == 2) {
    if (bwd_mfma_ok(p, p.q, p.dout)) {
      const dim3 grid(static_cast<unsigned>(ceil_div(p.rows, kBwMfWaves)));
      if (p.d == 64)
        sparse_attention_bwd_mfma_kernel<64><<<grid, 64 * kBwMfWaves, 0, st>>>(p);
      else
        sparse_attention_bwd_mfma_kernel<128><<<grid, 64 * kBwMfWaves, 0, st>>>(p);
      if (int s = check_launch("sparse_attention_bwd_mfma_kernel")) return s;
      if (!p.pfx) return SSA_OK;
      const dim3 pgrid(static_cast<unsigned>(kXcds * xcd_per((p.rows / p.n) * ceil_div(p.n, kPbWaves))));
      if (p.d == 64)
        prefix_attention_bwd_kernel<64><<<pgrid, 64 * kPbWaves, 0, st>>>(p);
      else
        prefix_attention_bwd_kernel<128><<<pgrid, 64 * kPbWaves, 0, st>>>(p);
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
    float* dq, float* dk, float* dv, int32_t* error_flag, const int32_t* row_prefix, void* workspace,
    size_t workspace_bytes, void* stream) {
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
  if (batch == 0 || n == 0) return SSA_OK;
  if (!q || !k || !v || !out || !dout || !dq || !dk || !dv || (top_k > 0 && !idx))
    return fail(SSA_ERR_INVALID_ARGUMENT, "sparse_attention_backward: null pointer");
  BwdParams p{};
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
  if (row_prefix && workspace) {
    const size_t need = bwd_ws_bytes(dtype, dout_dtype, batch, n, h_q, h_kv, d);
    if (workspace_bytes < need)
      return fail(SSA_ERR_WORKSPACE, "sparse_attention_backward: workspace %zu < %zu bytes", workspace_bytes, need);
    if (need > 0 && dtype == SSA_DTYPE_BF16 && bwd_mfma_ok(p, q, dout)) {
      p.pfx = row_prefix;
      p.pstats = static_cast<float*>(workspace);
    }
  }
  hipStream_t st = as_stream(stream);
  // dk and dv accumulate; dq rows are written whole by the row that owns them
  const int64_t kv_elems = batch * n * h_kv * d;
  zero_f32_kernel<<<dim3(static_cast<unsigned>(ceil_div(kv_elems, 256))), 256, 0, st>>>(dk, kv_elems);
  zero_f32_kernel<<<dim3(static_cast<unsigned>(ceil_div(kv_elems, 256))), 256, 0, st>>>(dv, kv_elems);
  if (int s = check_launch("zero_f32_kernel")) return s;
  if (dtype == SSA_DTYPE_BF16) return launch_bwd<uint16_t>(p, st);
  return launch_bwd<float>(p, st);
}
