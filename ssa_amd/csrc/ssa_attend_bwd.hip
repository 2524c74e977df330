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
  float inv_scale;  // 1 / scale_div
  int causal;
  float* dq;  // [B][n][h_q][d]
  float* dk;  // [B][n][h_kv][d]
  float* dv;  // [B][n][h_kv][d]
  int32_t* err;
  int64_t rows;
  const int32_t* order;  // nullable [B*h_kv][n]
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

template <typename T>
int launch_bwd(const BwdParams& p, hipStream_t st) {
  if (p.g <= 4) return launch_bwd_g<T, 4>(p, st);
  if (p.g <= 8) return launch_bwd_g<T, 8>(p, st);
  return launch_bwd_g<T, 16>(p, st);
}

}  // namespace
}  // namespace ssa

using namespace ssa;

extern "C" int ssa_sparse_attention_backward(
    const void* q, const void* k, const void* v, int dtype, int64_t batch, int64_t n, int h_q,
    int h_kv, int d, int64_t q_sb, int64_t q_sn, int64_t q_sh, int64_t k_sb, int64_t k_sn,
    int64_t k_sh, int64_t v_sb, int64_t v_sn, int64_t v_sh, const void* idx, int idx_dtype,
    int top_k, int64_t idx_sb, int64_t idx_sn, int64_t idx_sh, float scale_div, int causal,
    const int32_t* row_order, const void* out, int out_dtype, int64_t o_sb, int64_t o_sn,
    int64_t o_sh, const void* dout, int dout_dtype, int64_t do_sb, int64_t do_sn, int64_t do_sh,
    float* dq, float* dk, float* dv, int32_t* error_flag, void* stream) {
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
  p.causal = causal ? 1 : 0;
  p.dq = dq; p.dk = dk; p.dv = dv;
  p.err = error_flag;
  p.rows = batch * h_kv * n;
  p.order = row_order;
  if (p.rows >= (int64_t(1) << 31))
    return fail(SSA_ERR_UNSUPPORTED, "sparse_attention_backward: too many rows");
  hipStream_t st = as_stream(stream);
  // dk and dv accumulate; dq rows are written whole by the row that owns them
  const int64_t kv_elems = batch * n * h_kv * d;
  zero_f32_kernel<<<dim3(static_cast<unsigned>(ceil_div(kv_elems, 256))), 256, 0, st>>>(dk, kv_elems);
  zero_f32_kernel<<<dim3(static_cast<unsigned>(ceil_div(kv_elems, 256))), 256, 0, st>>>(dv, kv_elems);
  if (int s = check_launch("zero_f32_kernel")) return s;
  if (dtype == SSA_DTYPE_BF16) return launch_bwd<uint16_t>(p, st);
  return launch_bwd<float>(p, st);
}
