// Stage (d): gathered-KV exact attention (sparse_exact_attention,
// ssa/attention.py:12-115).
//
// One wave per (batch, kv head h, query i); the g = h_q/h_kv query heads of
// the group share the row's k gathered keys.  Keys stream in chunks of 64:
//   * Q.K^T on the matrix cores: A = the group's q rows (heads padded to 16),
//     B = 16 gathered K rows per MFMA, loaded straight from HBM into the B
//     fragment (each lane reads 16 contiguous bytes of one K row);
//   * online softmax in the exp2 domain (running max / sum per head);
//   * P.V on the vector ALUs: every lane owns d/64 feature columns, each
//     gathered V row is one coalesced wave-wide load, and the chunk's
//     probabilities are broadcast from LDS.
// `scale_div` is the reference's `scale` (a divisor).  Duplicated indices count
// twice, as in the reference.
#include "ssa_common.h"

namespace ssa {
namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float floatx4_t __attribute__((ext_vector_type(4)));

constexpr int kAttWaves = 4;
constexpr int kAttThreads = 64 * kAttWaves;
constexpr int kChunk = 64;

struct AttParams {
  const void* q;
  const void* k;
  const void* v;
  int64_t n;
  int h_q, h_kv, g;
  int64_t q_sb, q_sn, q_sh, k_sb, k_sn, k_sh, v_sb, v_sn, v_sh;
  const void* idx;
  int idx_i64, top_k;
  int64_t idx_sb, idx_sn, idx_sh;
  float qk_scale_log2;  // log2(e) / scale_div
  int causal;
  void* out;
  int out_bf16;
  int64_t o_sb, o_sn, o_sh;
  int32_t* err;
  int64_t rows;
};

__device__ __forceinline__ uint16_t f32_to_bf16_rne(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7F800000u) == 0x7F800000u && (u & 0x007FFFFFu)) return static_cast<uint16_t>((u >> 16) | 0x40u);
  u += 0x7FFFu + ((u >> 16) & 1u);
  return static_cast<uint16_t>(u >> 16);
}

template <int DPL>
__device__ __forceinline__ void load_cols(const uint16_t* p, float* o) {
  if constexpr (DPL == 1) {
    o[0] = bf16_bits_to_f32(*p);
  } else if constexpr (DPL == 2) {
    const uint32_t u = *reinterpret_cast<const uint32_t*>(p);
    o[0] = __uint_as_float(u << 16);
    o[1] = __uint_as_float(u & 0xFFFF0000u);
  } else {
    const uint2 u = *reinterpret_cast<const uint2*>(p);
    o[0] = __uint_as_float(u.x << 16);
    o[1] = __uint_as_float(u.x & 0xFFFF0000u);
    o[2] = __uint_as_float(u.y << 16);
    o[3] = __uint_as_float(u.y & 0xFFFF0000u);
  }
}

template <int DPL>
__device__ __forceinline__ void load_cols(const float* p, float* o) {
  if constexpr (DPL == 1) {
    o[0] = *p;
  } else if constexpr (DPL == 2) {
    const float2 u = *reinterpret_cast<const float2*>(p);
    o[0] = u.x;
    o[1] = u.y;
  } else {
    const float4 u = *reinterpret_cast<const float4*>(p);
    o[0] = u.x; o[1] = u.y; o[2] = u.z; o[3] = u.w;
  }
}

__device__ __forceinline__ float max16(float x) {
  x = fmaxf(x, __shfl_xor(x, 8, 16));
  x = fmaxf(x, __shfl_xor(x, 4, 16));
  x = fmaxf(x, __shfl_xor(x, 2, 16));
  x = fmaxf(x, __shfl_xor(x, 1, 16));
  return x;
}

__device__ __forceinline__ float sum16(float x) {
  x += __shfl_xor(x, 8, 16);
  x += __shfl_xor(x, 4, 16);
  x += __shfl_xor(x, 2, 16);
  x += __shfl_xor(x, 1, 16);
  return x;
}

// bf16: KB = D/32 MFMA k-blocks of 32 dims, fragment = 8 bf16 per lane.
// f32 : KB = D/16 blocks of 16 dims, fragment = 4 floats per lane, each block
//       issued as four 16x16x4 MFMAs (lane group q4 covers dims 4*q4 .. 4*q4+3).
template <typename T, int D>
struct QkFrag;

template <int D>
struct QkFrag<uint16_t, D> {
  static constexpr int KB = D / 32;
  bf16x8_t a[KB];
  __device__ void load_q(const uint16_t* qh, bool ok, int q4) {
#pragma unroll
    for (int kb = 0; kb < KB; ++kb) {
      if (ok) a[kb] = *reinterpret_cast<const bf16x8_t*>(qh + kb * 32 + q4 * 8);
      else a[kb] = bf16x8_t{};
    }
  }
  __device__ floatx4_t dot(const uint16_t* kr, int q4) const {
    floatx4_t acc = {0.f, 0.f, 0.f, 0.f};
    bf16x8_t bv[KB];
#pragma unroll
    for (int kb = 0; kb < KB; ++kb) bv[kb] = *reinterpret_cast<const bf16x8_t*>(kr + kb * 32 + q4 * 8);
#pragma unroll
    for (int kb = 0; kb < KB; ++kb) acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[kb], bv[kb], acc, 0, 0, 0);
    return acc;
  }
};

template <int D>
struct QkFrag<float, D> {
  static constexpr int KB = D / 16;
  float4 a[KB];
  __device__ void load_q(const float* qh, bool ok, int q4) {
#pragma unroll
    for (int kb = 0; kb < KB; ++kb) {
      if (ok) a[kb] = *reinterpret_cast<const float4*>(qh + kb * 16 + q4 * 4);
      else a[kb] = make_float4(0.f, 0.f, 0.f, 0.f);
    }
  }
  __device__ floatx4_t dot(const float* kr, int q4) const {
    floatx4_t acc = {0.f, 0.f, 0.f, 0.f};
    float4 bv[KB];
#pragma unroll
    for (int kb = 0; kb < KB; ++kb) bv[kb] = *reinterpret_cast<const float4*>(kr + kb * 16 + q4 * 4);
#pragma unroll
    for (int kb = 0; kb < KB; ++kb) {
      acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a[kb].x, bv[kb].x, acc, 0, 0, 0);
      acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a[kb].y, bv[kb].y, acc, 0, 0, 0);
      acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a[kb].z, bv[kb].z, acc, 0, 0, 0);
      acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a[kb].w, bv[kb].w, acc, 0, 0, 0);
    }
    return acc;
  }
};

template <typename T, int D, int GMAX>
__global__ __launch_bounds__(kAttThreads) void sparse_attention_kernel(AttParams p) {
  constexpr int DPL = D / 64;
  __shared__ float Ps[kAttWaves][kChunk * GMAX];
  __shared__ float alpha_s[kAttWaves][GMAX];
  __shared__ float lsum_s[kAttWaves][GMAX];

  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  const int q4 = lane >> 4;
  const int c16 = lane & 15;
  const int64_t row = static_cast<int64_t>(blockIdx.x) * kAttWaves + wave;  // (b*h_kv + h)*n + i
  const bool row_ok = row < p.rows;
  const int64_t rr = row_ok ? row : 0;
  const int64_t i = rr % p.n;
  const int64_t bh = rr / p.n;
  const int h = static_cast<int>(bh % p.h_kv);
  const int64_t bb = bh / p.h_kv;

  const T* qh = static_cast<const T*>(p.q) + bb * p.q_sb + i * p.q_sn +
                static_cast<int64_t>(h * p.g + (c16 < p.g ? c16 : 0)) * p.q_sh;
  QkFrag<T, D> frag;
  frag.load_q(qh, row_ok && c16 < p.g, q4);

  const T* kbase = static_cast<const T*>(p.k) + bb * p.k_sb + static_cast<int64_t>(h) * p.k_sh;
  const T* vbase = static_cast<const T*>(p.v) + bb * p.v_sb + static_cast<int64_t>(h) * p.v_sh + lane * DPL;
  const int64_t ibase = bb * p.idx_sb + i * p.idx_sn + static_cast<int64_t>(h) * p.idx_sh;

  float m_run[4], l_run[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    m_run[e] = -INFINITY;
    l_run[e] = 0.0f;
  }
  float oacc[GMAX][DPL];
#pragma unroll
  for (int gg = 0; gg < GMAX; ++gg)
#pragma unroll
    for (int e = 0; e < DPL; ++e) oacc[gg][e] = 0.0f;

  const int nchunks = (p.top_k + kChunk - 1) / kChunk;
  for (int ch = 0; ch < nchunks; ++ch) {
    const int slot = ch * kChunk + lane;
    bool ok = row_ok && slot < p.top_k;
    int64_t j = 0;
    if (ok) {
      j = p.idx_i64 ? static_cast<const int64_t*>(p.idx)[ibase + slot]
                    : static_cast<int64_t>(static_cast<const int32_t*>(p.idx)[ibase + slot]);
      if (j < 0 || j >= p.n) {
        ok = false;
        if (p.err) p.err[0] = 1;
      } else if (p.causal && j > i) {
        ok = false;
      }
    }
    const int jsafe = ok ? static_cast<int>(j) : 0;
    const uint64_t okbits = __ballot(ok);

    float st[4][4];
#pragma unroll
    for (int tile = 0; tile < 4; ++tile) {
      const int src = tile * 16 + c16;
      const int jt = __shfl(jsafe, src);
      const bool okt = (okbits >> src) & 1ull;
      floatx4_t s = {0.f, 0.f, 0.f, 0.f};
      if ((okbits >> (tile * 16)) & 0xFFFFull) s = frag.dot(kbase + static_cast<int64_t>(jt) * p.k_sn, q4);
#pragma unroll
      for (int e = 0; e < 4; ++e) st[tile][e] = okt ? s[e] * p.qk_scale_log2 : -INFINITY;
    }

#pragma unroll
    for (int e = 0; e < 4; ++e) {
      float mx = fmaxf(fmaxf(st[0][e], st[1][e]), fmaxf(st[2][e], st[3][e]));
      mx = max16(mx);
      const float mnew = fmaxf(m_run[e], mx);
      const bool dead = (mnew == -INFINITY);
      const float alpha = dead ? 1.0f : exp2f(m_run[e] - mnew);
      m_run[e] = mnew;
      float ps = 0.0f;
      const int head = 4 * q4 + e;
#pragma unroll
      for (int tile = 0; tile < 4; ++tile) {
        const float pv = dead ? 0.0f : exp2f(st[tile][e] - mnew);
        ps += pv;
        if (head < GMAX) Ps[wave][(tile * 16 + c16) * GMAX + head] = pv;
      }
      l_run[e] = l_run[e] * alpha + ps;
      if (c16 == 0 && head < GMAX) alpha_s[wave][head] = alpha;
    }
    __syncthreads();

    float al[GMAX];
#pragma unroll
    for (int gg = 0; gg < GMAX; ++gg) al[gg] = alpha_s[wave][gg];
#pragma unroll
    for (int gg = 0; gg < GMAX; ++gg)
#pragma unroll
      for (int e = 0; e < DPL; ++e) oacc[gg][e] *= al[gg];

    for (int kk = 0; kk < kChunk; ++kk) {
      if (!((okbits >> kk) & 1ull)) continue;
      const int jk = __builtin_amdgcn_readlane(jsafe, kk);
      float vv[DPL];
      load_cols<DPL>(vbase + static_cast<int64_t>(jk) * p.v_sn, vv);
      const float* pr = &Ps[wave][kk * GMAX];
#pragma unroll
      for (int gg = 0; gg < GMAX; ++gg) {
        const float pg = pr[gg];
#pragma unroll
        for (int e = 0; e < DPL; ++e) oacc[gg][e] = fma_rn(pg, vv[e], oacc[gg][e]);
      }
    }
    __syncthreads();
  }

#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const float lt = sum16(l_run[e]);
    const int head = 4 * q4 + e;
    if (c16 == 0 && head < GMAX) lsum_s[wave][head] = lt;
  }
  __syncthreads();
  if (!row_ok) return;
#pragma unroll
  for (int gg = 0; gg < GMAX; ++gg) {
    if (gg >= p.g) continue;
    const float ls = lsum_s[wave][gg];
    const float inv = ls > 0.0f ? 1.0f / ls : 0.0f;
    const int64_t ob = bb * p.o_sb + i * p.o_sn + static_cast<int64_t>(h * p.g + gg) * p.o_sh + lane * DPL;
#pragma unroll
    for (int e = 0; e < DPL; ++e) {
      const float o = oacc[gg][e] * inv;
      if (p.out_bf16) static_cast<uint16_t*>(p.out)[ob + e] = f32_to_bf16_rne(o);
      else static_cast<float*>(p.out)[ob + e] = o;
    }
  }
}

template <typename T, int D>
int launch_att_d(const AttParams& p, hipStream_t st) {
  const int64_t blocks = ceil_div(p.rows, kAttWaves);
  if (p.g <= 4) sparse_attention_kernel<T, D, 4><<<dim3(static_cast<unsigned>(blocks)), kAttThreads, 0, st>>>(p);
  else if (p.g <= 8) sparse_attention_kernel<T, D, 8><<<dim3(static_cast<unsigned>(blocks)), kAttThreads, 0, st>>>(p);
  else sparse_attention_kernel<T, D, 16><<<dim3(static_cast<unsigned>(blocks)), kAttThreads, 0, st>>>(p);
  return check_launch("sparse_attention_kernel");
}

template <typename T>
int launch_att(const AttParams& p, int d, hipStream_t st) {
  switch (d) {
    case 64: return launch_att_d<T, 64>(p, st);
    case 128: return launch_att_d<T, 128>(p, st);
    default: return launch_att_d<T, 256>(p, st);
  }
}

}  // namespace
}  // namespace ssa

using namespace ssa;

extern "C" int ssa_sparse_attention(const void* q, const void* k, const void* v, int dtype,
                                    int64_t batch, int64_t n, int h_q, int h_kv, int d,
                                    int64_t q_sb, int64_t q_sn, int64_t q_sh, int64_t k_sb,
                                    int64_t k_sn, int64_t k_sh, int64_t v_sb, int64_t v_sn,
                                    int64_t v_sh, const void* idx, int idx_dtype, int top_k,
                                    int64_t idx_sb, int64_t idx_sn, int64_t idx_sh,
                                    float scale_div, int causal, void* out, int out_dtype,
                                    int64_t o_sb, int64_t o_sn, int64_t o_sh, int32_t* error_flag,
                                    void* stream) {
  if (dtype != SSA_DTYPE_F32 && dtype != SSA_DTYPE_BF16)
    return fail(SSA_ERR_UNSUPPORTED, "sparse_attention: dtype %d not supported (f32, bf16)", dtype);
  if (out_dtype != SSA_DTYPE_F32 && out_dtype != SSA_DTYPE_BF16)
    return fail(SSA_ERR_UNSUPPORTED, "sparse_attention: out dtype %d not supported", out_dtype);
  if (idx_dtype != SSA_INDEX_I32 && idx_dtype != SSA_INDEX_I64)
    return fail(SSA_ERR_INVALID_ARGUMENT, "sparse_attention: idx dtype %d", idx_dtype);
  if (batch < 0 || n < 0 || h_q <= 0 || h_kv <= 0 || top_k < 0)
    return fail(SSA_ERR_INVALID_ARGUMENT, "sparse_attention: bad shape");
  if (h_q % h_kv != 0)
    return fail(SSA_ERR_INVALID_ARGUMENT, "num_q_heads must be divisible by num_kv_heads");
  if (h_q / h_kv > 16)
    return fail(SSA_ERR_UNSUPPORTED, "sparse_attention: group size %d > 16", h_q / h_kv);
  if (d != 64 && d != 128 && d != 256)
    return fail(SSA_ERR_UNSUPPORTED, "sparse_attention: head_dim %d not in {64, 128, 256}", d);
  if (!(scale_div > 0.0f) && !(scale_div < 0.0f))
    return fail(SSA_ERR_INVALID_ARGUMENT, "sparse_attention: scale must be non-zero");
  const int vec = (dtype == SSA_DTYPE_BF16) ? 8 : 4;
  if ((q_sb % vec) || (q_sn % vec) || (q_sh % vec) || (k_sb % vec) || (k_sn % vec) ||
      (k_sh % vec) || (reinterpret_cast<uintptr_t>(q) % 16) || (reinterpret_cast<uintptr_t>(k) % 16))
    return fail(SSA_ERR_UNSUPPORTED, "sparse_attention: q/k rows must be 16-byte aligned");
  const int esz = (dtype == SSA_DTYPE_BF16) ? 2 : 4;
  const int dpl_bytes = esz * (d / 64);
  if (((v_sb * esz) % dpl_bytes) || ((v_sn * esz) % dpl_bytes) || ((v_sh * esz) % dpl_bytes) ||
      (reinterpret_cast<uintptr_t>(v) % dpl_bytes))
    return fail(SSA_ERR_UNSUPPORTED, "sparse_attention: v rows misaligned");
  if (batch == 0 || n == 0) return SSA_OK;
  if (!q || !k || !v || !out || (top_k > 0 && !idx))
    return fail(SSA_ERR_INVALID_ARGUMENT, "sparse_attention: null pointer");
  AttParams p{};
  p.q = q;
  p.k = k;
  p.v = v;
  p.n = n;
  p.h_q = h_q;
  p.h_kv = h_kv;
  p.g = h_q / h_kv;
  p.q_sb = q_sb; p.q_sn = q_sn; p.q_sh = q_sh;
  p.k_sb = k_sb; p.k_sn = k_sn; p.k_sh = k_sh;
  p.v_sb = v_sb; p.v_sn = v_sn; p.v_sh = v_sh;
  p.idx = idx;
  p.idx_i64 = (idx_dtype == SSA_INDEX_I64);
  p.top_k = top_k;
  p.idx_sb = idx_sb; p.idx_sn = idx_sn; p.idx_sh = idx_sh;
  p.qk_scale_log2 = static_cast<float>(1.4426950408889634 / static_cast<double>(scale_div));
  p.causal = causal ? 1 : 0;
  p.out = out;
  p.out_bf16 = (out_dtype == SSA_DTYPE_BF16);
  p.o_sb = o_sb; p.o_sn = o_sn; p.o_sh = o_sh;
  p.err = error_flag;
  p.rows = batch * h_kv * n;
  if (ceil_div(p.rows, kAttWaves) >= (int64_t(1) << 31))
    return fail(SSA_ERR_UNSUPPORTED, "sparse_attention: too many rows");
  hipStream_t st = as_stream(stream);
  if (dtype == SSA_DTYPE_BF16) return launch_att<uint16_t>(p, d, st);
  return launch_att<float>(p, d, st);
}
