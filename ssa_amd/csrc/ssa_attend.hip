// Stage (d): gathered-KV exact attention (sparse_exact_attention,
// ssa/attention.py:12-115).
//
// One wave per (batch, kv head h, query i); the g = h_q/h_kv query heads of
// the group share the row's k gathered keys.  Keys stream in chunks of 64:
//   * Q.K^T on the matrix cores: A = the group's q rows (heads padded to 16),
//     B = 16 gathered K rows per MFMA, loaded straight from HBM into the B
//     fragment (each lane reads 16 contiguous bytes of one K row);
//   * online softmax in the exp2 domain (running max / sum per head);
//   * P.V on the vector ALUs: each lane owns d/16 feature columns of a quarter
//     of the chunk's keys, so one wave-wide load moves four whole V rows; the
//     chunk's probabilities are broadcast from LDS.
// `scale_div` is the reference's `scale` (a divisor).  Duplicated indices count
// twice, as in the reference.
#include "ssa_common.h"

namespace ssa {
namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float floatx4_t __attribute__((ext_vector_type(4)));

constexpr int kAttWaves = 4;
constexpr int kAttThreads = 64 * kAttWaves;
// 16-key MFMA tiles per chunk: 2 (32 keys) measured fastest against 1 and 4 at
// the headline shape (4 needs more registers than 3 blocks per CU leave).
constexpr int kTiles = 2;

// Blocks per CU the compiler must fit: 3 (12 waves/CU) for the bf16 d<=128 g<=4
// variants, where it fits the registers without spilling and measured fastest
// (32-key chunks: 5.84 ms vs 6.21 ms at 2 blocks on the c3 workload); 1 (the
// compiler's own choice) elsewhere.
template <typename T, int D, int GMAX>
struct AttMinBlocks {
  static constexpr int value = (sizeof(T) == 2 && D <= 128 && GMAX <= 4) ? 3 : 1;
};
constexpr int kChunk = 16 * kTiles;  // selected keys per chunk

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
  struct BFrag {
    bf16x8_t v[KB];
  };
  __device__ void load_k(BFrag& f, const uint16_t* kr, int q4) const {
#pragma unroll
    for (int kb = 0; kb < KB; ++kb) f.v[kb] = *reinterpret_cast<const bf16x8_t*>(kr + kb * 32 + q4 * 8);
  }
  __device__ floatx4_t dot(const BFrag& f, int q4) const {
    (void)q4;
    floatx4_t acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int kb = 0; kb < KB; ++kb) acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[kb], f.v[kb], acc, 0, 0, 0);
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
  struct BFrag {
    float4 v[KB];
  };
  __device__ void load_k(BFrag& f, const float* kr, int q4) const {
#pragma unroll
    for (int kb = 0; kb < KB; ++kb) f.v[kb] = *reinterpret_cast<const float4*>(kr + kb * 16 + q4 * 4);
  }
  __device__ floatx4_t dot(const BFrag& f, int q4) const {
    (void)q4;
    floatx4_t acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int kb = 0; kb < KB; ++kb) {
      acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a[kb].x, f.v[kb].x, acc, 0, 0, 0);
      acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a[kb].y, f.v[kb].y, acc, 0, 0, 0);
      acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a[kb].z, f.v[kb].z, acc, 0, 0, 0);
      acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a[kb].w, f.v[kb].w, acc, 0, 0, 0);
    }
    return acc;
  }
};

// V slice of one key owned by a lane in P.V: DQ = D/16 consecutive features.
template <typename T, int DQ>
struct VSlice {
  static constexpr int BYTES = DQ * static_cast<int>(sizeof(T));
  static constexpr int WORDS = BYTES / 4;
  uint32_t w[WORDS];
  __device__ __forceinline__ void load(const T* ptr) {
    if constexpr (BYTES % 16 == 0) {
#pragma unroll
      for (int i = 0; i < BYTES / 16; ++i) {
        const uint4 u = reinterpret_cast<const uint4*>(ptr)[i];
        w[4 * i] = u.x; w[4 * i + 1] = u.y; w[4 * i + 2] = u.z; w[4 * i + 3] = u.w;
      }
    } else {
      const uint2 u = *reinterpret_cast<const uint2*>(ptr);
      w[0] = u.x; w[1] = u.y;
    }
  }
  __device__ __forceinline__ float at(int e) const {
    if constexpr (sizeof(T) == 2) {
      const uint32_t x = w[e >> 1];
      return __uint_as_float((e & 1) ? (x & 0xFFFF0000u) : (x << 16));
    } else {
      return __uint_as_float(w[e]);
    }
  }
};

// LDS hand-off between lanes of one wave (each wave owns its LDS slices).
__device__ __forceinline__ void wave_lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
}

// Per chunk of kChunk selected keys (lanes < kChunk load the indices):
//   K: kTiles tiles of 16 keys; lane (q4, c16) loads 16 B of key tile*16+c16
//      per 32-dim block straight into the MFMA B fragment;
//   V: lane (q4, c16) owns features c16*DQ .. +DQ of keys 4r+q4, r < kChunk/4,
//      so each wave-wide load moves four whole V rows;
//   K and V loads of a chunk are issued together, with the next chunk's
//   indices, before any of them is consumed.
// P goes through LDS ([key][head]); the 4 lane quarters hold partial P.V sums
// over disjoint keys and are added once per row.
template <typename T, int D, int GMAX>
__global__ __launch_bounds__(kAttThreads, (AttMinBlocks<T, D, GMAX>::value)) void sparse_attention_kernel(AttParams p) {
  constexpr int DQ = D / 16;
  using VS = VSlice<T, DQ>;
  constexpr int KPL = kChunk / 4;  // keys per lane quarter per chunk
  constexpr int KPB = (VS::BYTES <= 16) ? KPL : (VS::BYTES <= 32 ? KPL / 2 : KPL / 4);  // keys per V batch
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
  const T* vbase = static_cast<const T*>(p.v) + bb * p.v_sb + static_cast<int64_t>(h) * p.v_sh + c16 * DQ;
  const int64_t ibase = bb * p.idx_sb + i * p.idx_sn + static_cast<int64_t>(h) * p.idx_sh;

  // Index of this lane's slot in chunk ch, range-checked on load: -1 = no slot,
  // -2 = outside [0, n) (reported through the error flag).
  auto load_idx = [&](int ch) -> int {
    const int slot = ch * kChunk + lane;
    if (!row_ok || lane >= kChunk || slot >= p.top_k) return -1;
    const int64_t j = p.idx_i64 ? static_cast<const int64_t*>(p.idx)[ibase + slot]
                                : static_cast<int64_t>(static_cast<const int32_t*>(p.idx)[ibase + slot]);
    if (j < 0 || j >= p.n) {
      if (p.err) p.err[0] = 1;
      return -2;
    }
    return static_cast<int>(j);
  };

  float m_run[4], l_run[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    m_run[e] = -INFINITY;
    l_run[e] = 0.0f;
  }
  float oacc[GMAX][DQ];
#pragma unroll
  for (int gg = 0; gg < GMAX; ++gg)
#pragma unroll
    for (int e = 0; e < DQ; ++e) oacc[gg][e] = 0.0f;

  const int nchunks = (p.top_k + kChunk - 1) / kChunk;
  int j_next = (nchunks > 0) ? load_idx(0) : -1;
  for (int ch = 0; ch < nchunks; ++ch) {
    const int j = j_next;
    const bool ok = j >= 0 && !(p.causal && j > i);
    const int jsafe = ok ? j : 0;
    const uint64_t okbits = __ballot(ok);

    // Issue K (4 tiles) and the first V batch, then the next chunk's indices.
    typename QkFrag<T, D>::BFrag kf[kTiles];
#pragma unroll
    for (int tile = 0; tile < kTiles; ++tile) {
      const int jt = __shfl(jsafe, tile * 16 + c16);
      if ((okbits >> (tile * 16)) & 0xFFFFull) frag.load_k(kf[tile], kbase + static_cast<int64_t>(jt) * p.k_sn, q4);
    }
    VS vv[KPB];
#pragma unroll
    for (int r = 0; r < KPB; ++r) {
      const int jv = __shfl(jsafe, 4 * r + q4);
      vv[r].load(vbase + static_cast<int64_t>(jv) * p.v_sn);
    }
    if (ch + 1 < nchunks) j_next = load_idx(ch + 1);

    float st[kTiles][4];
#pragma unroll
    for (int tile = 0; tile < kTiles; ++tile) {
      const int src = tile * 16 + c16;
      const bool okt = (okbits >> src) & 1ull;
      floatx4_t sc = {0.f, 0.f, 0.f, 0.f};
      if ((okbits >> (tile * 16)) & 0xFFFFull) sc = frag.dot(kf[tile], q4);
#pragma unroll
      for (int e = 0; e < 4; ++e) st[tile][e] = okt ? sc[e] * p.qk_scale_log2 : -INFINITY;
    }

#pragma unroll
    for (int e = 0; e < 4; ++e) {
      float mx = st[0][e];
#pragma unroll
      for (int tile = 1; tile < kTiles; ++tile) mx = fmaxf(mx, st[tile][e]);
      mx = max16(mx);
      const float mnew = fmaxf(m_run[e], mx);
      const bool dead = (mnew == -INFINITY);
      const float alpha = dead ? 1.0f : exp2f(m_run[e] - mnew);
      m_run[e] = mnew;
      float ps = 0.0f;
      const int head = 4 * q4 + e;
#pragma unroll
      for (int tile = 0; tile < kTiles; ++tile) {
        const float pv = dead ? 0.0f : exp2f(st[tile][e] - mnew);
        ps += pv;
        if (head < GMAX) Ps[wave][(tile * 16 + c16) * GMAX + head] = pv;
      }
      l_run[e] = l_run[e] * alpha + ps;
      if (c16 == 0 && head < GMAX) alpha_s[wave][head] = alpha;
    }
    wave_lds_sync();

#pragma unroll
    for (int gg = 0; gg < GMAX; ++gg) {
      const float al = alpha_s[wave][gg];
#pragma unroll
      for (int e = 0; e < DQ; ++e) oacc[gg][e] *= al;
    }
#pragma unroll
    for (int b0 = 0; b0 < KPL; b0 += KPB) {
      if (b0 > 0) {
#pragma unroll
        for (int r = 0; r < KPB; ++r) {
          const int jv = __shfl(jsafe, 4 * (b0 + r) + q4);
          vv[r].load(vbase + static_cast<int64_t>(jv) * p.v_sn);
        }
      }
#pragma unroll
      for (int r = 0; r < KPB; ++r) {
        const float* pr = &Ps[wave][(4 * (b0 + r) + q4) * GMAX];
        float pk[GMAX];
#pragma unroll
        for (int gg = 0; gg < GMAX; ++gg) pk[gg] = pr[gg];
#pragma unroll
        for (int gg = 0; gg < GMAX; ++gg)
#pragma unroll
          for (int e = 0; e < DQ; ++e) oacc[gg][e] = fma_rn(pk[gg], vv[r].at(e), oacc[gg][e]);
      }
    }
    wave_lds_sync();
  }

  // Quarter partial sums -> full P.V in every lane of a column group.
#pragma unroll
  for (int gg = 0; gg < GMAX; ++gg)
#pragma unroll
    for (int e = 0; e < DQ; ++e) {
      float x = oacc[gg][e];
      x += __shfl_xor(x, 16);
      x += __shfl_xor(x, 32);
      oacc[gg][e] = x;
    }
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const float lt = sum16(l_run[e]);
    const int head = 4 * q4 + e;
    if (c16 == 0 && head < GMAX) lsum_s[wave][head] = lt;
  }
  wave_lds_sync();
  if (!row_ok) return;
  // Lane quarter q4 writes heads q4, q4 + 4, ...
  // Each lane stores DQ contiguous outputs with vector stores (DQ*2 or DQ*4 bytes).
#pragma unroll
  for (int gg = 0; gg < GMAX; ++gg) {
    if ((gg & 3) != q4 || gg >= p.g) continue;
    const float ls = lsum_s[wave][gg];
    const float inv = ls > 0.0f ? 1.0f / ls : 0.0f;
    const int64_t ob = bb * p.o_sb + i * p.o_sn + static_cast<int64_t>(h * p.g + gg) * p.o_sh + c16 * DQ;
    if (p.out_bf16) {
      uint32_t packed[DQ / 2];
#pragma unroll
      for (int e = 0; e < DQ / 2; ++e)
        packed[e] = static_cast<uint32_t>(f32_to_bf16_rne(oacc[gg][2 * e] * inv)) |
                    (static_cast<uint32_t>(f32_to_bf16_rne(oacc[gg][2 * e + 1] * inv)) << 16);
      uint16_t* dst = static_cast<uint16_t*>(p.out) + ob;
      if constexpr (DQ % 8 == 0) {
#pragma unroll
        for (int e = 0; e < DQ / 8; ++e)
          reinterpret_cast<uint4*>(dst)[e] = make_uint4(packed[4 * e], packed[4 * e + 1], packed[4 * e + 2], packed[4 * e + 3]);
      } else {
        reinterpret_cast<uint2*>(dst)[0] = make_uint2(packed[0], packed[1]);
      }
    } else {
      float* dst = static_cast<float*>(p.out) + ob;
#pragma unroll
      for (int e = 0; e < DQ / 4; ++e)
        reinterpret_cast<float4*>(dst)[e] = make_float4(oacc[gg][4 * e] * inv, oacc[gg][4 * e + 1] * inv,
                                                        oacc[gg][4 * e + 2] * inv, oacc[gg][4 * e + 3] * inv);
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
      (k_sh % vec) || (v_sb % vec) || (v_sn % vec) || (v_sh % vec) ||
      (reinterpret_cast<uintptr_t>(q) % 16) || (reinterpret_cast<uintptr_t>(k) % 16) ||
      (reinterpret_cast<uintptr_t>(v) % 16))
    return fail(SSA_ERR_UNSUPPORTED, "sparse_attention: q/k/v rows must be 16-byte aligned");
  if ((o_sb % vec) || (o_sn % vec) || (o_sh % vec) || (reinterpret_cast<uintptr_t>(out) % 16))
    return fail(SSA_ERR_UNSUPPORTED, "sparse_attention: output rows must be 16-byte aligned");
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
