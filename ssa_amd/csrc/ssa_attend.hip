// Stage (d): gathered-KV exact attention (sparse_exact_attention,
// ssa/attention.py:12-115).
//
// One wave per (batch, kv head h, query i); the g = h_q/h_kv query heads of
// the group share the row's k gathered keys, which stream in chunks of 32 with
// an online softmax in the exp2 domain.  Two kernels:
//   * sparse_attention_mfma_kernel (bf16, g <= 8, d in {64, 128}): Q.K^T and
//     P.V both on the matrix cores (see the comment at the kernel);
//   * sparse_attention_kernel (fp32 inputs, g up to 16, any head dim that is a
//     multiple of 8 up to 256, padded to 32/64/128/256): Q.K^T on the matrix
//     cores, P.V on the vector ALUs in fp32 (each lane owns d/16 feature
//     columns of a quarter of the chunk's keys; P is broadcast from LDS).
// `scale_div` is the reference's `scale` (a divisor).  Duplicated indices count
// twice, as in the reference.
#include "ssa_common.h"
#include "ssa_internal.h"
#include "ssa_rows.h"

namespace ssa {
namespace {


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
  int d;  // head dim (<= the kernel's padded width D; dims >= d read as zero)
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
  const int32_t* order;  // nullable [B*h_kv][n_q]: query row processed at each slot
  int64_t n_q, q_pos0;   // query rows (q, idx, out) and the key position of row 0
  // Block mode (blk_log2 > 0): idx row qr >> blk_log2 holds key-block ids in
  // [0, nbk); key slot t of a row is key blk[t >> blk_log2] * 2^blk_log2 +
  // (t & (2^blk_log2 - 1)), and keys at or past n are dropped silently.
  int blk_log2;
  int64_t nbk;
  // Dense key prefix (nullable): pfx_x [B*h_kv][n_q] = X, the length of the
  // key prefix [0, X) that a row's indices hold exactly once, and pfx_part the
  // prefix's unnormalised attention state per (row, head): [B*h_kv*n_q][g][D + 4]
  // = O (D floats), running max, sum.  prefix_attention_kernel writes both; the
  // row kernel then drops the row's indices below X and starts from that state.
  int32_t* pfx_x;
  float* pfx_part;
  int pfx_given;  // pfx_x came from the selection (row_prefix): the prefix kernel only reads it
  // Nullable [B*h_kv*n_q][g][2]: the matrix-core row kernel leaves each (row,
  // head)'s softmax reference (running max, log2 units) and 1 / sum here, for
  // the backward; other paths write nothing.
  float* stats;
  // Matrix-core row kernel: wait for each chunk's gather right after issuing it
  // instead of computing the previous chunk meanwhile.  Set when a (batch, kv
  // head)'s K and V exceed kGatherWaitBytes but all heads' together fit the
  // 256 MB Infinity Cache: there the gathers come from past L2 but not from
  // HBM, and keeping one in flight during each chunk's MFMAs only adds
  // contention (c5, 64 MB per head and 128 MB in all: stage (d) 9.54 ms waiting
  // against 10.09 ms overlapped; n = 32768, 16 MB per head: 3.06 against 2.92
  // ms).  When they do not fit (n = 131072 with 8 kv heads, 512 MB), the
  // overlap hides HBM latency: 13.48 against 13.65 ms.
  int gather_wait;
};
constexpr int64_t kGatherWaitBytes = int64_t(32) << 20;
constexpr int64_t kInfinityCacheBytes = int64_t(256) << 20;

// Key of slot `slot` given the index entry loaded for it: -1 = none (block mode:
// past n), -2 = invalid index (reported through the error flag).
template <bool BLK>
__device__ __forceinline__ int att_key(const AttParams& p, int slot, int64_t jv) {
  if constexpr (!BLK) {
    if (jv < 0 || jv >= p.n) {
      if (p.err) p.err[0] = 1;
      return -2;
    }
    return static_cast<int>(jv);
  }
  if (jv < 0 || jv >= p.nbk) {
    if (p.err) p.err[0] = 1;
    return -2;
  }
  const int64_t j = (jv << p.blk_log2) + (slot & ((1 << p.blk_log2) - 1));
  return j < p.n ? static_cast<int>(j) : -1;
}

// att_key for a whole wave without divergent branches (the matrix-core row
// kernel): `use` marks the slots read; an invalid index among them raises the
// flag in a branch that only a wave holding one takes.
template <bool BLK>
__device__ __forceinline__ int att_key_wave(const AttParams& p, int slot, int64_t jv, bool use) {
  const bool bad = use && static_cast<uint64_t>(jv) >= static_cast<uint64_t>(BLK ? p.nbk : p.n);
  if (__ballot(bad) != 0ull && p.err != nullptr && bad) p.err[0] = 1;
  int key = static_cast<int>(jv);
  if constexpr (BLK) {
    const int64_t j = (jv << p.blk_log2) + (slot & ((1 << p.blk_log2) - 1));
    key = j < p.n ? static_cast<int>(j) : -1;
  }
  return !use ? -1 : bad ? -2 : key;
}

// Row processed by wave slot `lrow` (in (b*h_kv + h)*n_q + slot order): the query
// row r is the slot itself, or order[lrow] when a processing order is given; it
// sits at key position i = q_pos0 + r (the causal cut).  An order entry outside
// [0, n_q) drops the row and raises the error flag.
struct AttRow {
  int64_t r, i, bh;
  bool ok;
};
__device__ __forceinline__ AttRow att_row(const AttParams& p, int64_t lrow) {
  AttRow r;
  r.ok = lrow < p.rows;
  const int64_t l = r.ok ? lrow : 0;
  r.bh = udiv32(l, p.n_q);
  r.r = l - r.bh * p.n_q;
  if (p.order) {
    const int64_t o = p.order[l];
    if (o < 0 || o >= p.n_q) {
      if (r.ok && p.err) p.err[0] = 1;
      r.ok = false;
      r.r = 0;
    } else {
      r.r = o;
    }
  }
  r.i = p.q_pos0 + r.r;
  return r;
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
  __device__ void load_q(const uint16_t* qh, bool ok, int q4, int d) {
#pragma unroll
    for (int kb = 0; kb < KB; ++kb) {
      if (ok && kb * 32 + q4 * 8 < d) a[kb] = *reinterpret_cast<const bf16x8_t*>(qh + kb * 32 + q4 * 8);
      else a[kb] = bf16x8_t{};
    }
  }
  struct BFrag {
    bf16x8_t v[KB];
  };
  __device__ void load_k(BFrag& f, const uint16_t* kr, int q4, int d) const {
#pragma unroll
    for (int kb = 0; kb < KB; ++kb)
      f.v[kb] = (kb * 32 + q4 * 8 < d) ? *reinterpret_cast<const bf16x8_t*>(kr + kb * 32 + q4 * 8) : bf16x8_t{};
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
  __device__ void load_q(const float* qh, bool ok, int q4, int d) {
#pragma unroll
    for (int kb = 0; kb < KB; ++kb) {
      if (ok && kb * 16 + q4 * 4 < d) a[kb] = *reinterpret_cast<const float4*>(qh + kb * 16 + q4 * 4);
      else a[kb] = make_float4(0.f, 0.f, 0.f, 0.f);
    }
  }
  struct BFrag {
    float4 v[KB];
  };
  __device__ void load_k(BFrag& f, const float* kr, int q4, int d) const {
#pragma unroll
    for (int kb = 0; kb < KB; ++kb)
      f.v[kb] = (kb * 16 + q4 * 4 < d) ? *reinterpret_cast<const float4*>(kr + kb * 16 + q4 * 4)
                                       : make_float4(0.f, 0.f, 0.f, 0.f);
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
  // Only the first `nvalid` features exist (the head dim ends inside or before
  // this slice); the rest read as zero.  The head dim is a multiple of 8, so
  // each 16-byte piece is wholly inside or wholly outside it.
  __device__ __forceinline__ void load(const T* ptr, int nvalid) {
    if (nvalid <= 0) {
#pragma unroll
      for (int i = 0; i < WORDS; ++i) w[i] = 0u;
      return;
    }
    if constexpr (BYTES % 16 == 0) {
      constexpr int PE = 16 / static_cast<int>(sizeof(T));  // features per piece
#pragma unroll
      for (int i = 0; i < BYTES / 16; ++i) {
        const uint4 u = (i * PE < nvalid) ? reinterpret_cast<const uint4*>(ptr)[i] : make_uint4(0u, 0u, 0u, 0u);
        w[4 * i] = u.x; w[4 * i + 1] = u.y; w[4 * i + 2] = u.z; w[4 * i + 3] = u.w;
      }
    } else if constexpr (BYTES == 8) {
      const uint2 u = *reinterpret_cast<const uint2*>(ptr);
      w[0] = u.x; w[1] = u.y;
    } else {
      static_assert(BYTES == 4, "V slices are 4, 8 or a multiple of 16 bytes");
      w[0] = *reinterpret_cast<const uint32_t*>(ptr);
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
  const AttRow ar = att_row(p, static_cast<int64_t>(blockIdx.x) * kAttWaves + wave);
  const bool row_ok = ar.ok;
  const int64_t i = ar.i;  // key position (causal cut)
  const int64_t qr = ar.r;  // query row (q, idx, out)
  const int64_t bh = ar.bh;
  const int64_t bb = udiv32(bh, p.h_kv);
  const int h = static_cast<int>(bh - bb * p.h_kv);

  const T* qh = static_cast<const T*>(p.q) + bb * p.q_sb + qr * p.q_sn +
                static_cast<int64_t>(h * p.g + (c16 < p.g ? c16 : 0)) * p.q_sh;
  QkFrag<T, D> frag;
  frag.load_q(qh, row_ok && c16 < p.g, q4, p.d);
  const int vvalid = p.d - c16 * DQ;  // features of this lane's V / output slice that exist

  const T* kbase = static_cast<const T*>(p.k) + bb * p.k_sb + static_cast<int64_t>(h) * p.k_sh;
  const T* vbase = static_cast<const T*>(p.v) + bb * p.v_sb + static_cast<int64_t>(h) * p.v_sh + c16 * DQ;
  const int64_t ibase = bb * p.idx_sb + (qr >> p.blk_log2) * p.idx_sn + static_cast<int64_t>(h) * p.idx_sh;

  // Index of this lane's slot in chunk ch, range-checked on load: -1 = no slot,
  // -2 = outside [0, n) (reported through the error flag).
  auto load_idx = [&](int ch) -> int {
    const int slot = ch * kChunk + lane;
    if (!row_ok || lane >= kChunk || slot >= p.top_k) return -1;
    const int e = slot >> p.blk_log2;
    const int64_t jv = p.idx_i64 ? static_cast<const int64_t*>(p.idx)[ibase + e]
                                 : static_cast<int64_t>(static_cast<const int32_t*>(p.idx)[ibase + e]);
    return p.blk_log2 ? att_key<true>(p, slot, jv) : att_key<false>(p, slot, jv);
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
      if ((okbits >> (tile * 16)) & 0xFFFFull) frag.load_k(kf[tile], kbase + static_cast<int64_t>(jt) * p.k_sn, q4, p.d);
    }
    VS vv[KPB];
#pragma unroll
    for (int r = 0; r < KPB; ++r) {
      const int jv = __shfl(jsafe, 4 * r + q4);
      vv[r].load(vbase + static_cast<int64_t>(jv) * p.v_sn, vvalid);
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
          vv[r].load(vbase + static_cast<int64_t>(jv) * p.v_sn, vvalid);
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
    if ((gg & 3) != q4 || gg >= p.g || vvalid <= 0) continue;
    const float ls = lsum_s[wave][gg];
    const float inv = ls > 0.0f ? 1.0f / ls : 0.0f;
    const int64_t ob = bb * p.o_sb + qr * p.o_sn + static_cast<int64_t>(h * p.g + gg) * p.o_sh + c16 * DQ;
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
          if (e * 8 < vvalid)
            reinterpret_cast<uint4*>(dst)[e] = make_uint4(packed[4 * e], packed[4 * e + 1], packed[4 * e + 2], packed[4 * e + 3]);
      } else if constexpr (DQ == 4) {
        reinterpret_cast<uint2*>(dst)[0] = make_uint2(packed[0], packed[1]);
      } else {
        reinterpret_cast<uint32_t*>(dst)[0] = packed[0];
      }
    } else {
      float* dst = static_cast<float*>(p.out) + ob;
      if constexpr (DQ % 4 == 0) {
#pragma unroll
        for (int e = 0; e < DQ / 4; ++e)
          if (e * 4 < vvalid)
            reinterpret_cast<float4*>(dst)[e] = make_float4(oacc[gg][4 * e] * inv, oacc[gg][4 * e + 1] * inv,
                                                            oacc[gg][4 * e + 2] * inv, oacc[gg][4 * e + 3] * inv);
      } else {
        reinterpret_cast<float2*>(dst)[0] = make_float2(oacc[gg][0] * inv, oacc[gg][1] * inv);
      }
    }
  }
}

// ---- bf16, g <= 8, d <= 128: P.V on the matrix cores ----------------------
//
// Per chunk of 32 selected keys (one wave, one (batch, kv head, query) row):
//   gathers        K and V rows go straight to the wave's LDS slices with
//                  global_load_lds_dwordx4: each wave-wide load moves whole rows
//                  (1 KB = 4 rows at d = 128), the shape the texture path moves
//                  fastest (a load touching 16 rows x 64 B moves bytes about 3x
//                  slower from L2).  Row slots are XOR-swizzled (mf_swz) so the
//                  fragment reads below are free of bank conflicts;
//   pipelining     the chunk's fragments are read out of LDS, then the next
//                  chunk's loads are issued into the same slices and fly while
//                  this chunk computes;
//   S^T = K . Q^T  two 16x16x32 MFMA tiles per 32 dims: A = 16 K rows (lane
//                  (q4, c16): key 16t + c16, dims 8*q4 .. of each 32-dim block,
//                  one ds_read_b128), B = the group's q rows.  Lane (q4, c16)
//                  gets head c16's scores of keys 16t + 4*q4 + e;
//   softmax        online in the exp2 domain, per head, max and sum reduced
//                  across the four lanes that hold a head's keys;
//   P              split as P = P_hi + P_lo, both bf16 (relative error of the
//                  sum ~2^-17): head r's P_hi is row r and its P_lo row 8 + r of
//                  the 16-row P^T operand, so one MFMA covers both for g <= 8;
//   O^T += V^T P^T one 16x16x32 MFMA per 16 features: A = V^T, read with
//                  ds_read_b64_tr_b16 (each lane gets four rows of one feature
//                  column), B = P^T;
//   output         O = (row r + row 8 + r) / l, four contiguous features per lane
//                  and tile.
// Dropped slots (causal, past top_k, out of range) load zeros, so 0 * inf
// never reaches the sums.
// Waves per block and waves per SIMD of the matrix-core kernel.  Each wave keeps
// one chunk (16 KB at d = 128) of K and V in flight in its LDS slices, so the
// bytes in flight per CU are LDS-bound; the waves share nothing, so one-wave
// blocks let a CU hold 10 of them (160 KB) and start each as soon as one ends
// (c3 stage d: 3.90 ms against 4.04 with four-wave blocks, 3.95 with two).
// At least 2 waves per SIMD.  The d = 128 build needs 167 VGPRs (3 waves per
// SIMD), so the LDS's 10 waves per CU are the limit; forcing that bound while
// the build needed more cost 0.5 ms at c5 (spills) and gained nothing at c3.
constexpr int kMfWaves = 1;
constexpr int kMfMinWavesPerEu = 2;

// Issue one chunk's K and V loads: load r moves chunk rows KPI*r .. KPI*r +
// KPI - 1 into LDS at base + r KB, lane l fetching the segment of row KPI*r +
// l / SEGS that belongs in slot l % SEGS (seg16[r % SWZ_PERIOD], in bytes).
// jsafe (lanes < 32) is the chunk's key index per slot, negative for a dropped
// slot.  FULL: no dropped slot in the chunk; SAME: K and V share the row stride.
template <int D, bool FULL, bool SAME>
__device__ __forceinline__ void mf_issue(__amdgpu_buffer_rsrc_t krs, __amdgpu_buffer_rsrc_t vrs,
                                         unsigned char* kl, unsigned char* vl, int jsafe, int lrow,
                                         uint32_t ksn2, uint32_t vsn2,
                                         const uint32_t (&seg16)[MfShape<D>::SWZ_PERIOD]) {
  using S = MfShape<D>;
  int jr[S::NLD];
#pragma unroll
  for (int r = 0; r < S::NLD; ++r) jr[r] = __shfl(jsafe, S::KPI * r + lrow);
#pragma unroll
  for (int r = 0; r < S::NLD; ++r) {
    const uint32_t sg = seg16[r % S::SWZ_PERIOD];
    uint32_t ko = __umul24(static_cast<uint32_t>(jr[r]), ksn2) + sg;
    uint32_t vo = SAME ? ko : __umul24(static_cast<uint32_t>(jr[r]), vsn2) + sg;
    if (!FULL) {
      ko = jr[r] >= 0 ? ko : kOobOffset;
      vo = jr[r] >= 0 ? vo : kOobOffset;
    }
    __builtin_amdgcn_raw_ptr_buffer_load_lds(krs, (lds_void_ptr)(kl + r * 1024), 16, static_cast<int>(ko), 0, 0, 0);
    __builtin_amdgcn_raw_ptr_buffer_load_lds(vrs, (lds_void_ptr)(vl + r * 1024), 16, static_cast<int>(vo), 0, 0, 0);
  }
}

// One (batch, kv head, query) row on one wave, with the wave's LDS slices kl
// and vl (kMfChunk rows of K and of V each).  NSPLIT > 1: the wave takes only
// chunks c0, c0 + NSPLIT, ... and leaves its unnormalised state in `part`
// (O [8][D], the running max [8] and sum [8] per head) for a combine step.
template <int D, bool BLK, int NSPLIT = 1>
__device__ __forceinline__ void attend_row_mfma(const AttParams& p, const AttRow& ar, unsigned char* kl,
                                                unsigned char* vl, int c0 = 0, float* part = nullptr) {
  using S = MfShape<D>;
  const int lane = threadIdx.x & 63;
  const int q4 = lane >> 4;
  const int c16 = lane & 15;
  const bool row_ok = ar.ok;
  const int64_t i = ar.i;  // key position (causal cut)
  const int64_t qr = ar.r;  // query row (q, idx, out)
  const int64_t bh = ar.bh;
  const int64_t bb = udiv32(bh, p.h_kv);
  const int h = static_cast<int>(bh - bb * p.h_kv);

  const uint16_t* qh = static_cast<const uint16_t*>(p.q) + bb * p.q_sb + qr * p.q_sn +
                       static_cast<int64_t>(h * p.g + (c16 < p.g ? c16 : 0)) * p.q_sh;
  bf16x8_t qf[S::KB];
#pragma unroll
  for (int kb = 0; kb < S::KB; ++kb)
    qf[kb] = (row_ok && c16 < p.g) ? *reinterpret_cast<const bf16x8_t*>(qh + kb * 32 + q4 * 8)
                                   : bf16x8_t{};

  const uint16_t* kbase = static_cast<const uint16_t*>(p.k) + bb * p.k_sb + static_cast<int64_t>(h) * p.k_sh;
  const uint16_t* vbase = static_cast<const uint16_t*>(p.v) + bb * p.v_sb + static_cast<int64_t>(h) * p.v_sh;
  const int64_t ibase = bb * p.idx_sb + (BLK ? qr >> p.blk_log2 : qr) * p.idx_sn + static_cast<int64_t>(h) * p.idx_sh;

  // Index entry of slot l of chunk ch as loaded (int32 entries in the low
  // word, slot 0's entry where slot_at drops the slot), and its key (-1 past top_k,
  // l >= kMfChunk or on a dropped row).  Loading and checking apart keeps the
  // check's wait away from the load: a batch of index loads goes out before
  // the first check, and the next chunk's indices fly with its K/V gathers.
  // (two dword loads with no branch on the index type: the low word, and the
  // high word or, for int32 entries, the same word again; a branch here would
  // make the compiler wait for the load, and with it for the chunk's gathers)
  auto slot_at = [&](int ch, int l) { return row_ok && l < kMfChunk && ch * kMfChunk + l < p.top_k; };
  const int ewords = p.idx_i64 ? 2 : 1;
  const uint32_t* iwords = static_cast<const uint32_t*>(p.idx) + ibase * ewords;
  auto raw_at = [&](int ch, int l) -> uint64_t {
    const int slot = slot_at(ch, l) ? ch * kMfChunk + l : 0;
    const uint32_t* w = iwords + (BLK ? slot >> p.blk_log2 : slot) * ewords;
    return (static_cast<uint64_t>(w[ewords - 1]) << 32) | w[0];
  };
  auto key_at = [&](int ch, int l, uint64_t raw) -> int {
    const int64_t jv = p.idx_i64 ? static_cast<int64_t>(raw)
                                 : static_cast<int64_t>(static_cast<int32_t>(static_cast<uint32_t>(raw)));
    return att_key_wave<BLK>(p, ch * kMfChunk + l, jv, slot_at(ch, l));
  };
  auto load_idx = [&](int ch) { return key_at(ch, lane, raw_at(ch, lane)); };
  // Load r of a chunk: lane l fetches the segment stored in slot l % SEGS of
  // chunk row KPI*r + l / SEGS; the LDS address is the load's base + 16*l.
  // Loads go through buffer descriptors of this head's K and V rows with 32-bit
  // byte offsets (the host checks that every row fits below 2^31 bytes and that
  // n and the row strides fit 24 bits); a dropped slot (jsafe < 0) gets an
  // offset past the end, which loads zeros.
  const int lrow = lane / S::SEGS;
  const int lslot = lane % S::SEGS;
  const uint32_t ksn2 = 2u * static_cast<uint32_t>(p.k_sn), vsn2 = 2u * static_cast<uint32_t>(p.v_sn);
  const int kbytes = static_cast<int>((p.n - 1) * p.k_sn * 2 + 2 * D);
  const int vbytes = static_cast<int>((p.n - 1) * p.v_sn * 2 + 2 * D);
  const __amdgpu_buffer_rsrc_t krs = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(kbase), 0, kbytes, kBufferWord3);
  const __amdgpu_buffer_rsrc_t vrs = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(vbase), 0, vbytes, kBufferWord3);
  uint32_t seg16[S::SWZ_PERIOD];
#pragma unroll
  for (int r = 0; r < S::SWZ_PERIOD; ++r) seg16[r] = static_cast<uint32_t>((lslot ^ mf_swz<D>(S::KPI * r + lrow)) << 4);
  const bool same_stride = ksn2 == vsn2;
  auto issue = [&](int jsafe, bool full) {
    if (same_stride) {
      if (full) mf_issue<D, true, true>(krs, vrs, kl, vl, jsafe, lrow, ksn2, vsn2, seg16);
      else mf_issue<D, false, true>(krs, vrs, kl, vl, jsafe, lrow, ksn2, vsn2, seg16);
    } else {
      if (full) mf_issue<D, true, false>(krs, vrs, kl, vl, jsafe, lrow, ksn2, vsn2, seg16);
      else mf_issue<D, false, false>(krs, vrs, kl, vl, jsafe, lrow, ksn2, vsn2, seg16);
    }
  };
  // keys below the row's dense prefix were attended by prefix_attention_kernel,
  // which clamps a caller's X to [0, min(top_k, n)] the same way
  const int xpre = (NSPLIT == 1 && !BLK && p.pfx_x && row_ok)
                       ? min(max(p.pfx_x[bh * p.n_q + qr], 0),
                             static_cast<int>(min(static_cast<int64_t>(p.top_k), p.n)))
                       : 0;
  // (the causal cut as an int: keys and n fit 24 bits)
  const int icut = p.causal ? static_cast<int>(min(i, static_cast<int64_t>(INT32_MAX))) : INT32_MAX;
  auto chunk_ok = [&](int j) { return j >= xpre && j <= icut; };

  // Fragment addresses (fixed per lane): K tile t, block kb; V^T tile t (rows
  // 4*q4 + c16/4, +16 for the second half of the chunk).
  const int vkey = 4 * q4 + (c16 >> 2);
  const int vswz = mf_swz<D>(vkey);
  const int kswz = mf_swz<D>(c16);

  const bool hi_row = c16 < p.g;
  const bool lo_row = c16 >= 8 && c16 < 8 + p.g;
  const bool cpos = p.qk_scale_log2 > 0.0f && p.qk_scale_log2 <= 3.4e38f;
  const float cmul = cpos ? p.qk_scale_log2 : 1.0f;
  float m_run = -INFINITY;
  float l_run = 0.0f;
  floatx4_t oacc[S::NT];
#pragma unroll
  for (int t = 0; t < S::NT; ++t) oacc[t] = floatx4_t{0.f, 0.f, 0.f, 0.f};
  if (xpre > 0 && hi_row) {
    // column c16 < g (head c16's P_hi) carries the prefix state; P_lo columns start at 0
    const float* pp = p.pfx_part + ((bh * p.n_q + qr) * p.g + c16) * (D + 4);
#pragma unroll
    for (int t = 0; t < S::NT; ++t) {
      const float4 o4 = *reinterpret_cast<const float4*>(pp + 16 * t + 4 * q4);
      oacc[t] = floatx4_t{o4.x, o4.y, o4.z, o4.w};
    }
    m_run = pp[D];
    l_run = (q4 == 0) ? pp[D + 1] : 0.0f;
  }

  const int nchunks = (p.top_k + kMfChunk - 1) / kMfChunk;
  // this wave's chunks: c0, c0 + NSPLIT, ... (all of them when NSPLIT = 1)
  const int nmine = (nchunks > c0) ? (nchunks - c0 + NSPLIT - 1) / NSPLIT : 0;
  auto chunk_of = [&](int u) { return c0 + u * NSPLIT; };
  LiveChunks lc;
  if (xpre > 0)
    lc.build(nmine, lane, [&](int u, int l) { return raw_at(chunk_of(u), l); },
             [&](int u, int l, uint64_t jv) { return key_at(chunk_of(u), l, jv); }, chunk_ok);
  else
    lc.all_live(nmine);
  // The next live chunk's index entries (jn_raw, for chunk un) are loaded
  // while the current chunk's gathers fly and checked only after the wait
  // that the gathers need anyway.  Every chunk issues its loads, also one
  // whose slots all turn out dropped (only a chunk past the causal cut can):
  // those load zeros, its scores are masked to -inf and it adds nothing, and
  // the loop keeps a single path, so the accumulators stay in place across
  // iterations (a separate skip path made the compiler copy all 32 of them
  // twice per chunk).
  int u = lc.next(-1);
  int un = nmine;
  uint64_t okbits = 0;
  uint64_t jn_raw = 0;
  if (u < nmine) {
    const int j0 = lc.get(u, lane, [&](int v) { return load_idx(chunk_of(v)); });
    const bool ok0 = chunk_ok(j0);
    okbits = __ballot(ok0);
    issue(ok0 ? j0 : -1, static_cast<uint32_t>(okbits) == 0xFFFFFFFFu);
    un = lc.next(u);
    if (un < nmine) jn_raw = raw_at(chunk_of(un), lane);
  }
  // u = un: issue chunk u from jn_raw and prefetch the indices of the live
  // chunk after it
  auto advance = [&]() {
    u = un;
    if (u < nmine) {
      const int jn = key_at(chunk_of(u), lane, jn_raw);
      const bool okn = chunk_ok(jn);
      okbits = __ballot(okn);
      issue(okn ? jn : -1, static_cast<uint32_t>(okbits) == 0xFFFFFFFFu);
      if (NSPLIT == 1 && p.gather_wait) __builtin_amdgcn_s_waitcnt(kWaitVm0);  // (not the few-row split kernel)
      un = lc.next(u);
      if (un < nmine) jn_raw = raw_at(chunk_of(un), lane);
    }
  };
  while (u < nmine) {
    // This chunk's rows are in LDS once its loads have completed.
    __builtin_amdgcn_s_waitcnt(kWaitVm0);
    bf16x8_t kf[2][S::KB];
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int kb = 0; kb < S::KB; ++kb)
        kf[t][kb] = *(lds_bf16x8_ptr)(kl + (16 * t + c16) * S::ROW + (((kb * 4 + q4) ^ kswz) << 4));
    bf16x8_t vt[S::NT];
#pragma unroll
    for (int t = 0; t < S::NT; ++t) {
      const int off = vkey * S::ROW + (((2 * t + ((c16 & 3) >> 1)) ^ vswz) << 4) + (c16 & 1) * 8;
      const v4i16_t a0 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4i16_ptr)(vl + off));
      const v4i16_t a1 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4i16_ptr)(vl + off + 16 * S::ROW));
      vt[t] = __builtin_bit_cast(
          bf16x8_t, make_uint4(__builtin_bit_cast(uint2, a0).x, __builtin_bit_cast(uint2, a0).y,
                               __builtin_bit_cast(uint2, a1).x, __builtin_bit_cast(uint2, a1).y));
    }
    // The slices are free once the reads have returned: start the next chunk.
    __builtin_amdgcn_s_waitcnt(kWaitLgkm0);
    const uint64_t okb = okbits;
    okbits = 0;
    advance();

    // Scores of eight keys of head c16 (keys 16t + 4*q4 + e), unscaled: the
    // scale c enters through the running maximum (max(s) c is the maximum of
    // the scaled scores for c > 0) and the exponent's fma.  A caller's scale
    // that makes c non-positive or infinite scales the scores first (cmul = 1).
    float sc[8];
    const bool full = static_cast<uint32_t>(okb) == 0xFFFFFFFFu;
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      floatx4_t s = {0.f, 0.f, 0.f, 0.f};
      if ((okb >> (16 * t)) & 0xFFFFull) {
#pragma unroll
        for (int kb = 0; kb < S::KB; ++kb) s = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kf[t][kb], qf[kb], s, 0, 0, 0);
      }
#pragma unroll
      for (int e = 0; e < 4; ++e) sc[4 * t + e] = s[e];
    }
    if (!cpos) {
#pragma unroll
      for (int x = 0; x < 8; ++x) sc[x] *= p.qk_scale_log2;
    }
    if (!full) {
      // bit 16t + e: key 16t + 4*q4 + e ((lane >> 2) & 12 = 4*q4, recomputed here
      // rather than kept live across the loop)
      const uint32_t mine = static_cast<uint32_t>(okb) >> ((lane >> 2) & 12);
#pragma unroll
      for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int e = 0; e < 4; ++e)
          if (!((mine >> (16 * t + e)) & 1u)) sc[4 * t + e] = -INFINITY;
    }
    // (a NaN score makes the output NaN with either kind of maximum)
    float mx = max_nan(max_nan(max_nan(sc[0], sc[1]), sc[2]), max_nan(sc[3], sc[4]));
    mx = max_nan(max_nan(mx, sc[5]), max_nan(sc[6], sc[7]));
    mx = rows4_reduce(mx, max_nan) * cmul;
    const float mnew = fmaxf(m_run, mx);
    // A head with no valid key yet (mnew = -inf) subtracts 0 instead: its
    // weights exp2(-inf) are 0 and alpha multiplies an all-zero state.
    // v_exp_f32 directly: weights below 2^-126 (denormal) do not matter here.
    const float mref = (mnew == -INFINITY) ? 0.0f : mnew;
    const float alpha = __builtin_amdgcn_exp2f(m_run - mref);
    m_run = mnew;
    float pr[8];
    float ps = 0.0f;
#pragma unroll
    for (int x = 0; x < 8; ++x) {
      pr[x] = __builtin_amdgcn_exp2f(fmaf(sc[x], cmul, -mref));
      ps += pr[x];
    }
    l_run = l_run * alpha + ps;

    // P^T operand: rows c16 < g take P_hi of head c16, rows 8 + r take P_lo of head r.
    uint32_t pb[4];
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      const uint32_t hi = pack_bf16x2(pr[2 * w], pr[2 * w + 1]);
      const uint32_t lo = pack_bf16x2(pr[2 * w] - __uint_as_float(hi << 16),
                                      pr[2 * w + 1] - __uint_as_float(hi & 0xFFFF0000u));
      const uint32_t lo_in = dpp_from_minus8(lo);
      pb[w] = hi_row ? hi : (lo_row ? lo_in : 0u);
    }
    // (cross-lane reads happen in every lane, before any lane-dependent select)
    const float alpha_in = __uint_as_float(dpp_from_minus8(__float_as_uint(alpha)));
    const float a_row = hi_row ? alpha : alpha_in;
    const bf16x8_t pbv = __builtin_bit_cast(bf16x8_t, make_uint4(pb[0], pb[1], pb[2], pb[3]));
    // Rescale only when some head's running max moved (alpha = 1 otherwise).
    if (__ballot(a_row != 1.0f)) {
#pragma unroll
      for (int t = 0; t < S::NT; ++t) oacc[t] *= a_row;
    }
#pragma unroll
    for (int t = 0; t < S::NT; ++t) oacc[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(vt[t], pbv, oacc[t], 0, 0, 0);
  }

  // l: partial sums of the four lanes holding a head's keys; O: hi row + lo row.
  const float lt = rows4_reduce(l_run, [](float a, float b) { return a + b; });
#pragma unroll
  for (int t = 0; t < S::NT; ++t)
#pragma unroll
    for (int e = 0; e < 4; ++e) oacc[t][e] += dpp_from_plus8(oacc[t][e]);
  if constexpr (NSPLIT > 1) {
    if (!row_ok || !hi_row) return;
    float* po = part + c16 * D + 4 * q4;
#pragma unroll
    for (int t = 0; t < S::NT; ++t)
      *reinterpret_cast<float4*>(po + 16 * t) = make_float4(oacc[t][0], oacc[t][1], oacc[t][2], oacc[t][3]);
    if (q4 == 0) {
      part[8 * D + c16] = m_run;
      part[8 * D + 8 + c16] = lt;
    }
    return;
  }
  if (!row_ok || !hi_row) return;
  const float inv = lt > 0.0f ? 1.0f / lt : 0.0f;
  if (p.stats && q4 == 0) {
    float* sp = p.stats + ((bh * p.n_q + qr) * p.g + c16) * 2;
    sp[0] = (m_run == -INFINITY) ? 0.0f : m_run;
    sp[1] = inv;
  }
  const int64_t ob = bb * p.o_sb + qr * p.o_sn + static_cast<int64_t>(h * p.g + c16) * p.o_sh + 4 * q4;
  if (p.out_bf16) {
    // v_cvt_pk_bf16_f32: round to nearest even, the bits f32_to_bf16_rne gives
    // for every non-NaN value, two values per instruction
    uint16_t* dst = static_cast<uint16_t*>(p.out) + ob;
#pragma unroll
    for (int t = 0; t < S::NT; ++t)
      *reinterpret_cast<uint2*>(dst + 16 * t) =
          make_uint2(pack_bf16x2(oacc[t][0] * inv, oacc[t][1] * inv), pack_bf16x2(oacc[t][2] * inv, oacc[t][3] * inv));
  } else {
    float* dst = static_cast<float*>(p.out) + ob;
#pragma unroll
    for (int t = 0; t < S::NT; ++t)
      *reinterpret_cast<float4*>(dst + 16 * t) =
          make_float4(oacc[t][0] * inv, oacc[t][1] * inv, oacc[t][2] * inv, oacc[t][3] * inv);
  }
}

template <int D, bool BLK>
__global__ __launch_bounds__(64 * kMfWaves) __attribute__((amdgpu_waves_per_eu(kMfMinWavesPerEu, 8))) void
sparse_attention_mfma_kernel(AttParams p) {
  using S = MfShape<D>;
  __shared__ __align__(16) unsigned char kv_lds[kMfWaves][2][kMfChunk * S::ROW];
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  // With a row order (rows that share codebook buckets, hence keys, next to
  // each other) XCD x takes a contiguous range of blocks, so its L2 holds the
  // keys its rows share; without one, consecutive blocks go to different
  // XCDs, which measured faster for index sets with no such sharing.
  const int64_t blk = p.order ? xcd_block(blockIdx.x, xcd_per(ceil_div(p.rows, kMfWaves))) : blockIdx.x;
  const AttRow ar = att_row(p, blk * kMfWaves + wave);
  attend_row_mfma<D, BLK>(p, ar, kv_lds[wave][0], kv_lds[wave][1]);
}

// ---- dense key prefix of many rows ------------------------------------------
//
// A row with fewer candidates than top_k fills its list with the lowest keys
// it does not hold already, so its indices cover a prefix [0, X) of the keys
// (at the headline shape 54% of all selected slots lie in such prefixes, and
// neighbouring rows have similar X).  Gathering those keys row by row moves the
// same few hundred K/V rows once per row through each CU; here one block takes
// kPfxQv query vectors (R = kPfxQv / g consecutive rows of one (batch, kv
// head), all their heads) and streams the keys [0, max X) through LDS once for
// all of them:
//   1. X per row from pfx_x: the selection's row_prefix, or else what
//      prefix_x_kernel found in the indices.
//   2. Chunks of 32 consecutive keys, three LDS buffers: every wave loads its
//      share of chunk u + 2 while the block computes chunk u (one barrier per
//      chunk).  Each wave scores its two 16-query tiles (S^T = K.Q^T on the
//      matrix cores, queries as the 16 columns), masks keys at or past the
//      query row's X (and past its position when causal), runs the online
//      softmax in the exp2 domain and accumulates O^T += V^T (P_hi + P_lo) as
//      two MFMAs (P split into bf16 hi and lo as in the row kernel).
//   3. The unnormalised state (O, running max, sum) of each query goes to
//      pfx_part; the row kernel starts from it and skips indices below X.
constexpr int kPfxWaves = 4;
constexpr int kPfxQv = 32 * kPfxWaves;  // query vectors per block: two 16-column tiles per wave
constexpr int kPfxXMax = 1024;          // longest prefix looked for in the indices
constexpr int kPfxBufs = 3;

// X per row from its indices, when the caller gives no row_prefix: one wave per
// row ((batch, kv head, query) in natural order).  The indices below
// xb = min(top_k, kPfxXMax, n) set bits of a 32-word LDS bitmap, X is the first
// clear bit, lowered to the smallest index that occurs twice (duplicates count
// twice in the reference, so a prefix must hold each key once); X goes to
// pfx_x.  The rows' index loads are 16-byte pieces where the layout allows.
constexpr int kPfxXWaves = 4;
__global__ __launch_bounds__(64 * kPfxXWaves) void prefix_x_kernel(AttParams p) {
  __shared__ uint32_t bits[kPfxXWaves][kPfxXMax / 32];
  __shared__ int s_dup[kPfxXWaves];
  const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
  const int lane = threadIdx.x & 63;
  const int64_t lrow = min(static_cast<int64_t>(blockIdx.x) * kPfxXWaves + wave, p.rows - 1);
  const int64_t bh = udiv32(lrow, p.n_q), r = lrow - bh * p.n_q;
  const int64_t bb = udiv32(bh, p.h_kv);
  const int h = static_cast<int>(bh - bb * p.h_kv);
  const int xb = static_cast<int>(min(static_cast<int64_t>(min(p.top_k, kPfxXMax)), p.n));
  const int words = (xb + 31) >> 5;
  uint32_t* bw = bits[wave];
  if (lane < kPfxXMax / 32) bw[lane] = 0u;
  if (lane == 0) s_dup[wave] = 0x7FFFFFFF;
  __syncthreads();
  auto mark = [&](int64_t j) {
    if (j >= 0 && j < xb) {
      const uint32_t bit = 1u << (j & 31);
      if (atomicOr(&bw[j >> 5], bit) & bit) atomicMin(&s_dup[wave], static_cast<int>(j));
    }
  };
  const int64_t ib = bb * p.idx_sb + r * p.idx_sn + static_cast<int64_t>(h) * p.idx_sh;
  const int top_k = p.top_k;
  if (!p.idx_i64 && (top_k & 3) == 0 &&
      (reinterpret_cast<uintptr_t>(static_cast<const int32_t*>(p.idx) + ib) & 15) == 0) {
    const int4* row4 = reinterpret_cast<const int4*>(static_cast<const int32_t*>(p.idx) + ib);
    for (int e = lane; e < (top_k >> 2); e += 64) {
      const int4 v = row4[e];
      mark(v.x);
      mark(v.y);
      mark(v.z);
      mark(v.w);
    }
  } else if (p.idx_i64 && (top_k & 1) == 0 &&
             (reinterpret_cast<uintptr_t>(static_cast<const int64_t*>(p.idx) + ib) & 15) == 0) {
    const longlong2* row2 = reinterpret_cast<const longlong2*>(static_cast<const int64_t*>(p.idx) + ib);
    for (int e = lane; e < (top_k >> 1); e += 64) {
      const longlong2 v = row2[e];
      mark(v.x);
      mark(v.y);
    }
  } else {
    for (int e = lane; e < top_k; e += 64)
      mark(p.idx_i64 ? static_cast<const int64_t*>(p.idx)[ib + e]
                     : static_cast<int64_t>(static_cast<const int32_t*>(p.idx)[ib + e]));
  }
  __syncthreads();
  // first clear bit below 32 * words: the lowest word that is not full
  const uint32_t v = (lane < words) ? bw[lane] : 0u;
  const uint64_t open = __ballot(lane < words && v != 0xFFFFFFFFu);
  int x = 32 * words;
  if (open != 0ull) {
    const int w0 = __ffsll(static_cast<unsigned long long>(open)) - 1;
    const uint32_t vw = static_cast<uint32_t>(lane_value(static_cast<int>(v), w0));
    x = 32 * w0 + __ffs(~vw) - 1;
  }
  if (lane == 0) p.pfx_x[lrow] = min(min(x, xb), s_dup[wave]);
}

template <int D>
__global__ __launch_bounds__(64 * kPfxWaves, 2) void prefix_attention_kernel(AttParams p) {
  using S = MfShape<D>;
  constexpr int kLoadsPerWave = S::NLD / kPfxWaves;  // of K and of V, per chunk
  static_assert(S::NLD % kPfxWaves == 0, "chunk loads split evenly over the waves");
  __shared__ __align__(16) unsigned char kv[kPfxBufs][2][kMfChunk * S::ROW];  // [buffer][K, V]
  __shared__ int s_x[kPfxQv];
  __shared__ int s_xmax;
  const int g = p.g;
  const int R = kPfxQv / g;  // rows per block
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int q4 = lane >> 4, c16 = lane & 15;
  const int64_t tiles = udiv32(p.n_q + R - 1, R);
  const int64_t nblk = udiv32(p.rows, p.n_q) * tiles;
  const int64_t blk = xcd_block(blockIdx.x, xcd_per(nblk));
  if (blk >= nblk) return;
  const int64_t bh = udiv32(blk, tiles);
  const int64_t r0 = (blk - bh * tiles) * R;
  const int64_t bb = udiv32(bh, p.h_kv);
  const int h = static_cast<int>(bh - bb * p.h_kv);
  const int nr = static_cast<int>(min(static_cast<int64_t>(R), p.n_q - r0));

  // 1. X of each row (from the selection, or from prefix_x_kernel)
  if (tid == 0) s_xmax = 0;
  {
    const int xcap = static_cast<int>(min(static_cast<int64_t>(p.top_k), p.n));
    if (tid < R) s_x[tid] = (tid < nr) ? min(max(p.pfx_x[bh * p.n_q + r0 + tid], 0), xcap) : 0;
    __syncthreads();
  }
  if (tid < R) atomicMax(&s_xmax, s_x[tid]);
  __syncthreads();
  const int xmax = s_xmax;
  if (xmax == 0) return;

  // 2. the prefix keys, 32 at a time, for the block's query vectors
  bf16x8_t qf[2][S::KB];
  int xr[2], ilim[2];
  bool qok[2];
#pragma unroll
  for (int qt = 0; qt < 2; ++qt) {
    const int qv = 32 * wave + 16 * qt + c16;
    const int r = qv / g, hh = qv - r * g;
    qok[qt] = qv < R * g && r < nr;
    xr[qt] = qok[qt] ? s_x[r] : 0;
    ilim[qt] = p.causal ? static_cast<int>(min(p.q_pos0 + r0 + r, static_cast<int64_t>(0x7FFFFFFF)))
                        : 0x7FFFFFFF;
    const uint16_t* qh = static_cast<const uint16_t*>(p.q) + bb * p.q_sb + (r0 + (qok[qt] ? r : 0)) * p.q_sn +
                         static_cast<int64_t>(h * g + (qok[qt] ? hh : 0)) * p.q_sh;
#pragma unroll
    for (int kb = 0; kb < S::KB; ++kb)
      qf[qt][kb] = qok[qt] ? *reinterpret_cast<const bf16x8_t*>(qh + kb * 32 + q4 * 8) : bf16x8_t{};
  }
  const uint16_t* kbase = static_cast<const uint16_t*>(p.k) + bb * p.k_sb + static_cast<int64_t>(h) * p.k_sh;
  const uint16_t* vbase = static_cast<const uint16_t*>(p.v) + bb * p.v_sb + static_cast<int64_t>(h) * p.v_sh;
  const int kbytes = static_cast<int>((p.n - 1) * p.k_sn * 2 + 2 * D);
  const int vbytes = static_cast<int>((p.n - 1) * p.v_sn * 2 + 2 * D);
  const __amdgpu_buffer_rsrc_t krs =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(kbase), 0, kbytes, kBufferWord3);
  const __amdgpu_buffer_rsrc_t vrs =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(vbase), 0, vbytes, kBufferWord3);
  uint32_t seg16[S::SWZ_PERIOD];
  row_seg16<D>(lane, seg16);
  const uint32_t ksn2 = 2u * static_cast<uint32_t>(p.k_sn), vsn2 = 2u * static_cast<uint32_t>(p.v_sn);
  // This wave's share of chunk ch: loads r = wave * kLoadsPerWave + t of K
  // and of V (load r moves chunk rows KPI*r .. KPI*r + KPI - 1).
  auto issue = [&](int ch) {
    unsigned char* kl = kv[ch % kPfxBufs][0];
    unsigned char* vl = kv[ch % kPfxBufs][1];
#pragma unroll
    for (int t = 0; t < kLoadsPerWave; ++t) {
      const int r = wave * kLoadsPerWave + t;
      const int j = ch * kMfChunk + S::KPI * r + lane / S::SEGS;
      const uint32_t sg = seg16[r % S::SWZ_PERIOD];
      const uint32_t ko = j < xmax ? __umul24(static_cast<uint32_t>(j), ksn2) + sg : kOobOffset;
      const uint32_t vo = j < xmax ? __umul24(static_cast<uint32_t>(j), vsn2) + sg : kOobOffset;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(krs, (lds_void_ptr)(kl + r * 1024), 16, static_cast<int>(ko), 0, 0, 0);
      __builtin_amdgcn_raw_ptr_buffer_load_lds(vrs, (lds_void_ptr)(vl + r * 1024), 16, static_cast<int>(vo), 0, 0, 0);
    }
  };

  float m_run[2] = {-INFINITY, -INFINITY};
  float l_run[2] = {0.0f, 0.0f};
  floatx4_t oacc[2][S::NT];
#pragma unroll
  for (int qt = 0; qt < 2; ++qt)
#pragma unroll
    for (int t = 0; t < S::NT; ++t) oacc[qt][t] = floatx4_t{0.f, 0.f, 0.f, 0.f};
  const int kswz = mf_swz<D>(c16);
  const int nch = (xmax + kMfChunk - 1) / kMfChunk;
  // Keys below jfull[qt] (the wave's smallest min(X, position + 1) of tile qt)
  // need no mask: the chunks below it skip the per-key tests.
  int jfull[2];
#pragma unroll
  for (int qt = 0; qt < 2; ++qt) {
    int jl = qok[qt] ? min(xr[qt], ilim[qt] == 0x7FFFFFFF ? 0x7FFFFFFF : ilim[qt] + 1) : 0x7FFFFFFF;
    jl = min(jl, __shfl_xor(jl, 1));
    jl = min(jl, __shfl_xor(jl, 2));
    jl = min(jl, __shfl_xor(jl, 4));
    jl = min(jl, __shfl_xor(jl, 8));
    jl = min(jl, __shfl_xor(jl, 16));
    jl = min(jl, __shfl_xor(jl, 32));
    jfull[qt] = __builtin_amdgcn_readfirstlane(jl);
  }
  // The scale c enters through the running maximum and the exponent's fma when
  // it is positive and finite (max(s) c is the maximum of the scaled scores);
  // otherwise the scores are scaled first (cmul = 1).
  const bool cpos = p.qk_scale_log2 > 0.0f && p.qk_scale_log2 <= 3.4e38f;
  const float cmul = cpos ? p.qk_scale_log2 : 1.0f;
  issue(0);
  if (nch > 1) issue(1);
  for (int u = 0; u < nch; ++u) {
    // this wave's share of chunk u has landed (chunk u + 1's may still fly)
    if (u + 1 < nch) __builtin_amdgcn_s_waitcnt(kWaitVmBase | (2 * kLoadsPerWave));
    else __builtin_amdgcn_s_waitcnt(kWaitVm0);
    // every share of chunk u is in LDS, and every wave is done with chunk u - 1
    __syncthreads();
    if (u + 2 < nch) issue(u + 2);
    const unsigned char* kl = kv[u % kPfxBufs][0];
    const unsigned char* vl = kv[u % kPfxBufs][1];
    bf16x8_t kf[2][S::KB];
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int kb = 0; kb < S::KB; ++kb)
        kf[t][kb] = *(lds_bf16x8_ptr)(kl + (16 * t + c16) * S::ROW + (((kb * 4 + q4) ^ kswz) << 4));
    bf16x8_t vt[S::NT];
#pragma unroll
    for (int t = 0; t < S::NT; ++t) vt[t] = rows_transposed<D>(vl, t, q4, c16);
    const int jbase = u * kMfChunk + 4 * q4;
#pragma unroll
    for (int qt = 0; qt < 2; ++qt) {
      float sc[8];
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        floatx4_t sv = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int kb = 0; kb < S::KB; ++kb) sv = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kf[t][kb], qf[qt][kb], sv, 0, 0, 0);
#pragma unroll
        for (int e = 0; e < 4; ++e) sc[4 * t + e] = sv[e];
      }
      if (!cpos) {
#pragma unroll
        for (int x = 0; x < 8; ++x) sc[x] *= p.qk_scale_log2;
      }
      if ((u + 1) * kMfChunk > jfull[qt]) {
#pragma unroll
        for (int t = 0; t < 2; ++t)
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const int j = jbase + 16 * t + e;
            if (!(j < xr[qt] && j <= ilim[qt])) sc[4 * t + e] = -INFINITY;
          }
      }
      float mx = max_nan(max_nan(max_nan(sc[0], sc[1]), sc[2]), max_nan(sc[3], sc[4]));
      mx = max_nan(max_nan(mx, sc[5]), max_nan(sc[6], sc[7]));
      mx = rows4_reduce(mx, max_nan) * cmul;
      const float mnew = fmaxf(m_run[qt], mx);
      const float mref = (mnew == -INFINITY) ? 0.0f : mnew;
      const float alpha = __builtin_amdgcn_exp2f(m_run[qt] - mref);
      m_run[qt] = mnew;
      float pr[8];
      float ps = 0.0f;
#pragma unroll
      for (int x = 0; x < 8; ++x) {
        pr[x] = __builtin_amdgcn_exp2f(fmaf(sc[x], cmul, -mref));
        ps += pr[x];
      }
      l_run[qt] = l_run[qt] * alpha + ps;
      uint32_t ph[4], pl[4];
#pragma unroll
      for (int w = 0; w < 4; ++w) {
        ph[w] = pack_bf16x2(pr[2 * w], pr[2 * w + 1]);
        pl[w] = pack_bf16x2(pr[2 * w] - __uint_as_float(ph[w] << 16),
                            pr[2 * w + 1] - __uint_as_float(ph[w] & 0xFFFF0000u));
      }
      const bf16x8_t phv = __builtin_bit_cast(bf16x8_t, make_uint4(ph[0], ph[1], ph[2], ph[3]));
      const bf16x8_t plv = __builtin_bit_cast(bf16x8_t, make_uint4(pl[0], pl[1], pl[2], pl[3]));
      if (__ballot(alpha != 1.0f)) {
#pragma unroll
        for (int t = 0; t < S::NT; ++t) oacc[qt][t] *= alpha;
      }
#pragma unroll
      for (int t = 0; t < S::NT; ++t) {
        oacc[qt][t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(vt[t], phv, oacc[qt][t], 0, 0, 0);
        oacc[qt][t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(vt[t], plv, oacc[qt][t], 0, 0, 0);
      }
    }
  }

  // 3. the state of each query with a prefix
#pragma unroll
  for (int qt = 0; qt < 2; ++qt) {
    const float lt = rows4_reduce(l_run[qt], [](float a, float b) { return a + b; });
    if (!qok[qt] || xr[qt] == 0) continue;
    const int qv = 32 * wave + 16 * qt + c16;
    const int r = qv / g, hh = qv - r * g;
    float* pp = p.pfx_part + ((bh * p.n_q + r0 + r) * g + hh) * (D + 4);
#pragma unroll
    for (int t = 0; t < S::NT; ++t)
      *reinterpret_cast<float4*>(pp + 16 * t + 4 * q4) =
          make_float4(oacc[qt][t][0], oacc[qt][t][1], oacc[qt][t][2], oacc[qt][t][3]);
    if (q4 == 0) {
      pp[D] = m_run[qt];
      pp[D + 1] = lt;
    }
  }
}

// Few rows (decoding): one block of kSplitWaves waves per row, wave w taking
// chunks w, w + kSplitWaves, ...; the waves' partial states (per head: running
// max m_w, sum l_w, unnormalised O_w) combine as O = sum_w 2^(m_w - M) O_w /
// sum_w 2^(m_w - M) l_w with M = max_w m_w.  A row otherwise runs its chunks
// one after another on one wave, which leaves the GPU idle when a call has a
// few rows.
constexpr int kSplitWaves = 4;
constexpr int64_t kSplitRowsMax = 512;

template <int D>
__global__ __launch_bounds__(64 * kSplitWaves) void sparse_attention_split_kernel(AttParams p) {
  using S = MfShape<D>;
  __shared__ __align__(16) unsigned char kv_lds[kSplitWaves][2][kMfChunk * S::ROW];
  __shared__ __align__(16) float part[kSplitWaves][8 * D + 16];
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const AttRow ar = att_row(p, blockIdx.x);
  attend_row_mfma<D, false, kSplitWaves>(p, ar, kv_lds[wave][0], kv_lds[wave][1], wave, part[wave]);
  __syncthreads();
  if (!ar.ok) return;
  const int64_t bb = udiv32(ar.bh, p.h_kv);
  const int h = static_cast<int>(ar.bh - bb * p.h_kv);
  for (int e = threadIdx.x; e < p.g * D; e += 64 * kSplitWaves) {
    const int hh = e / D, dim = e - hh * D;
    float M = -INFINITY;
#pragma unroll
    for (int w = 0; w < kSplitWaves; ++w) M = fmaxf(M, part[w][8 * D + hh]);
    float L = 0.0f, O = 0.0f;
    if (M != -INFINITY) {
#pragma unroll
      for (int w = 0; w < kSplitWaves; ++w) {
        const float mw = part[w][8 * D + hh];
        if (mw == -INFINITY) continue;  // no valid key in this wave's chunks
        const float a = __builtin_amdgcn_exp2f(mw - M);
        L += a * part[w][8 * D + 8 + hh];
        O += a * part[w][hh * D + dim];
      }
    }
    const float val = L > 0.0f ? O / L : 0.0f;
    const int64_t ob = bb * p.o_sb + ar.r * p.o_sn + static_cast<int64_t>(h * p.g + hh) * p.o_sh + dim;
    if (p.out_bf16) static_cast<uint16_t*>(p.out)[ob] = f32_to_bf16_rne(val);
    else static_cast<float*>(p.out)[ob] = val;
  }
}

template <typename T, int D>
int launch_att_d(const AttParams& p, hipStream_t st) {
  const int64_t blocks = ceil_div(p.rows, kAttWaves);
  if constexpr (sizeof(T) == 2 && D >= 64 && D <= 128) {
    // 32-bit buffer offsets: rows below 2^31 bytes, n and byte strides below 2^24.
    const auto fits = [&](int64_t sn) {
      return sn >= 0 && 2 * sn < (int64_t(1) << 24) && (p.n - 1) * sn * 2 + 2 * D < (int64_t(1) << 31);
    };
    if (p.g <= 8 && p.d == D && p.n < (int64_t(1) << 24) && fits(p.k_sn) && fits(p.v_sn)) {
      if (p.blk_log2 == 0 && p.rows <= kSplitRowsMax && p.top_k >= 2 * kSplitWaves * kMfChunk) {
        AttParams ps = p;
        ps.pfx_x = nullptr;
        sparse_attention_split_kernel<D><<<dim3(static_cast<unsigned>(p.rows)), 64 * kSplitWaves, 0, st>>>(ps);
        return check_launch("sparse_attention_split_kernel");
      }
      AttParams pr = p;
      if (p.blk_log2 == 0 && p.pfx_x) {
        if (!p.pfx_given) {
          prefix_x_kernel<<<dim3(static_cast<unsigned>(ceil_div(p.rows, kPfxXWaves))), 64 * kPfxXWaves, 0, st>>>(p);
          if (int s = check_launch("prefix_x_kernel")) return s;
        }
        const int64_t rows_per = kPfxQv / p.g;
        const int64_t pblocks = (p.rows / p.n_q) * ceil_div(p.n_q, rows_per);
        prefix_attention_kernel<D><<<dim3(static_cast<unsigned>(kXcds * xcd_per(pblocks))), 64 * kPfxWaves, 0, st>>>(p);
        if (int s = check_launch("prefix_attention_kernel")) return s;
      } else {
        pr.pfx_x = nullptr;
      }
      const dim3 grid(static_cast<unsigned>(kXcds * xcd_per(ceil_div(p.rows, kMfWaves))));
      if (p.blk_log2 > 0) sparse_attention_mfma_kernel<D, true><<<grid, 64 * kMfWaves, 0, st>>>(pr);
      else sparse_attention_mfma_kernel<D, false><<<grid, 64 * kMfWaves, 0, st>>>(pr);
      return check_launch("sparse_attention_mfma_kernel");
    }
  }
  if (p.g <= 4) sparse_attention_kernel<T, D, 4><<<dim3(static_cast<unsigned>(blocks)), kAttThreads, 0, st>>>(p);
  else if (p.g <= 8) sparse_attention_kernel<T, D, 8><<<dim3(static_cast<unsigned>(blocks)), kAttThreads, 0, st>>>(p);
  else sparse_attention_kernel<T, D, 16><<<dim3(static_cast<unsigned>(blocks)), kAttThreads, 0, st>>>(p);
  return check_launch("sparse_attention_kernel");
}

template <typename T>
int launch_att(const AttParams& p, int d, hipStream_t st) {
  // Padded width: the smallest of 32, 64, 128, 256 that holds d.
  if (d <= 32) return launch_att_d<T, 32>(p, st);
  if (d <= 64) return launch_att_d<T, 64>(p, st);
  if (d <= 128) return launch_att_d<T, 128>(p, st);
  return launch_att_d<T, 256>(p, st);
}

}  // namespace
}  // namespace ssa

using namespace ssa;

namespace ssa {
// Workspace of the dense-prefix path: X per row, then the prefix state per
// (row, head).  Zero where the path does not run (fp32, head dims other than
// 64 and 128, groups over 8, fewer than 64 keys per row, block mode).
size_t attention_ws_bytes(int dtype, int64_t batch, int64_t n_q, int h_q, int h_kv, int d, int top_k) {
  if (dtype != SSA_DTYPE_BF16 || (d != 64 && d != 128) || h_kv <= 0 || h_q % h_kv != 0 || h_q / h_kv > 8 ||
      top_k < 2 * kMfChunk || batch <= 0 || n_q <= 0)
    return 0;
  const size_t rows = static_cast<size_t>(batch * h_kv * n_q);
  return align_up(sizeof(int32_t) * rows, 256) +
         sizeof(float) * rows * static_cast<size_t>(h_q / h_kv) * static_cast<size_t>(d + 4);
}

// Token indices (blk_log2 = 0, top_k keys per row) or key-block ids
// (blk_log2 > 0: top_k = blocks per row, nbk blocks in all).
int attention_entry(const void* q, const void* k, const void* v, int dtype, int64_t batch, int64_t n,
                    int64_t n_q, int64_t q_pos0, int h_q, int h_kv, int d, int64_t q_sb, int64_t q_sn,
                    int64_t q_sh, int64_t k_sb, int64_t k_sn, int64_t k_sh, int64_t v_sb, int64_t v_sn,
                    int64_t v_sh, const void* idx, int idx_dtype, int top_k, int64_t idx_sb, int64_t idx_sn,
                    int64_t idx_sh, float scale_div, int causal, const int32_t* row_order, void* out,
                    int out_dtype, int64_t o_sb, int64_t o_sn, int64_t o_sh, int32_t* error_flag,
                    void* stream, int blk_log2, int64_t nbk, void* workspace, size_t workspace_bytes,
                    const int32_t* row_prefix, float* row_stats) {
  if (n_q < 0 || q_pos0 < 0 || q_pos0 + n_q > n)
    return fail(SSA_ERR_INVALID_ARGUMENT, "sparse_attention: query rows [%lld, %lld) outside the %lld keys",
                static_cast<long long>(q_pos0), static_cast<long long>(q_pos0 + n_q),
                static_cast<long long>(n));
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
  if (d < 8 || d > 256 || d % 8 != 0)
    return fail(SSA_ERR_UNSUPPORTED, "sparse_attention: head_dim %d (need a multiple of 8 in [8, 256])", d);
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
  if (batch == 0 || n == 0 || n_q == 0) return SSA_OK;
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
  p.d = d;
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
  p.rows = batch * h_kv * n_q;
  p.order = row_order;
  p.n_q = n_q;
  p.q_pos0 = q_pos0;
  p.blk_log2 = blk_log2;
  p.nbk = nbk;
  if (blk_log2 > 0) {
    if ((static_cast<int64_t>(top_k) << blk_log2) >= (int64_t(1) << 31))
      return fail(SSA_ERR_UNSUPPORTED, "block_sparse_attention: blocks x block_size must be < 2^31");
    p.top_k = top_k << blk_log2;
  }
  if (p.rows >= (int64_t(1) << 31))
    return fail(SSA_ERR_UNSUPPORTED, "sparse_attention: too many rows");
  if (workspace) {
    const size_t need = attention_ws_bytes(dtype, batch, n_q, h_q, h_kv, d, blk_log2 > 0 ? 0 : top_k);
    if (workspace_bytes < need)
      return fail(SSA_ERR_WORKSPACE, "sparse_attention: workspace %zu < %zu bytes", workspace_bytes, need);
    if (need > 0) {
      p.pfx_x = row_prefix ? const_cast<int32_t*>(row_prefix) : static_cast<int32_t*>(workspace);
      p.pfx_given = row_prefix ? 1 : 0;
      p.pfx_part = reinterpret_cast<float*>(static_cast<char*>(workspace) +
                                            align_up(sizeof(int32_t) * static_cast<size_t>(p.rows), 256));
    }
  }
  if (blk_log2 == 0) p.stats = row_stats;
  const int64_t head_kv_bytes = n * d * 2 * 2;
  p.gather_wait = (head_kv_bytes > kGatherWaitBytes && head_kv_bytes * batch * h_kv <= kInfinityCacheBytes) ? 1 : 0;
  hipStream_t st = as_stream(stream);
  if (dtype == SSA_DTYPE_BF16) return launch_att<uint16_t>(p, d, st);
  return launch_att<float>(p, d, st);
}
}  // namespace ssa

extern "C" int ssa_sparse_attention_block(
    const void* q, const void* k, const void* v, int dtype, int64_t batch, int64_t n, int64_t n_q,
    int64_t q_pos0, int h_q, int h_kv, int d, int64_t q_sb, int64_t q_sn, int64_t q_sh, int64_t k_sb,
    int64_t k_sn, int64_t k_sh, int64_t v_sb, int64_t v_sn, int64_t v_sh, const void* idx,
    int idx_dtype, int top_k, int64_t idx_sb, int64_t idx_sn, int64_t idx_sh, float scale_div,
    int causal, const int32_t* row_order, const int32_t* row_prefix, void* out, int out_dtype,
    int64_t o_sb, int64_t o_sn, int64_t o_sh, int32_t* error_flag, float* row_stats, void* workspace,
    size_t workspace_bytes, void* stream) {
  return attention_entry(q, k, v, dtype, batch, n, n_q, q_pos0, h_q, h_kv, d, q_sb, q_sn, q_sh, k_sb, k_sn,
                         k_sh, v_sb, v_sn, v_sh, idx, idx_dtype, top_k, idx_sb, idx_sn, idx_sh, scale_div,
                         causal, row_order, out, out_dtype, o_sb, o_sn, o_sh, error_flag, stream, 0, 0,
                         workspace, workspace_bytes, row_prefix, row_stats);
}

extern "C" size_t ssa_sparse_attention_workspace_bytes(int dtype, int64_t batch, int64_t n_q, int h_q,
                                                       int h_kv, int d, int top_k) {
  return attention_ws_bytes(dtype, batch, n_q, h_q, h_kv, d, top_k);
}

extern "C" int ssa_block_sparse_attention(
    const void* q, const void* k, const void* v, int dtype, int64_t batch, int64_t n, int h_q, int h_kv,
    int d, int64_t q_sb, int64_t q_sn, int64_t q_sh, int64_t k_sb, int64_t k_sn, int64_t k_sh, int64_t v_sb,
    int64_t v_sn, int64_t v_sh, const void* blocks, int idx_dtype, int block_size, int n_k_blocks,
    int64_t b_sb, int64_t b_sq, int64_t b_sh, float scale_div, void* out, int out_dtype, int64_t o_sb,
    int64_t o_sn, int64_t o_sh, int32_t* error_flag, void* stream) {
  if (block_size < 2 || block_size > 256 || (block_size & (block_size - 1)) != 0)
    return fail(SSA_ERR_INVALID_ARGUMENT, "block_sparse_attention: block_size %d (need a power of 2 in [2, 256])",
                block_size);
  if (n_k_blocks < 0) return fail(SSA_ERR_INVALID_ARGUMENT, "block_sparse_attention: n_k_blocks < 0");
  int lg = 0;
  while ((1 << lg) < block_size) ++lg;
  const int64_t nbk = (n + block_size - 1) / block_size;
  return attention_entry(q, k, v, dtype, batch, n, n, 0, h_q, h_kv, d, q_sb, q_sn, q_sh, k_sb, k_sn, k_sh,
                         v_sb, v_sn, v_sh, blocks, idx_dtype, n_k_blocks, b_sb, b_sq, b_sh, scale_div, 1,
                         nullptr, out, out_dtype, o_sb, o_sn, o_sh, error_flag, stream, lg, nbk, nullptr, 0);
}

extern "C" int ssa_sparse_attention(const void* q, const void* k, const void* v, int dtype,
                                    int64_t batch, int64_t n, int h_q, int h_kv, int d,
                                    int64_t q_sb, int64_t q_sn, int64_t q_sh, int64_t k_sb,
                                    int64_t k_sn, int64_t k_sh, int64_t v_sb, int64_t v_sn,
                                    int64_t v_sh, const void* idx, int idx_dtype, int top_k,
                                    int64_t idx_sb, int64_t idx_sn, int64_t idx_sh,
                                    float scale_div, int causal, const int32_t* row_order,
                                    const int32_t* row_prefix, void* out, int out_dtype,
                                    int64_t o_sb, int64_t o_sn, int64_t o_sh, int32_t* error_flag,
                                    float* row_stats, void* workspace, size_t workspace_bytes, void* stream) {
  return attention_entry(q, k, v, dtype, batch, n, n, 0, h_q, h_kv, d, q_sb, q_sn, q_sh, k_sb, k_sn, k_sh,
                         v_sb, v_sn, v_sh, idx, idx_dtype, top_k, idx_sb, idx_sn, idx_sh, scale_div, causal,
                         row_order, out, out_dtype, o_sb, o_sn, o_sh, error_flag, stream, 0, 0, workspace,
                         workspace_bytes, row_prefix, row_stats);
}
