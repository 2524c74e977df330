// Rotary position embedding on [batch][n][heads][d] rows, in place or into
// another buffer: the layer prologue between the q/k projections and routing.
//
// Two callers, one rule.  Features j < rot rotate in pairs (j, j + rot/2):
//   out[j]         = x[j] * cos[j]         - x[j + rot/2] * sin[j]
//   out[j + rot/2] = x[j + rot/2] * cos[j + rot/2] + x[j] * sin[j + rot/2]
// and features j >= rot pass through.  The angle row is either the token's
// position or its head index:
//   * SSAAttention (ssa/ssa_layer.py:115-120 calling ssa/utils.py:7-41 on an
//     [n, heads, d] tensor): rot = d/2, the angle row is the HEAD index, the
//     table is freqs[:, :d/2] (or freqs[position_ids[b]] per batch element);
//   * Hugging Face Qwen2 (training/train_qwen.py:134-135,
//     apply_rotary_pos_emb): rot = d, the angle row is the POSITION, the table
//     is the model's cos/sin [batch][n][d].
// Arithmetic follows torch's elementwise ops exactly (x * cos, rotate_half(x)
// * sin and their sum are three rounded ops; nothing fuses): with bf16 x and
// bf16 tables every intermediate rounds to bf16 (torch's bf16 arithmetic);
// otherwise the intermediates are fp32 (bf16 inputs widen exactly) and only the
// result rounds to the output type.
//
// One thread per VEC consecutive pairs (VEC = 4 when the row layout allows
// 8-byte bf16 / 16-byte fp32 accesses, else 1); the grid covers rows x pairs,
// plus the pass-through features when out is not x.

#include "ssa_common.h"

namespace ssa {
namespace {

constexpr int kRopeThreads = 256;

struct RopeParams {
  const void* x;
  void* out;
  const void* cs;
  const void* sn;
  int64_t n, rows;              // rows = batch * n * h
  int h, d, half, rot, work;    // work = pairs/VEC + copy/VEC per row
  int64_t x_sb, x_sn, x_sh, o_sb, o_sn, o_sh, t_sb, t_sr;
  int by_head, inverse, copy_tail;
  int narrow;  // rows * work < 2^32: thread indices divide in 32 bits
};

template <typename T> struct Elem;
template <> struct Elem<float> {
  __device__ static float get(const float* p, int64_t i) { return p[i]; }
  __device__ static void put(float* p, int64_t i, float v) { p[i] = v; }
};
template <> struct Elem<uint16_t> {
  __device__ static float get(const uint16_t* p, int64_t i) { return bf16_bits_to_f32(p[i]); }
  __device__ static void put(uint16_t* p, int64_t i, float v) { p[i] = f32_to_bf16_rne(v); }
};

template <int VEC, typename T>
__device__ __forceinline__ void load_vec(const T* p, int64_t i, float (&v)[VEC]) {
  if constexpr (VEC == 4 && sizeof(T) == 2) {
    const uint2 u = *reinterpret_cast<const uint2*>(p + i);
    v[0] = __uint_as_float(u.x << 16);
    v[1] = __uint_as_float(u.x & 0xFFFF0000u);
    v[2] = __uint_as_float(u.y << 16);
    v[3] = __uint_as_float(u.y & 0xFFFF0000u);
  } else if constexpr (VEC == 4 && sizeof(T) == 4) {
    const float4 u = *reinterpret_cast<const float4*>(p + i);
    v[0] = u.x; v[1] = u.y; v[2] = u.z; v[3] = u.w;
  } else {
#pragma unroll
    for (int e = 0; e < VEC; ++e) v[e] = Elem<T>::get(p, i + e);
  }
}

template <int VEC, typename T>
__device__ __forceinline__ void store_vec(T* p, int64_t i, const float (&v)[VEC]) {
  if constexpr (VEC == 4 && sizeof(T) == 2) {
    uint2 u;
    u.x = static_cast<uint32_t>(f32_to_bf16_rne(v[0])) | (static_cast<uint32_t>(f32_to_bf16_rne(v[1])) << 16);
    u.y = static_cast<uint32_t>(f32_to_bf16_rne(v[2])) | (static_cast<uint32_t>(f32_to_bf16_rne(v[3])) << 16);
    *reinterpret_cast<uint2*>(p + i) = u;
  } else if constexpr (VEC == 4 && sizeof(T) == 4) {
    *reinterpret_cast<float4*>(p + i) = make_float4(v[0], v[1], v[2], v[3]);
  } else {
#pragma unroll
    for (int e = 0; e < VEC; ++e) Elem<T>::put(p, i + e, v[e]);
  }
}

// Rounds an intermediate to the op type: bf16 (RB) or fp32.
template <bool RB>
__device__ __forceinline__ float op_round(float v) {
  if constexpr (RB) return bf16_bits_to_f32(f32_to_bf16_rne(v));
  return v;
}

template <typename TX, typename TT, typename TO, int VEC>
__global__ __launch_bounds__(kRopeThreads) void rope_kernel(RopeParams p) {
  constexpr bool RB = sizeof(TX) == 2 && sizeof(TT) == 2;
  const int64_t t = static_cast<int64_t>(blockIdx.x) * kRopeThreads + threadIdx.x;
  if (t >= p.rows * p.work) return;
  // (a 64-bit division is about a hundred instructions per thread)
  const int64_t row = p.narrow ? udiv32(t, p.work) : t / p.work;
  const int w = static_cast<int>(t - row * p.work);
  const int64_t bi = p.narrow ? udiv32(row, p.h) : row / p.h;
  const int hh = static_cast<int>(row - bi * p.h);
  const int64_t b = p.narrow ? udiv32(bi, p.n) : bi / p.n;
  const int64_t i = bi - b * p.n;
  const TX* x = static_cast<const TX*>(p.x) + b * p.x_sb + i * p.x_sn + hh * p.x_sh;
  TO* o = static_cast<TO*>(p.out) + b * p.o_sb + i * p.o_sn + hh * p.o_sh;
  const int pairs = p.half / VEC;
  if (w >= pairs) {  // pass-through features rot .. d-1
    const int j = p.rot + (w - pairs) * VEC;
    float v[VEC];
    load_vec<VEC>(x, j, v);
    store_vec<VEC>(o, j, v);
    return;
  }
  const int j = w * VEC;
  const int64_t trow = b * p.t_sb + (p.by_head ? static_cast<int64_t>(hh) : i) * p.t_sr;
  const TT* cs = static_cast<const TT*>(p.cs) + trow;
  const TT* sn = static_cast<const TT*>(p.sn) + trow;
  float x1[VEC], x2[VEC], c1[VEC], c2[VEC], s1[VEC], s2[VEC], y1[VEC], y2[VEC];
  load_vec<VEC>(x, j, x1);
  load_vec<VEC>(x, j + p.half, x2);
  load_vec<VEC>(cs, j, c1);
  load_vec<VEC>(cs, j + p.half, c2);
  load_vec<VEC>(sn, j, s1);
  load_vec<VEC>(sn, j + p.half, s2);
  if (!p.inverse) {
#pragma unroll
    for (int e = 0; e < VEC; ++e) {  // x * cos + rotate_half(x) * sin, rotate_half(x) = [-x2, x1]
      y1[e] = op_round<RB>(op_round<RB>(x1[e] * c1[e]) + op_round<RB>((-x2[e]) * s1[e]));
      y2[e] = op_round<RB>(op_round<RB>(x2[e] * c2[e]) + op_round<RB>(x1[e] * s2[e]));
    }
  } else {
#pragma unroll
    for (int e = 0; e < VEC; ++e) {  // the transpose of the rotation (gradient of the above)
      y1[e] = op_round<RB>(op_round<RB>(x1[e] * c1[e]) + op_round<RB>(x2[e] * s2[e]));
      y2[e] = op_round<RB>(op_round<RB>(x2[e] * c2[e]) + op_round<RB>((-x1[e]) * s1[e]));
    }
  }
  store_vec<VEC>(o, j, y1);
  store_vec<VEC>(o, j + p.half, y2);
}

template <typename TX, typename TT, typename TO>
int launch_rope(const RopeParams& p0, int vec, hipStream_t st) {
  RopeParams p = p0;
  const int tail = p.copy_tail ? (p.d - p.rot) : 0;
  p.work = (p.half + tail) / vec;
  const int64_t total = p.rows * p.work;
  if (total == 0) return SSA_OK;
  const int64_t grid = ceil_div(total, kRopeThreads);
  if (grid > 0x7FFFFFFF) return fail(SSA_ERR_UNSUPPORTED, "ssa_rope: too many rows");
  p.narrow = total < (int64_t(1) << 32) ? 1 : 0;
  if (vec == 4)
    rope_kernel<TX, TT, TO, 4><<<dim3(static_cast<unsigned>(grid)), dim3(kRopeThreads), 0, st>>>(p);
  else
    rope_kernel<TX, TT, TO, 1><<<dim3(static_cast<unsigned>(grid)), dim3(kRopeThreads), 0, st>>>(p);
  return check_launch("ssa_rope");
}

template <typename TX, typename TT>
int dispatch_out(const RopeParams& p, int out_dtype, int vec, hipStream_t st) {
  if (out_dtype == SSA_DTYPE_F32) return launch_rope<TX, TT, float>(p, vec, st);
  return launch_rope<TX, TT, uint16_t>(p, vec, st);
}

bool dtype_ok(int t) { return t == SSA_DTYPE_F32 || t == SSA_DTYPE_BF16; }
int esize(int t) { return t == SSA_DTYPE_F32 ? 4 : 2; }

}  // namespace
}  // namespace ssa

using namespace ssa;

extern "C" int ssa_rope(const void* x, int dtype, int64_t batch, int64_t n, int h, int d,
                        int64_t x_sb, int64_t x_sn, int64_t x_sh, const void* cos_table,
                        const void* sin_table, int table_dtype, int64_t t_sb, int64_t t_sr,
                        int64_t table_rows, int rot, int angle_axis, int inverse, void* out,
                        int out_dtype, int64_t o_sb, int64_t o_sn, int64_t o_sh, void* stream) {
  if (!dtype_ok(dtype) || !dtype_ok(table_dtype) || !dtype_ok(out_dtype))
    return fail(SSA_ERR_UNSUPPORTED, "ssa_rope: element types must be f32 or bf16");
  if (batch < 0 || n < 0 || h <= 0 || d <= 0)
    return fail(SSA_ERR_INVALID_ARGUMENT, "ssa_rope: bad shape batch=%lld n=%lld h=%d d=%d",
                (long long)batch, (long long)n, h, d);
  if (rot <= 0 || rot > d || (rot & 1))
    return fail(SSA_ERR_INVALID_ARGUMENT, "ssa_rope: rot=%d must be even and in (0, d=%d]", rot, d);
  if (angle_axis != SSA_ROPE_BY_POSITION && angle_axis != SSA_ROPE_BY_HEAD)
    return fail(SSA_ERR_INVALID_ARGUMENT, "ssa_rope: angle_axis must be SSA_ROPE_BY_POSITION or _BY_HEAD");
  const int64_t need_rows = angle_axis == SSA_ROPE_BY_HEAD ? h : n;
  if (table_rows < need_rows)
    return fail(SSA_ERR_INVALID_ARGUMENT, "ssa_rope: the angle table has %lld rows, needs %lld",
                (long long)table_rows, (long long)need_rows);
  if (batch == 0 || n == 0) return SSA_OK;
  if (!x || !out || !cos_table || !sin_table)
    return fail(SSA_ERR_INVALID_ARGUMENT, "ssa_rope: null pointer");
  const bool in_place = x == out;
  if (in_place && (dtype != out_dtype || x_sb != o_sb || x_sn != o_sn || x_sh != o_sh))
    return fail(SSA_ERR_INVALID_ARGUMENT, "ssa_rope: in place needs the same type and strides");
  RopeParams p{};
  p.x = x; p.out = out; p.cs = cos_table; p.sn = sin_table;
  p.n = n; p.rows = batch * n * h;
  p.h = h; p.d = d; p.rot = rot; p.half = rot / 2;
  p.x_sb = x_sb; p.x_sn = x_sn; p.x_sh = x_sh;
  p.o_sb = o_sb; p.o_sn = o_sn; p.o_sh = o_sh;
  p.t_sb = t_sb; p.t_sr = t_sr;
  p.by_head = angle_axis == SSA_ROPE_BY_HEAD;
  p.inverse = inverse != 0;
  p.copy_tail = !in_place;
  // VEC = 4 when every row start and both halves are 4-element aligned
  auto al = [](const void* ptr, int bytes) { return (reinterpret_cast<uintptr_t>(ptr) % bytes) == 0; };
  const bool v4 = p.half % 4 == 0 && (d - rot) % 4 == 0 && x_sb % 4 == 0 && x_sn % 4 == 0 &&
                  x_sh % 4 == 0 && o_sb % 4 == 0 && o_sn % 4 == 0 && o_sh % 4 == 0 &&
                  t_sb % 4 == 0 && t_sr % 4 == 0 && al(x, 4 * esize(dtype)) &&
                  al(out, 4 * esize(out_dtype)) && al(cos_table, 4 * esize(table_dtype)) &&
                  al(sin_table, 4 * esize(table_dtype)) && rot % 4 == 0;
  const int vec = v4 ? 4 : 1;
  hipStream_t st = as_stream(stream);
  if (dtype == SSA_DTYPE_F32) {
    if (table_dtype == SSA_DTYPE_F32) return dispatch_out<float, float>(p, out_dtype, vec, st);
    return dispatch_out<float, uint16_t>(p, out_dtype, vec, st);
  }
  if (table_dtype == SSA_DTYPE_F32) return dispatch_out<uint16_t, float>(p, out_dtype, vec, st);
  return dispatch_out<uint16_t, uint16_t>(p, out_dtype, vec, st);
}
