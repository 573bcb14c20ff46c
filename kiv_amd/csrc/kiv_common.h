// Device helpers shared by the tiered-cache kernels (gfx950, wave64).
//
// Element types are carried as raw bits (uint16_t for fp16/bf16, float for
// fp32) and widened to fp32 in registers; every row is moved with 16-byte
// vector accesses, so a row of D elements is D / VEC "chunks".
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace kiv {

enum Dt { DT_F32 = 0, DT_F16 = 1, DT_BF16 = 2 };

template <int DT> struct Elem;
template <> struct Elem<DT_F32> { enum { BYTES = 4, VEC = 4 }; };
template <> struct Elem<DT_F16> { enum { BYTES = 2, VEC = 8 }; };
template <> struct Elem<DT_BF16> { enum { BYTES = 2, VEC = 8 }; };

__device__ __forceinline__ float bf16_bits_to_f32(uint32_t h) { return __uint_as_float(h << 16); }

// Round-to-nearest-even fp32 -> bf16 (quiet NaN kept).
__device__ __forceinline__ uint32_t f32_to_bf16_bits(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7f800000u) == 0x7f800000u && (u & 0x007fffffu)) return (u >> 16) | 0x40u;
  u += 0x7fffu + ((u >> 16) & 1u);
  return u >> 16;
}

__device__ __forceinline__ float f16_bits_to_f32(uint32_t h) {
  return (float)__builtin_bit_cast(_Float16, (uint16_t)h);
}

// Hardware conversion, round-to-nearest-even.
__device__ __forceinline__ uint32_t f32_to_f16_bits(float f) {
  return (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)f);
}

// Value of x after a round trip through the activation dtype.
template <int DT> __device__ __forceinline__ float round_act(float x) {
  if constexpr (DT == DT_F32) return x;
  else if constexpr (DT == DT_F16) return f16_bits_to_f32(f32_to_f16_bits(x));
  else return bf16_bits_to_f32(f32_to_bf16_bits(x));
}

// Score as a dtype matmul followed by "* scaling" produces it: the fp32
// accumulated dot is rounded to the dtype, multiplied in fp32 by the
// scale and rounded again.  With round == false the score stays fp32.
template <int DT> __device__ __forceinline__ float score_of(float dot, float scale, bool round) {
  if (round) return round_act<DT>(round_act<DT>(dot) * scale);
  return dot * scale;
}

// Returns x unchanged but hides its origin from the optimiser, so that a
// double -> float -> half sequence is not folded into one double -> half
// rounding (which differs from rounding twice on rare values).
__device__ __forceinline__ float opaque_f32(float x) {
  asm volatile("" : "+v"(x));
  return x;
}

// Order-preserving map float -> uint32 (larger float => larger key);
// -0.0 is folded onto +0.0 first so equal values share one key.
__device__ __forceinline__ uint32_t order_key(float f) {
  f = f + 0.0f;
  uint32_t u = __float_as_uint(f);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}
__device__ __forceinline__ float key_to_float(uint32_t k) {
  uint32_t u = (k & 0x80000000u) ? (k & 0x7fffffffu) : ~k;
  return __uint_as_float(u);
}

// One 16-byte chunk held in registers, widened to fp32.
template <int DT> __device__ __forceinline__ void unpack_chunk(const uint4 &v, float *out) {
  if constexpr (DT == DT_F32) {
    out[0] = __uint_as_float(v.x); out[1] = __uint_as_float(v.y);
    out[2] = __uint_as_float(v.z); out[3] = __uint_as_float(v.w);
  } else {
    const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      if constexpr (DT == DT_BF16) {
        out[2 * i] = __uint_as_float(w[i] << 16);
        out[2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u);
      } else {
        out[2 * i] = f16_bits_to_f32(w[i] & 0xffffu);
        out[2 * i + 1] = f16_bits_to_f32(w[i] >> 16);
      }
    }
  }
}

// 16-byte load of one chunk, widened to fp32.
template <int DT> __device__ __forceinline__ void load_chunk(const void *p, float *out) {
  unpack_chunk<DT>(*reinterpret_cast<const uint4 *>(p), out);
}

// Store VEC fp32 values rounded (RNE) to the dtype as one 16-byte chunk.
template <int DT> __device__ __forceinline__ void store_chunk(void *p, const float *in) {
  uint4 v;
  if constexpr (DT == DT_F32) {
    v.x = __float_as_uint(in[0]); v.y = __float_as_uint(in[1]);
    v.z = __float_as_uint(in[2]); v.w = __float_as_uint(in[3]);
  } else {
    uint32_t w[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      uint32_t lo, hi;
      if constexpr (DT == DT_BF16) { lo = f32_to_bf16_bits(in[2 * i]); hi = f32_to_bf16_bits(in[2 * i + 1]); }
      else { lo = f32_to_f16_bits(in[2 * i]); hi = f32_to_f16_bits(in[2 * i + 1]); }
      w[i] = (lo & 0xffffu) | (hi << 16);
    }
    v.x = w[0]; v.y = w[1]; v.z = w[2]; v.w = w[3];
  }
  *reinterpret_cast<uint4 *>(p) = v;
}

// Single element (mask values, summaries) load / store.
template <int DT> __device__ __forceinline__ float load_elem(const void *p, int64_t i) {
  if constexpr (DT == DT_F32) return reinterpret_cast<const float *>(p)[i];
  else if constexpr (DT == DT_F16) return f16_bits_to_f32(reinterpret_cast<const uint16_t *>(p)[i]);
  else return bf16_bits_to_f32(reinterpret_cast<const uint16_t *>(p)[i]);
}
template <int DT> __device__ __forceinline__ void store_elem(void *p, int64_t i, float x) {
  if constexpr (DT == DT_F32) reinterpret_cast<float *>(p)[i] = x;
  else if constexpr (DT == DT_F16) reinterpret_cast<uint16_t *>(p)[i] = (uint16_t)f32_to_f16_bits(x);
  else reinterpret_cast<uint16_t *>(p)[i] = (uint16_t)f32_to_bf16_bits(x);
}

// ---- cross-lane reductions (VALU only: DPP and gfx950 permlane swaps)
// DPP controls: quad_perm [1,0,3,2] = 0xB1, [2,3,0,1] = 0x4E, row_ror:n =
// 0x120 + n, row_half_mirror = 0x141, row_mirror = 0x140.
template <int CTRL> __device__ __forceinline__ float dpp_f32(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, true));
}
template <int CTRL> __device__ __forceinline__ int dpp_i32(int v) {
  return __builtin_amdgcn_update_dpp(0, v, CTRL, 0xF, 0xF, true);
}
// Sum of lane i and lane i ^ 16 (rows of 16 lanes, swapped in pairs).
__device__ __forceinline__ float row_pair_sum(float v) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
// Sum of lane i and lane i ^ 32.
__device__ __forceinline__ float half_wave_sum(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float row_pair_max(float v) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float half_wave_max(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}

// AND and OR over the wave; every lane gets both.  All 64 lanes must be
// active (DPP reads of inactive lanes return 0).
__device__ __forceinline__ void wave_and_or_u32(uint32_t &a, uint32_t &o) {
  a &= (uint32_t)dpp_i32<0xB1>((int)a);
  o |= (uint32_t)dpp_i32<0xB1>((int)o);
  a &= (uint32_t)dpp_i32<0x4E>((int)a);
  o |= (uint32_t)dpp_i32<0x4E>((int)o);
  a &= (uint32_t)dpp_i32<0x141>((int)a);
  o |= (uint32_t)dpp_i32<0x141>((int)o);
  a &= (uint32_t)dpp_i32<0x140>((int)a);
  o |= (uint32_t)dpp_i32<0x140>((int)o);
  const auto ra = __builtin_amdgcn_permlane16_swap(a, a, false, false);
  const auto ro = __builtin_amdgcn_permlane16_swap(o, o, false, false);
  a = ra[0] & ra[1];
  o = ro[0] | ro[1];
  const auto sa = __builtin_amdgcn_permlane32_swap(a, a, false, false);
  const auto so = __builtin_amdgcn_permlane32_swap(o, o, false, false);
  a = sa[0] & sa[1];
  o = so[0] | so[1];
}

// Minimum over the wave; every lane gets it.  All 64 lanes must be active.
__device__ __forceinline__ uint32_t wave_min_u32(uint32_t v) {
  v = min(v, (uint32_t)dpp_i32<0xB1>((int)v));
  v = min(v, (uint32_t)dpp_i32<0x4E>((int)v));
  v = min(v, (uint32_t)dpp_i32<0x141>((int)v));
  v = min(v, (uint32_t)dpp_i32<0x140>((int)v));
  const auto r = __builtin_amdgcn_permlane16_swap(v, v, false, false);
  v = min(r[0], r[1]);
  const auto t = __builtin_amdgcn_permlane32_swap(v, v, false, false);
  return min(t[0], t[1]);
}

// Maximum over the wave; every lane gets it.  All 64 lanes must be active.
__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) {
  v = max(v, (uint32_t)dpp_i32<0xB1>((int)v));
  v = max(v, (uint32_t)dpp_i32<0x4E>((int)v));
  v = max(v, (uint32_t)dpp_i32<0x141>((int)v));
  v = max(v, (uint32_t)dpp_i32<0x140>((int)v));
  const auto r = __builtin_amdgcn_permlane16_swap(v, v, false, false);
  v = max(r[0], r[1]);
  const auto t = __builtin_amdgcn_permlane32_swap(v, v, false, false);
  return max(t[0], t[1]);
}

// Number of set bits of a wave mask below the calling lane.
__device__ __forceinline__ int lane_rank(uint64_t mask) {
  return (int)__builtin_amdgcn_mbcnt_hi((uint32_t)(mask >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)mask, 0u));
}

// The value of the first active lane, as a wave-uniform (scalar) value.
__device__ __forceinline__ uint32_t uniform_u32(uint32_t x) { return (uint32_t)__builtin_amdgcn_readfirstlane((int)x); }
__device__ __forceinline__ uint64_t uniform_u64(uint64_t x) {
  return ((uint64_t)uniform_u32((uint32_t)(x >> 32)) << 32) | uniform_u32((uint32_t)x);
}

// Sum over an aligned group of LG lanes; every lane of the group gets it.
template <int LG> __device__ __forceinline__ float group_sum(float v) {
  if constexpr (LG >= 2) v += dpp_f32<0xB1>(v);
  if constexpr (LG >= 4) v += dpp_f32<0x4E>(v);
  if constexpr (LG >= 8) v += dpp_f32<0x141>(v);
  if constexpr (LG >= 16) v += dpp_f32<0x140>(v);
  if constexpr (LG >= 32) v = row_pair_sum(v);
  if constexpr (LG >= 64) v = half_wave_sum(v);
  return v;
}

// Sum over the 64 / LG groups of a wave, lane by lane within the group
// (lane i adds lanes i + LG, i + 2 LG, ...); every lane gets its column sum.
template <int LG> __device__ __forceinline__ float across_groups_sum(float v) {
  if constexpr (LG <= 1) v += dpp_f32<0x121>(v);
  if constexpr (LG <= 2) v += dpp_f32<0x122>(v);
  if constexpr (LG <= 4) v += dpp_f32<0x124>(v);
  if constexpr (LG <= 8) v += dpp_f32<0x128>(v);
  if constexpr (LG <= 16) v = row_pair_sum(v);
  if constexpr (LG <= 32) v = half_wave_sum(v);
  return v;
}

__device__ __forceinline__ float wave_max(float v) {
  v = fmaxf(v, dpp_f32<0xB1>(v));
  v = fmaxf(v, dpp_f32<0x4E>(v));
  v = fmaxf(v, dpp_f32<0x141>(v));
  v = fmaxf(v, dpp_f32<0x140>(v));
  v = row_pair_max(v);
  return half_wave_max(v);
}
__device__ __forceinline__ float wave_sum(float v) { return group_sum<64>(v); }

__device__ __forceinline__ int wave_sum_i32(int v) {
  v += dpp_i32<0xB1>(v);
  v += dpp_i32<0x4E>(v);
  v += dpp_i32<0x141>(v);
  v += dpp_i32<0x140>(v);
  const auto r = __builtin_amdgcn_permlane16_swap((uint32_t)v, (uint32_t)v, false, false);
  v = (int)(r[0] + r[1]);
  const auto r2 = __builtin_amdgcn_permlane32_swap((uint32_t)v, (uint32_t)v, false, false);
  return (int)(r2[0] + r2[1]);
}

// ---- packed dot products of one 16-byte chunk (fp32 accumulation)
// The last pair is always accumulated with plain FMAs: every result of this
// helper feeds a DPP reduction, and a v_dot2c result read directly by a DPP
// operand needs more wait states than the compiler inserts after an EXEC
// restore (measured on gfx950: wrong sums for 8-lane groups).  A plain FMA
// as the final writer keeps the DPP read on the ordinary VALU hazard path.
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));

// D += A B on one 16x16 tile, K = 32 (8 consecutive k of one A row / B column per lane).
template <int DT> __device__ __forceinline__ f32x4_t mfma_16x16x32(const uint4 &a, const uint4 &b, f32x4_t c) {
  if constexpr (DT == DT_BF16)
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a), __builtin_bit_cast(bf16x8_t, b),
                                                    c, 0, 0, 0);
  else
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8_t, a), __builtin_bit_cast(f16x8_t, b), c,
                                                   0, 0, 0);
}

template <int DT> __device__ __forceinline__ float chunk_dot(const uint4 &x, const uint4 &q, float acc) {
  if constexpr (DT == DT_BF16) {
    acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, x.x), __builtin_bit_cast(bf16x2_t, q.x), acc, false);
    acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, x.y), __builtin_bit_cast(bf16x2_t, q.y), acc, false);
    acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, x.z), __builtin_bit_cast(bf16x2_t, q.z), acc, false);
    acc = fmaf(__uint_as_float(x.w << 16), __uint_as_float(q.w << 16), acc);
    acc = fmaf(__uint_as_float(x.w & 0xffff0000u), __uint_as_float(q.w & 0xffff0000u), acc);
  } else if constexpr (DT == DT_F16) {
    acc = __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2_t, x.x), __builtin_bit_cast(f16x2_t, q.x), acc, false);
    acc = __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2_t, x.y), __builtin_bit_cast(f16x2_t, q.y), acc, false);
    acc = __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2_t, x.z), __builtin_bit_cast(f16x2_t, q.z), acc, false);
    acc = fmaf(f16_bits_to_f32(x.w & 0xffffu), f16_bits_to_f32(q.w & 0xffffu), acc);
    acc = fmaf(f16_bits_to_f32(x.w >> 16), f16_bits_to_f32(q.w >> 16), acc);
  } else {
    acc = fmaf(__uint_as_float(x.x), __uint_as_float(q.x), acc);
    acc = fmaf(__uint_as_float(x.y), __uint_as_float(q.y), acc);
    acc = fmaf(__uint_as_float(x.z), __uint_as_float(q.z), acc);
    acc = fmaf(__uint_as_float(x.w), __uint_as_float(q.w), acc);
  }
  return acc;
}

__device__ __forceinline__ uint4 load16(const void *p) { return *reinterpret_cast<const uint4 *>(p); }
// Raw buffer of `bytes` bytes at `base` (a block-uniform address, kept in
// SGPRs).  A load whose offset is at or past `bytes` returns zeros without
// touching memory.  Offsets stay below 2^31.  Buffer loads count only in
// vmcnt (a flat load also counts in lgkmcnt, which every LDS wait and
// barrier drains).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t tile_rsrc(const char *base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<char *>(base), (short)0, (int)bytes, 0x00020000);
}
__device__ __forceinline__ uint4 buf_load16(__amdgpu_buffer_rsrc_t r, uint32_t voff) {
  typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
  const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(r, (int)voff, 0, 0);
  return make_uint4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ uint32_t buf_load4(__amdgpu_buffer_rsrc_t r, uint32_t voff) {
  return __builtin_amdgcn_raw_buffer_load_b32(r, (int)voff, 0, 0);
}

// Evicted rows that one extra block per kv row of another launch copies
// into the partial page (count 0: none): token t of row r = b*hkv + h goes
// from the strided input (element strides, in16 = 16 / element bytes
// elements per chunk) to partial slot t_dst0 + t.  Used only by launches
// that do not read the partial page themselves.
// Rows a retrieval writes in its first launch: `count` evicted rows into
// the partial page (from k / v, element strides ks* / vs*), and
// `hot_count` rows into the caller's hot window (from hk / hv to dk / dv,
// element strides hks* / hvs* / dks* / dvs*).  One block per kv row r.
struct AppendRows {
  const char *k, *v;
  int64_t ks0, ks1, ks2, vs0, vs1, vs2;
  char *part_k, *part_v;
  int64_t t_dst0;
  int count, hkv, page_size, cpr, in16;
  const char *hk, *hv;
  char *dk, *dv;
  int64_t hks0, hks1, hks2, hvs0, hvs1, hvs2, dks0, dks1, dks2, dvs0, dvs1, dvs2;
  int hot_count;
};

__device__ __forceinline__ void append_rows(const AppendRows &ap, int r) {
  const int b = r / ap.hkv, h = r % ap.hkv;
  const int eb = 16 / ap.in16;
  for (int i = threadIdx.x; i < ap.count * ap.cpr; i += blockDim.x) {
    const int t = i / ap.cpr, c = i % ap.cpr;
    const int64_t e0 = (int64_t)c * ap.in16;
    const int64_t src_k = ((int64_t)b * ap.ks0 + (int64_t)h * ap.ks1 + (int64_t)t * ap.ks2 + e0) * eb;
    const int64_t src_v = ((int64_t)b * ap.vs0 + (int64_t)h * ap.vs1 + (int64_t)t * ap.vs2 + e0) * eb;
    const int64_t dst = (((int64_t)r * ap.page_size + ap.t_dst0 + t) * ap.cpr + c) * 16;
    *reinterpret_cast<uint4 *>(ap.part_k + dst) = load16(ap.k + src_k);
    *reinterpret_cast<uint4 *>(ap.part_v + dst) = load16(ap.v + src_v);
  }
  for (int i = threadIdx.x; i < ap.hot_count * ap.cpr; i += blockDim.x) {
    const int t = i / ap.cpr, c = i % ap.cpr;
    const int64_t e0 = (int64_t)c * ap.in16;
    const int64_t sk = ((int64_t)b * ap.hks0 + (int64_t)h * ap.hks1 + (int64_t)t * ap.hks2 + e0) * eb;
    const int64_t sv = ((int64_t)b * ap.hvs0 + (int64_t)h * ap.hvs1 + (int64_t)t * ap.hvs2 + e0) * eb;
    const int64_t tk = ((int64_t)b * ap.dks0 + (int64_t)h * ap.dks1 + (int64_t)t * ap.dks2 + e0) * eb;
    const int64_t tv = ((int64_t)b * ap.dvs0 + (int64_t)h * ap.dvs1 + (int64_t)t * ap.dvs2 + e0) * eb;
    *reinterpret_cast<uint4 *>(ap.dk + tk) = load16(ap.hk + sk);
    *reinterpret_cast<uint4 *>(ap.dv + tv) = load16(ap.hv + sv);
  }
}

// Inclusive prefix sum over the NT threads of a block.  `tmp` is LDS with
// room for NT / 64 ints.  Contains two barriers; every thread must call it.
template <int NT> __device__ __forceinline__ int block_incl_scan(int v, int *tmp, int *total) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    int t = __shfl_up(v, o, 64);
    if (lane >= o) v += t;
  }
  if (lane == 63) tmp[wave] = v;
  __syncthreads();
  int before = 0, all = 0;
#pragma unroll
  for (int w = 0; w < NT / 64; ++w) {
    int t = tmp[w];
    before += (w < wave) ? t : 0;
    all += t;
  }
  if (total) *total = all;
  __syncthreads();
  return v + before;
}

}  // namespace kiv
