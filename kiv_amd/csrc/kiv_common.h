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

// 16-byte load of one chunk, widened to fp32.
template <int DT> __device__ __forceinline__ void load_chunk(const void *p, float *out) {
  const uint4 v = *reinterpret_cast<const uint4 *>(p);
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

// Sum over an aligned group of LG lanes (butterfly; every lane gets the sum).
template <int LG> __device__ __forceinline__ float group_sum(float v) {
#pragma unroll
  for (int m = LG / 2; m >= 1; m >>= 1) v += __shfl_xor(v, m, LG);
  return v;
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) v = fmaxf(v, __shfl_xor(v, m, 64));
  return v;
}
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) v += __shfl_xor(v, m, 64);
  return v;
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

// Agent-scope (whole-GPU) atomics and coherent loads/stores for data that
// blocks of one grid exchange.
__device__ __forceinline__ int atomic_add_acq_rel(int *p, int v) {
  return __hip_atomic_fetch_add(p, v, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void coherent_store_u32(uint32_t *p, uint32_t v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint32_t coherent_load_u32(uint32_t *p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void coherent_store_f32(float *p, float v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float coherent_load_f32(float *p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

}  // namespace kiv
