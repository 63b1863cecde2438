// Device-side helpers for the gfx950 decoder KV-cache kernels: 16-byte element
// vectors for fp32/fp16/bf16, fp32 dot products on packed halves, wave64 lane
// exchanges, and the (max, sum, acc) merge of online softmax states.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "speech_kv.h"

namespace skv {

constexpr float kNegInf = -__builtin_huge_valf();
constexpr float kLog2e = 1.4426950408889634f;

typedef _Float16 half2v __attribute__((ext_vector_type(2)));
typedef __bf16 bf162v __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// 16-byte streaming load (nontemporal hint: K/V rows are read exactly once).
__device__ __forceinline__ uint4 load_stream(const uint4* p) {
  const u32x4 v = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
  return make_uint4(v.x, v.y, v.z, v.w);
}

// 16-byte streaming store (nontemporal hint): for bulk copies whose destination is not
// read again by the same kernel.
__device__ __forceinline__ void store_stream(uint4* p, const uint4& v) {
  __builtin_nontemporal_store(u32x4{v.x, v.y, v.z, v.w}, reinterpret_cast<u32x4*>(p));
}

// Element traits: EPL = elements carried by one 16-byte lane load.
template <int DT> struct Elt;
template <> struct Elt<SKV_F32> { static constexpr int EPL = 4; };
template <> struct Elt<SKV_F16> { static constexpr int EPL = 8; };
template <> struct Elt<SKV_BF16> { static constexpr int EPL = 8; };

__device__ __forceinline__ float bf16_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }

// Round-to-nearest-even fp32 -> bf16 bits (NaN stays NaN), matching torch's cast.
__device__ __forceinline__ uint32_t f32_to_bf16_bits(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (u >> 16) | 0x40u;
  u += 0x7fffu + ((u >> 16) & 1u);
  return u >> 16;
}

__device__ __forceinline__ uint32_t pack_half2(float a, float b) {
  _Float16 ha = (_Float16)a, hb = (_Float16)b;
  uint16_t ua = __builtin_bit_cast(uint16_t, ha), ub = __builtin_bit_cast(uint16_t, hb);
  return (uint32_t)ua | ((uint32_t)ub << 16);
}

// Sum over the EPL lane elements of q*k in fp32. fp16/bf16 use the packed
// v_dot2_f32_{f16,bf16} (products of 16-bit values are exact in fp32).
template <int DT> __device__ __forceinline__ float dot16(const uint4& q, const uint4& k);
template <> __device__ __forceinline__ float dot16<SKV_F32>(const uint4& q, const uint4& k) {
  float s = __uint_as_float(q.x) * __uint_as_float(k.x);
  s = fmaf(__uint_as_float(q.y), __uint_as_float(k.y), s);
  s = fmaf(__uint_as_float(q.z), __uint_as_float(k.z), s);
  s = fmaf(__uint_as_float(q.w), __uint_as_float(k.w), s);
  return s;
}
template <> __device__ __forceinline__ float dot16<SKV_F16>(const uint4& q, const uint4& k) {
  float s = __builtin_amdgcn_fdot2(__builtin_bit_cast(half2v, q.x), __builtin_bit_cast(half2v, k.x), 0.f, false);
  s = __builtin_amdgcn_fdot2(__builtin_bit_cast(half2v, q.y), __builtin_bit_cast(half2v, k.y), s, false);
  s = __builtin_amdgcn_fdot2(__builtin_bit_cast(half2v, q.z), __builtin_bit_cast(half2v, k.z), s, false);
  s = __builtin_amdgcn_fdot2(__builtin_bit_cast(half2v, q.w), __builtin_bit_cast(half2v, k.w), s, false);
  return s;
}
template <> __device__ __forceinline__ float dot16<SKV_BF16>(const uint4& q, const uint4& k) {
  float s = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf162v, q.x), __builtin_bit_cast(bf162v, k.x), 0.f, false);
  s = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf162v, q.y), __builtin_bit_cast(bf162v, k.y), s, false);
  s = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf162v, q.z), __builtin_bit_cast(bf162v, k.z), s, false);
  s = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf162v, q.w), __builtin_bit_cast(bf162v, k.w), s, false);
  return s;
}

// acc[e] += p * v[e] for the EPL elements of one 16-byte vector.
template <int DT> __device__ __forceinline__ void axpy16(float p, const uint4& v, float* acc);
template <> __device__ __forceinline__ void axpy16<SKV_F32>(float p, const uint4& v, float* acc) {
  acc[0] = fmaf(p, __uint_as_float(v.x), acc[0]);
  acc[1] = fmaf(p, __uint_as_float(v.y), acc[1]);
  acc[2] = fmaf(p, __uint_as_float(v.z), acc[2]);
  acc[3] = fmaf(p, __uint_as_float(v.w), acc[3]);
}
template <> __device__ __forceinline__ void axpy16<SKV_F16>(float p, const uint4& v, float* acc) {
  const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    half2v h = __builtin_bit_cast(half2v, w[i]);
    acc[2 * i] = fmaf(p, (float)h.x, acc[2 * i]);
    acc[2 * i + 1] = fmaf(p, (float)h.y, acc[2 * i + 1]);
  }
}
template <> __device__ __forceinline__ void axpy16<SKV_BF16>(float p, const uint4& v, float* acc) {
  const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    acc[2 * i] = fmaf(p, bf16_lo(w[i]), acc[2 * i]);
    acc[2 * i + 1] = fmaf(p, bf16_hi(w[i]), acc[2 * i + 1]);
  }
}

// Pack EPL fp32 values into one 16-byte vector of the output dtype.
template <int DT> __device__ __forceinline__ uint4 pack16(const float* a);
template <> __device__ __forceinline__ uint4 pack16<SKV_F32>(const float* a) {
  return make_uint4(__float_as_uint(a[0]), __float_as_uint(a[1]), __float_as_uint(a[2]), __float_as_uint(a[3]));
}
template <> __device__ __forceinline__ uint4 pack16<SKV_F16>(const float* a) {
  return make_uint4(pack_half2(a[0], a[1]), pack_half2(a[2], a[3]), pack_half2(a[4], a[5]), pack_half2(a[6], a[7]));
}
template <> __device__ __forceinline__ uint4 pack16<SKV_BF16>(const float* a) {
  uint4 r;
  r.x = f32_to_bf16_bits(a[0]) | (f32_to_bf16_bits(a[1]) << 16);
  r.y = f32_to_bf16_bits(a[2]) | (f32_to_bf16_bits(a[3]) << 16);
  r.z = f32_to_bf16_bits(a[4]) | (f32_to_bf16_bits(a[5]) << 16);
  r.w = f32_to_bf16_bits(a[6]) | (f32_to_bf16_bits(a[7]) << 16);
  return r;
}

__device__ __forceinline__ int lane_id() {
  return (int)__builtin_amdgcn_mbcnt_hi(~0u, __builtin_amdgcn_mbcnt_lo(~0u, 0u));
}

// DPP controls (gfx9 encoding) used below; each reads lane f(i) into lane i.
constexpr int kDppXor1 = 0xB1;        // quad_perm [1,0,3,2]: i ^ 1
constexpr int kDppXor2 = 0x4E;        // quad_perm [2,3,0,1]: i ^ 2
constexpr int kDppXor3 = 0x1B;        // quad_perm [3,2,1,0]: i ^ 3
constexpr int kDppHalfMirror = 0x141; // i ^ 7 (mirror of each 8-lane half row)
constexpr int kDppRowMirror = 0x140;  // i ^ 15 (mirror of each 16-lane row)

// A DPP read with no old value to keep (bound_ctrl): the compiler then folds the
// permute into the instruction that consumes it (one v_add_f32_dpp per
// reduction step instead of a copy, a v_mov_b32_dpp and the add).
template <int CTRL> __device__ __forceinline__ float dpp(float x) {
  return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(x), CTRL, 0xF, 0xF, true));
}

// Value of lane (lane ^ OFF), all in VALU and with every lane active (a DPP
// read of a lane that is switched off returns zero, so no lane-dependent
// branch may surround these): DPP within 16-lane rows, where
// i^4 = (i^3)^7 and i^8 = (i^7)^15 compose two permutes; the gfx950
// permlane16/32 swaps across rows. A swap of a register with itself returns
// {even-half copy, odd-half copy} of the 16/32 split, so the partner's value
// is picked by the lane's OFF bit with a select.
template <int OFF> __device__ __forceinline__ float xor_lane(float x) {
  if constexpr (OFF == 1) {
    return dpp<kDppXor1>(x);
  } else if constexpr (OFF == 2) {
    return dpp<kDppXor2>(x);
  } else if constexpr (OFF == 4) {
    return dpp<kDppXor3>(dpp<kDppHalfMirror>(x));
  } else if constexpr (OFF == 8) {
    return dpp<kDppHalfMirror>(dpp<kDppRowMirror>(x));
  } else if constexpr (OFF == 16) {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return __uint_as_float((lane_id() & 16) ? r[0] : r[1]);
  } else {
    static_assert(OFF == 32, "xor_lane: offset must be a power of two below 64");
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return __uint_as_float((lane_id() & 32) ? r[0] : r[1]);
  }
}

// Maximum of two scores (or running maxima), NaN-propagating: gfx950's v_maximum3_f32, one
// instruction. fmaxf (IEEE maxNum) first quiets each operand the compiler cannot prove
// canonical (a cross-lane result, a loop-carried value): one extra instruction per operand.
__device__ __forceinline__ float max_score(float a, float b) { return __builtin_elementwise_maximum(a, b); }

// Workgroup barrier that orders LDS only. __syncthreads() is also a release of
// global memory, which makes every wave wait for all of its outstanding global
// loads and stores before the barrier; a loop that stages tiles through LDS
// while the next tiles' global loads are in flight needs only the LDS order.
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// Sum over groups of W adjacent lanes (W a power of two <= 64); every lane of
// a group ends with the same bits. After the quad steps all lanes of a quad
// (then of an 8-lane half row) hold one value, so the mirrors pair each lane
// with a lane of the other half: one DPP op per step.
template <int W> __device__ __forceinline__ float group_sum(float x) {
  if constexpr (W >= 2) x += xor_lane<1>(x);
  if constexpr (W >= 4) x += xor_lane<2>(x);
  if constexpr (W >= 8) x += dpp<kDppHalfMirror>(x);
  if constexpr (W >= 16) x += dpp<kDppRowMirror>(x);
  if constexpr (W >= 32) x += xor_lane<16>(x);
  if constexpr (W >= 64) x += xor_lane<32>(x);
  return x;
}

// Merge (m, l, acc) with (m2, l2, a2): both are base-2 online-softmax states.
template <int N>
__device__ __forceinline__ void merge_state(float& m, float& l, float* acc, float m2, float l2, const float* a2) {
  const float mm = fmaxf(m, m2);
  const float ref = (mm == kNegInf) ? 0.f : mm;
  const float s1 = __builtin_amdgcn_exp2f(m - ref);
  const float s2 = __builtin_amdgcn_exp2f(m2 - ref);
  l = l * s1 + l2 * s2;
#pragma unroll
  for (int e = 0; e < N; ++e) acc[e] = acc[e] * s1 + a2[e] * s2;
  m = mm;
}

}  // namespace skv
