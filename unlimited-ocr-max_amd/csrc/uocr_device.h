// Device-side helpers shared by the MoE kernels (gfx950, wave64).
//
// Every rounding here is part of the decode path's arithmetic contract: the
// CPU oracle evaluates the same steps in the same order, so results agree bit
// for bit.  The build passes -ffp-contract=off, so the only fused
// multiply-adds are the explicit __builtin_fmaf calls.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "uocr_kernels.h"

namespace uocr {

constexpr int kWave = 64;

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef uint64_t u64x2 __attribute__((ext_vector_type(2)));

#define UOCR_GLOBAL __attribute__((address_space(1)))
#define UOCR_CONST __attribute__((address_space(4)))

// A 16-byte global load that bypasses cache retention: the expert weights
// are read once per call, so they should not evict activations and tables.
// (Pointers reach the kernels inside argument structs, where the compiler
// sees generic pointers; the casts state the global address space.)
#ifndef UOCR_WEIGHT_NT
#define UOCR_WEIGHT_NT 1
#endif
__device__ __forceinline__ i32x4 load_w16(const void* p) {
#if UOCR_WEIGHT_NT
  return __builtin_nontemporal_load((const UOCR_GLOBAL i32x4*)p);
#else
  return *(const UOCR_GLOBAL i32x4*)p;
#endif
}
__device__ __forceinline__ int4 load_nt16(const void* p) {
  const i32x4 v = load_w16(p);
  return make_int4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ uint4 load_nt16u(const void* p) {
  const i32x4 v = load_w16(p);
  return make_uint4((uint32_t)v.x, (uint32_t)v.y, (uint32_t)v.z, (uint32_t)v.w);
}

__device__ __forceinline__ float4 ldg_f4(const void* p) {
  const f32x4 v = *(const UOCR_GLOBAL f32x4*)p;
  return make_float4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ uint4 ldg_u4(const void* p) {
  const i32x4 v = *(const UOCR_GLOBAL i32x4*)p;
  return make_uint4((uint32_t)v.x, (uint32_t)v.y, (uint32_t)v.z, (uint32_t)v.w);
}

// Plain global load of a scalar.
template <typename T>
__device__ __forceinline__ T ldg(const T* p) {
  return *(const UOCR_GLOBAL T*)p;
}

// A load of memory no thread writes during the kernel, through the constant
// address space: at a wave-uniform address it becomes a scalar load.
template <typename T>
__device__ __forceinline__ T ldc(const T* p) {
  return *(const UOCR_CONST T*)p;
}

template <typename T>
__device__ __forceinline__ void stg(T* p, T v) {
  *(UOCR_GLOBAL T*)p = v;
}

__device__ __forceinline__ float bf16_bits_to_f32(uint32_t bits16) {
  return __uint_as_float(bits16 << 16);
}

// The low and high bf16 of a packed pair, widened exactly.
__device__ __forceinline__ float bf16_lo(uint32_t pair) { return __uint_as_float(pair << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t pair) { return __uint_as_float(pair & 0xFFFF0000u); }

// fp32 -> bf16 bits, round-to-nearest-even, NaN -> 0x7FC0.
__device__ __forceinline__ uint16_t f32_to_bf16_rne(float f) {
  if (f != f) return 0x7FC0;
  uint32_t u = __float_as_uint(f);
  u += 0x7FFFu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

// Two fp32 -> packed bf16 pair (lo in the low half), round-to-nearest-even
// (v_cvt_pk_bf16_f32).  Same bits as f32_to_bf16_rne for every non-NaN input.
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  bf16x2 v;
  v.x = (__bf16)lo;
  v.y = (__bf16)hi;
  return __builtin_bit_cast(uint32_t, v);
}

// Workgroup barrier ordering LDS only.  __syncthreads() fences every address
// space, which on gfx950 waits for all outstanding global loads (vmcnt(0)) and
// so cancels any register prefetch in flight across it; this one waits for
// LDS traffic alone.
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// Signed byte B (0..3) of a packed word, converted exactly to fp32 in one
// instruction: v_cvt_f32_i32 with an SDWA byte select and sign extension.
template <int B>
__device__ __forceinline__ float i8_to_f32(int v) {
  float r;
  if constexpr (B == 0)
    asm("v_cvt_f32_i32_sdwa %0, sext(%1) dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:BYTE_0" : "=v"(r) : "v"(v));
  else if constexpr (B == 1)
    asm("v_cvt_f32_i32_sdwa %0, sext(%1) dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:BYTE_1" : "=v"(r) : "v"(v));
  else if constexpr (B == 2)
    asm("v_cvt_f32_i32_sdwa %0, sext(%1) dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:BYTE_2" : "=v"(r) : "v"(v));
  else
    asm("v_cvt_f32_i32_sdwa %0, sext(%1) dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:BYTE_3" : "=v"(r) : "v"(v));
  return r;
}

__device__ __forceinline__ float pow2i(int n) { return __uint_as_float((uint32_t)(n + 127) << 23); }

// exp(x): Cody-Waite reduction by ln 2 (16-bit head + tail), the degree-7
// Taylor polynomial of e^r on |r| <= ln2/2 in Horner form, two exact
// power-of-two scalings.  Within 2 ulp of exp over the fp32 range.
__device__ __forceinline__ float uexp(float x) {
  if (x != x) return x;
  if (x > 88.72283f) return __builtin_huge_valf();
  if (x < -103.972f) return 0.0f;
  const float t = x * 1.44269502f;
  const float n = __builtin_rintf(t);
  float r = __builtin_fmaf(-n, 0.693145751953125f, x);
  r = __builtin_fmaf(-n, 1.42860677e-06f, r);
  float p = 1.98412701e-04f;
  p = __builtin_fmaf(p, r, 1.38888892e-03f);
  p = __builtin_fmaf(p, r, 8.33333377e-03f);
  p = __builtin_fmaf(p, r, 4.16666679e-02f);
  p = __builtin_fmaf(p, r, 1.66666672e-01f);
  p = __builtin_fmaf(p, r, 0.5f);
  p = __builtin_fmaf(p, r, 1.0f);
  p = __builtin_fmaf(p, r, 1.0f);
  const int ni = (int)n;
  const int n1 = ni / 2;
  const int n2 = ni - n1;
  return (p * pow2i(n1)) * pow2i(n2);
}

// silu(g) = g / (1 + exp(-g)), each step rounded to fp32 (IEEE division).
__device__ __forceinline__ float silu(float g) {
  const float e = uexp(-g);
  const float d = 1.0f + e;
  return g / d;
}

// Halving-tree sum over the 64 lanes: v[l] += v[l + off] for off = 32..1;
// lane 0 ends with the total.  Lanes >= off read lanes past the wave, whose
// values are never used.
__device__ __forceinline__ float wave_tree_sum(float v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v = v + __shfl_down(v, off, kWave);
  return v;
}

__device__ __forceinline__ int lane_id() { return (int)(threadIdx.x & (kWave - 1)); }

// v of lane l + OFF for lanes l < OFF (OFF = 32, 16, 8, 4, 2, 1; other
// lanes get values that are never used): v_permlane32/16_swap for the two
// halving steps across 16-lane rows, DPP row_shl inside a row.  No LDS round
// trip.
template <int OFF>
__device__ __forceinline__ uint32_t from_up(uint32_t v) {
  if constexpr (OFF == 32) return __builtin_amdgcn_permlane32_swap(v, v, false, false)[1];
  else if constexpr (OFF == 16) return __builtin_amdgcn_permlane16_swap(v, v, false, false)[1];
  else return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x100 + OFF, 0xf, 0xf, false);
}
template <int OFF>
__device__ __forceinline__ float from_up(float v) { return __uint_as_float(from_up<OFF>(__float_as_uint(v))); }

// Halving-tree sum over the 64 lanes, v[l] += v[l + off] for off = 32..1,
// broadcast from lane 0 (the same additions, in the same order, as
// wave_tree_sum).
__device__ __forceinline__ float tree_sum(float v) {
  v = v + from_up<32>(v);
  v = v + from_up<16>(v);
  v = v + from_up<8>(v);
  v = v + from_up<4>(v);
  v = v + from_up<2>(v);
  v = v + from_up<1>(v);
  return __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(v)));
}
// tree_sum of N values at once, with the same additions in the same order.
// The two steps across 16-lane rows run on pairs of values:
// permlane32_swap(a, b) leaves [a lo, b lo] and [a hi, b hi], whose sum holds
// a's step-32 partials in lanes 0-31 and b's in lanes 32-63; permlane16_swap
// does the same for rows.  Lane 16 r of out[j] then holds the total of
// v[4 j + tree_row_value(r)] (rows hold values 0, 2, 1, 3 of the quad).
__device__ __forceinline__ int tree_row_value(int r) { return ((r & 1) << 1) | (r >> 1); }
template <int N>
__device__ __forceinline__ void tree_sum_quads(const float (&v)[N], float (&out)[N / 4]) {
  static_assert(N % 4 == 0, "values come in quads");
  float c[N / 2];
#pragma unroll
  for (int i = 0; i < N / 2; ++i) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v[2 * i]), __float_as_uint(v[2 * i + 1]),
                                                    false, false);
    c[i] = __uint_as_float(r[0]) + __uint_as_float(r[1]);
  }
#pragma unroll
  for (int j = 0; j < N / 4; ++j) {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(c[2 * j]), __float_as_uint(c[2 * j + 1]),
                                                    false, false);
    float e = __uint_as_float(r[0]) + __uint_as_float(r[1]);
    e = e + from_up<8>(e);
    e = e + from_up<4>(e);
    e = e + from_up<2>(e);
    e = e + from_up<1>(e);
    out[j] = e;
  }
}
// Inclusive prefix sum over the 64 lanes (lane l: v[0] + ... + v[l]) in DPP
// steps, no LDS round trip: row_shr 1, 2, 4, 8 inside each 16-lane row, then
// row_bcast 15 (a row's last lane into the next row, rows 1 and 3) and
// row_bcast 31 (lane 31 into rows 2 and 3).  Integer sums: exact in any order.
__device__ __forceinline__ int wave_scan_i(int v) {
  const int l = (int)(threadIdx.x & 63);
  const int r = l & 15;
  int t = __builtin_amdgcn_update_dpp(0, v, 0x111, 0xf, 0xf, false);
  if (r >= 1) v += t;
  t = __builtin_amdgcn_update_dpp(0, v, 0x112, 0xf, 0xf, false);
  if (r >= 2) v += t;
  t = __builtin_amdgcn_update_dpp(0, v, 0x114, 0xf, 0xf, false);
  if (r >= 4) v += t;
  t = __builtin_amdgcn_update_dpp(0, v, 0x118, 0xf, 0xf, false);
  if (r >= 8) v += t;
  t = __builtin_amdgcn_update_dpp(0, v, 0x142, 0xf, 0xf, false);
  if ((l & 31) >= 16) v += t;
  t = __builtin_amdgcn_update_dpp(0, v, 0x143, 0xf, 0xf, false);
  if (l >= 32) v += t;
  return v;
}
// Sum over the 64 lanes, broadcast (the halving tree of tree_sum on integers).
__device__ __forceinline__ int wave_sum_i(int v) {
  v += (int)from_up<32>((uint32_t)v);
  v += (int)from_up<16>((uint32_t)v);
  v += (int)from_up<8>((uint32_t)v);
  v += (int)from_up<4>((uint32_t)v);
  v += (int)from_up<2>((uint32_t)v);
  v += (int)from_up<1>((uint32_t)v);
  return __builtin_amdgcn_readfirstlane(v);
}
__device__ __forceinline__ float tree_max(float v) {
  v = fmaxf(v, from_up<32>(v));
  v = fmaxf(v, from_up<16>(v));
  v = fmaxf(v, from_up<8>(v));
  v = fmaxf(v, from_up<4>(v));
  v = fmaxf(v, from_up<2>(v));
  v = fmaxf(v, from_up<1>(v));
  return __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(v)));
}
__device__ __forceinline__ uint32_t tree_umax(uint32_t v) {
  v = max(v, from_up<32>(v));
  v = max(v, from_up<16>(v));
  v = max(v, from_up<8>(v));
  v = max(v, from_up<4>(v));
  v = max(v, from_up<2>(v));
  v = max(v, from_up<1>(v));
  return (uint32_t)__builtin_amdgcn_readfirstlane((int)v);
}
__device__ __forceinline__ uint32_t tree_sum_u32(uint32_t v) {
  v += from_up<32>(v);
  v += from_up<16>(v);
  v += from_up<8>(v);
  v += from_up<4>(v);
  v += from_up<2>(v);
  v += from_up<1>(v);
  return (uint32_t)__builtin_amdgcn_readfirstlane((int)v);
}
__device__ __forceinline__ uint32_t tree_or(uint32_t v) {
  v |= from_up<32>(v);
  v |= from_up<16>(v);
  v |= from_up<8>(v);
  v |= from_up<4>(v);
  v |= from_up<2>(v);
  v |= from_up<1>(v);
  return (uint32_t)__builtin_amdgcn_readfirstlane((int)v);
}


__device__ __forceinline__ int clamp_expert(int32_t key, int E) {
  int e = key;
  e = e < 0 ? 0 : e;
  return e >= E ? E - 1 : e;
}

}  // namespace uocr
