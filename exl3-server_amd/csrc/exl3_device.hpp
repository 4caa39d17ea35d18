// Device-side building blocks shared by every EXL3 kernel (gfx950, wave64).
//
// Format (reference exl3.h:4-21, exl3.cpp:55-107): one 16x16 tile is 8*K little-endian
// 32-bit ring words (256*K bits, read MSB first). Stream position p's 16-bit state is
// the window of ring bits ending (exclusive) at bit (p+1)*K; p = L*8 + i (L = one of
// 32 "reference lanes") maps to tile element row = 2*(L%4) + {0,1,8,9}[i%4],
// col = L/4 + 8*(i/4).
//
// In the GEMV kernels eight lanes share a tile: lane m of a tile holds that tile's ring
// words [m*K, m*K+K) plus the word just before them, which is exactly the bit range
// of reference lanes 4m..4m+3, i.e. all 16 k-rows of output columns m and m+8 (the
// wave-step layout over tiles is in qmv_core.hpp).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

typedef _Float16 f16;
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));

namespace exl3d {

constexpr float kHadScale = 1.0f / 11.313708498984761f;  // 1/sqrt(128), f32

template <typename T, typename U>
__device__ __forceinline__ T bitcast(U u) {
  static_assert(sizeof(T) == sizeof(U), "bitcast size");
  return __builtin_bit_cast(T, u);
}

// Materialises an f32 value in a register. Every f32 -> f16 conversion goes through it:
// the backend otherwise folds fptrunc(fmul) (and fptrunc(fadd)) into v_fma_mixlo_f16,
// which rounds the exact result once, straight to f16, where the reference rounds to
// f32 first and then to f16.
__device__ __forceinline__ float f32_rounded(float v) {
  asm volatile("" : "+v"(v));
  return v;
}
__device__ __forceinline__ f16 to_f16(float v) { return (f16)f32_rounded(v); }
__device__ __forceinline__ float f16_to_f32(uint16_t h) { return (float)bitcast<f16>(h); }
__device__ __forceinline__ uint16_t f32_to_f16(float v) { return bitcast<uint16_t>(to_f16(v)); }
// Two f32 values rounded to f16 and packed (a in the low half): one v_cvt_pk_f16_f32 on
// gfx950 (round to nearest even, as v_cvt_f16_f32), in place of two conversions and an or.
__device__ __forceinline__ uint32_t pack_f16x2(float a, float b) {
  const f16x2 v = {to_f16(a), to_f16(b)};
  return bitcast<uint32_t>(v);
}

// ---------------------------------------------------------------------------------
// Procedural codebooks (reference exl3.cpp:21-42; GPU form trellis_gemm.cpp:333-356).
// Every intermediate is exact, so the single f16 rounding of the hardware op is the
// reference's rounding: mcg/3inst add two f16 halves, mul1 is one f16 fma.
// ---------------------------------------------------------------------------------
template <int CB>
__device__ __forceinline__ uint32_t cb_hash(uint32_t s) {
  if constexpr (CB == 1) return s * 0xCBAC1FEDu;
  else {
    // 3inst: s * 89226354 + 64248484 (mod 2^32) as the low word of one v_mad_u64_u32.
    // The compiler spells it v_mul_lo_u32 + v_add_u32; the fused form issues at the
    // multiply's rate, so the 3inst decode costs what the mcg one does (K4 decode +
    // MFMA measured on gfx950: 13.2 -> 15.8 weights/clk/CU, every state bit-equal).
    uint64_t r, carry;
    const uint64_t addend = 64248484u;
    asm("v_mad_u64_u32 %0, %1, %2, %3, %4" : "=v"(r), "=s"(carry) : "v"(s), "v"(89226354u), "v"(addend));
    (void)carry;
    return (uint32_t)r;
  }
}

template <int CB>
__device__ __forceinline__ f16 decode_one(uint32_t s) {
  if constexpr (CB == 2) {
    const uint32_t h = s * 0x83DCD12Du;
    const uint32_t sum = __builtin_amdgcn_sad_u8(h, 0u, 0x6400u);  // 0x6400 + byte sum
    const f16 v = bitcast<f16>((uint16_t)sum);
    return __builtin_fmaf16(v, bitcast<f16>((uint16_t)0x1EEE), bitcast<f16>((uint16_t)0xC931));
  } else {
    const uint32_t m = (cb_hash<CB>(s) & 0x8FFF8FFFu) ^ 0x3B603B60u;
    const f16x2 v = bitcast<f16x2>(m);
    return v.x + v.y;
  }
}

// ---------------------------------------------------------------------------------
// Ring windows inside one lane's bit string. W[0] is the word before the lane's own
// words, W[1..K] are its own K words (ring words m*K .. m*K+K-1 of the tile). The lane
// decodes tile positions p = 32*m + t, t = 0..31, whose windows end at local bit
// 32 + (t+1)*K; the state's least significant bit is local bit 31 + (t+1)*K.
// F[w] = the 32 bits straddling W[w-1] | W[w] (low half of W[w-1], high half of W[w]).
// ---------------------------------------------------------------------------------
template <int K, int T>
__device__ __forceinline__ uint32_t lane_state(const uint32_t (&W)[K + 1],
                                               const uint32_t (&F)[K + 1]) {
  constexpr int lsb = 31 + (T + 1) * K;
  constexpr int wi = lsb / 32;
  constexpr int sh = 31 - (lsb % 32);
  if constexpr (sh <= 16) return __builtin_amdgcn_ubfe(W[wi], sh, 16);
  else return __builtin_amdgcn_ubfe(F[wi], sh - 16, 16);
}

template <int K>
__device__ __forceinline__ void lane_funnels(const uint32_t (&W)[K + 1], uint32_t (&F)[K + 1]) {
  F[0] = 0;
#pragma unroll
  for (int w = 1; w <= K; ++w) F[w] = __builtin_amdgcn_alignbit(W[w - 1], W[w], 16);
}


// ---------------------------------------------------------------------------------
// Lane exchange v <- v[lane ^ D] without the LDS crossbar's address arithmetic:
// D = 1, 2: DPP quad permutes; D = 4, 8, 16: ds_swizzle xor mode (within 32 lanes);
// D = 32: v_permlane32_swap (the two wave halves exchanged).
// ---------------------------------------------------------------------------------
template <int D>
__device__ __forceinline__ float xor_lanes(float v) {
  const int iv = __builtin_bit_cast(int, v);
  if constexpr (D == 1) {
    return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(iv, 0xB1, 0xF, 0xF, false));
  } else if constexpr (D == 2) {
    return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(iv, 0x4E, 0xF, 0xF, false));
  } else if constexpr (D == 4 || D == 8 || D == 16) {
    return __builtin_bit_cast(float, __builtin_amdgcn_ds_swizzle(iv, 0x1F | (D << 10)));
  } else {
    static_assert(D == 32, "xor distance");
    // vdst' = (lo: v[i], hi: v[i - 32]), vsrc' = (lo: v[i + 32], hi: v[i])
    const auto r = __builtin_amdgcn_permlane32_swap(iv, iv, false, false);
    const int lane = threadIdx.x & 63;
    return __builtin_bit_cast(float, lane < 32 ? (int)r[1] : (int)r[0]);
  }
}

// ---------------------------------------------------------------------------------
// 128-point Sylvester Hadamard over one wave: lane l holds elements 2l and 2l+1.
// Stage order len = 1, 2, ..., 64 with (x[j], x[j+len]) -> (a + b, a - b), the f32
// association of reference exl3.cpp:140-150 and trellis_gemm.cpp:387-396. NB
// independent vectors go through the stages together, so their lane exchanges overlap.
// ---------------------------------------------------------------------------------
template <int D, int NB>
__device__ __forceinline__ void fwht_stage(float (&v0)[NB], float (&v1)[NB]) {
  const bool upper = ((threadIdx.x & 63) & D) != 0;
  if constexpr (NB == 1) {
    // one vector: a select and an add per value (the per-stage sign register of the
    // form below costs as much, and is kept live across callers' loops)
    const float p0 = xor_lanes<D>(v0[0]), p1 = xor_lanes<D>(v1[0]);
    v0[0] = upper ? (p0 - v0[0]) : (v0[0] + p0);
    v1[0] = upper ? (p1 - v1[0]) : (v1[0] + p1);
    return;
  }
  // upper lanes: p - v, lower lanes: v + p (p = v[lane ^ D]), as one fma(sgn, v, p) per
  // value: sgn * v is exact, so the single rounding gives the same bits (signed zeros
  // included) as the subtraction or addition, in one VALU op instead of a select and
  // an add
  const float sgn = upper ? -1.0f : 1.0f;
  if constexpr (D == 32) {
    // v_permlane32_swap(v, v) gives r0 = (lo: v[i], hi: v[i - 32]) and r1 = (lo:
    // v[i + 32], hi: v[i]): lower lanes v + p = r0 + r1, upper lanes p - v = r0 - r1
#pragma unroll
    for (int i = 0; i < NB; ++i) {
      const int a = __builtin_bit_cast(int, v0[i]), b = __builtin_bit_cast(int, v1[i]);
      const auto ra = __builtin_amdgcn_permlane32_swap(a, a, false, false);
      const auto rb = __builtin_amdgcn_permlane32_swap(b, b, false, false);
      v0[i] = __builtin_fmaf(sgn, __builtin_bit_cast(float, (int)ra[1]), __builtin_bit_cast(float, (int)ra[0]));
      v1[i] = __builtin_fmaf(sgn, __builtin_bit_cast(float, (int)rb[1]), __builtin_bit_cast(float, (int)rb[0]));
    }
  } else {
    float p0[NB], p1[NB];
#pragma unroll
    for (int i = 0; i < NB; ++i) {
      p0[i] = xor_lanes<D>(v0[i]);
      p1[i] = xor_lanes<D>(v1[i]);
    }
#pragma unroll
    for (int i = 0; i < NB; ++i) {
      v0[i] = __builtin_fmaf(sgn, v0[i], p0[i]);
      v1[i] = __builtin_fmaf(sgn, v1[i], p1[i]);
    }
  }
}

template <int NB>
__device__ __forceinline__ void wave_fwht128_n(float (&v0)[NB], float (&v1)[NB]) {
#pragma unroll
  for (int i = 0; i < NB; ++i) {
    const float a = v0[i], b = v1[i];
    v0[i] = a + b;
    v1[i] = a - b;
  }
  fwht_stage<1>(v0, v1);
  fwht_stage<2>(v0, v1);
  fwht_stage<4>(v0, v1);
  fwht_stage<8>(v0, v1);
  fwht_stage<16>(v0, v1);
  fwht_stage<32>(v0, v1);
}

__device__ __forceinline__ void wave_fwht128(float &v0, float &v1) {
  float a[1] = {v0}, b[1] = {v1};
  wave_fwht128_n<1>(a, b);
  v0 = a[0];
  v1 = b[0];
}

// Round-trip helpers for the two sides of a trellis linear (trellis_gemm.cpp:383-399).
// pre : xhat = f16( fwht(f32(x) * f32(s)) * scale )
// post: y    = f16( (fwht(f32(f16(yhat))) * scale) * f32(s) )
// NB independent 128-blocks at once (their butterfly stages interleaved).
template <int NB>
__device__ __forceinline__ void wave_had_pre_n(float (&v0)[NB], float (&v1)[NB],
                                               const float (&s0)[NB], const float (&s1)[NB]) {
#pragma unroll
  for (int i = 0; i < NB; ++i) {
    v0[i] = v0[i] * s0[i];
    v1[i] = v1[i] * s1[i];
  }
  wave_fwht128_n<NB>(v0, v1);
#pragma unroll
  for (int i = 0; i < NB; ++i) {
    v0[i] = f32_rounded(v0[i] * kHadScale);
    v1[i] = f32_rounded(v1[i] * kHadScale);
  }
}

__device__ __forceinline__ void wave_had_pre(float &v0, float &v1, float s0, float s1) {
  v0 = v0 * s0;
  v1 = v1 * s1;
  wave_fwht128(v0, v1);
  v0 = f32_rounded(v0 * kHadScale);
  v1 = f32_rounded(v1 * kHadScale);
}

__device__ __forceinline__ void wave_had_post(float &v0, float &v1, float s0, float s1) {
  v0 = (float)to_f16(v0);
  v1 = (float)to_f16(v1);
  wave_fwht128(v0, v1);
  v0 = f32_rounded(f32_rounded(v0 * kHadScale) * s0);
  v1 = f32_rounded(f32_rounded(v1 * kHadScale) * s1);
}

// NB independent post rotations at once (same arithmetic as wave_had_post).
template <int NB>
__device__ __forceinline__ void wave_had_post_n(float (&v0)[NB], float (&v1)[NB],
                                                const float (&s0)[NB], const float (&s1)[NB]) {
#pragma unroll
  for (int i = 0; i < NB; ++i) {
    v0[i] = (float)to_f16(v0[i]);
    v1[i] = (float)to_f16(v1[i]);
  }
  wave_fwht128_n<NB>(v0, v1);
#pragma unroll
  for (int i = 0; i < NB; ++i) {
    v0[i] = f32_rounded(f32_rounded(v0[i] * kHadScale) * s0[i]);
    v1[i] = f32_rounded(f32_rounded(v1[i] * kHadScale) * s1[i]);
  }
}

}  // namespace exl3d
