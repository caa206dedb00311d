// Device helpers shared by the gfx950 kernels: bf16 conversion, MFMA wrappers,
// cross-lane reductions and the QK-RMSNorm + RoPE row transform.
//
// Lane layout used throughout ("row-quad" layout): a wavefront of 64 lanes holds 16
// rows of head_dim bf16 values. Lane l serves row n = l % 16 and, for every k-step
// t < head_dim / 32, the 8 channels d = 32 t + 8 g + j (j < 8) with g = l / 16. This
// is the operand layout of v_mfma_f32_16x16x32_bf16 (A: row = lane % 16; B: column
// = lane % 16; both take 8 consecutive reduction indices per lane), so a row loaded
// this way is directly an MFMA operand, and a row's sum of squares is a lane-local
// sum followed by two cross-lane steps (xor 16, xor 32).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace fm {

typedef __attribute__((ext_vector_type(8))) __bf16 bf16x8_t;
typedef __attribute__((ext_vector_type(4))) __bf16 bf16x4_t;
typedef __attribute__((ext_vector_type(4))) float f32x4_t;
typedef __attribute__((ext_vector_type(4))) uint32_t u32x4_t;
typedef __attribute__((ext_vector_type(2))) uint32_t u32x2_t;

__device__ __forceinline__ float bf16_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }
__device__ __forceinline__ float bf16_to_f32(uint32_t h) { return __uint_as_float(h << 16); }

typedef __attribute__((ext_vector_type(2))) __bf16 bf16x2_t;

// float32 -> bf16, round to nearest even: gfx950's v_cvt_pk_bf16_f32 (two values per
// instruction).
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  const bf16x2_t v = {(__bf16)lo, (__bf16)hi};
  return __builtin_bit_cast(uint32_t, v);
}
__device__ __forceinline__ float round_bf16(float f) { return (float)(__bf16)f; }

// float32 <-> fp16 (round to nearest even), two values per dword.
typedef __attribute__((ext_vector_type(2))) _Float16 f16x2_t;
__device__ __forceinline__ uint32_t pack_f16x2(float lo, float hi) {
  const f16x2_t v = {(_Float16)lo, (_Float16)hi};
  return __builtin_bit_cast(uint32_t, v);
}
__device__ __forceinline__ float f16_lo(uint32_t w) { return (float)__builtin_bit_cast(f16x2_t, w)[0]; }
__device__ __forceinline__ float f16_hi(uint32_t w) { return (float)__builtin_bit_cast(f16x2_t, w)[1]; }

// D(16x16 f32) += A(16x32 bf16) * B(32x16 bf16); operands as 4 packed dwords.
__device__ __forceinline__ f32x4_t mfma_16x16x32(u32x4_t a, u32x4_t b, f32x4_t c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                  __builtin_bit_cast(bf16x8_t, b), c, 0, 0, 0);
}
// D(16x16 f32) += A(16x16 bf16) * B(16x16 bf16); operands as 2 packed dwords.
__device__ __forceinline__ f32x4_t mfma_16x16x16(u32x2_t a, u32x2_t b, f32x4_t c) {
  return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(__builtin_bit_cast(bf16x4_t, a),
                                                    __builtin_bit_cast(bf16x4_t, b), c, 0, 0, 0);
}

// D(16x16 f32) += A(16x32 e4m3) * B(32x16 e4m3) (gfx950: OCP e4m3); 8 bytes per lane each,
// lane (row / column n, g) holding reduction indices 8 g .. 8 g + 7.
__device__ __forceinline__ f32x4_t mfma_16x16x32_f8(u32x2_t a, u32x2_t b, f32x4_t c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_fp8_fp8(__builtin_bit_cast(long, a), __builtin_bit_cast(long, b), c, 0,
                                                     0, 0);
}

// D(16x16 f32) += A(16x128 e4m3) * B(128x16 e4m3) (v_mfma_scale_f32_16x16x128_f8f6f4, both
// formats e4m3, unit block scales); 32 bytes per lane each. The reduction index's lane
// layout only has to agree between A and B: a lane's 32 bytes of A and of B must hold
// the same 32 channels in the same order.
typedef __attribute__((ext_vector_type(8))) int i32x8_t;
__device__ __forceinline__ f32x4_t mfma_16x16x128_f8(const i32x8_t &a, const i32x8_t &b, f32x4_t c) {
  return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a, b, c, 0, 0, 0, 0x7f7f7f7f, 0, 0x7f7f7f7f);
}
// Two e4m3 values (bytes 0, 1 of w, or 2, 3 with hi) as bf16x2, exactly.
__device__ __forceinline__ uint32_t e4m3x2_to_bf16x2(uint32_t w, bool hi) {
  typedef __attribute__((ext_vector_type(2))) __bf16 b2_t;
  const b2_t v = hi ? __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w, 1.0f, true)
                    : __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w, 1.0f, false);
  return __builtin_bit_cast(uint32_t, v);
}

// Cross-lane pairs with gfx950's v_permlane16_swap / v_permlane32_swap: each returns,
// in every lane l, the two values {v[l], v[l ^ 16]} (resp. {v[l], v[l ^ 32]}) in some
// order, so a symmetric operation of the pair gives the same bits in both lanes.
struct LanePair {
  float a, b;
};
__device__ __forceinline__ LanePair pair16(float v) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return {__uint_as_float(r[0]), __uint_as_float(r[1])};
}
__device__ __forceinline__ LanePair pair32(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return {__uint_as_float(r[0]), __uint_as_float(r[1])};
}
// Reductions over the four lanes l, l^16, l^32, l^48 (the 4 groups of one row); all
// four lanes end with identical bits.
__device__ __forceinline__ float sum_over_groups(float v) {
  LanePair p = pair16(v);
  v = __fadd_rn(p.a, p.b);
  p = pair32(v);
  return __fadd_rn(p.a, p.b);
}
__device__ __forceinline__ float max_over_groups(float v) {
  LanePair p = pair16(v);
  v = fmaxf(p.a, p.b);
  p = pair32(v);
  return fmaxf(p.a, p.b);
}

// The wavefront index inside the workgroup, as a provably wave-uniform (scalar) value,
// so that everything derived from it stays in SGPRs and uniform branches.
__device__ __forceinline__ int wave_id() { return __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6)); }

__device__ __forceinline__ u32x4_t load16(const void *p) {
  return *reinterpret_cast<const u32x4_t *>(p);
}
__device__ __forceinline__ void store16(void *p, u32x4_t v) { *reinterpret_cast<u32x4_t *>(p) = v; }
// Non-temporal (streaming) store, for the bf16 query pass's packed rows and the merged
// attention output: measured to shorten those two kernels (batch-64 paged drafter call:
// 1.5-3 us per call). Not for the split partials or the e4m3 packed rows, which their next
// reader then took longer to fetch, nor for the cache writers, which it slowed.
__device__ __forceinline__ void store16_nt(void *p, u32x4_t v) {
  __builtin_nontemporal_store(v, reinterpret_cast<u32x4_t *>(p));
}

// The rotary table of the kernels: cos/sin of pair i at row r.
struct Rope {
  const float *cos;
  const float *sin;
  int64_t row_stride;
  int64_t pair_stride;
  int64_t rows;  // > 0: clamp the row into [0, rows)
};

__device__ __forceinline__ int64_t clamp_row(const Rope &rope, int64_t r) {
  if (rope.rows > 0) r = r < 0 ? 0 : (r >= rope.rows ? rope.rows - 1 : r);
  return r;
}

// The per-lane operands of the prologue for one row in the row-quad layout (x[t] holds
// channels 32 t + 8 g + (0..7), i.e. the pairs 16 t + 4 g + (0..3)): the norm weights
// of those channels and the rotary cos / sin of those pairs.
template <int D>
struct PrologueOps {
  float w[D / 32][8];
  float c[D / 32][4], s[D / 32][4];
};

typedef __attribute__((ext_vector_type(4), aligned(4))) float f32x4u_t;  // 4-byte aligned
typedef __attribute__((address_space(1))) const f32x4u_t g_f32x4u_t;     // global memory
typedef __attribute__((address_space(1))) const float g_cfloat_t;

// The rotary cos / sin of this lane's pairs at table row rope_row into ops.c / ops.s, with
// global loads (they count on vmcnt only, never on the LDS counter): 16-byte loads where
// the table layout allows (contiguous pairs, or (cos, sin) interleaved), else per element.
template <int D>
__device__ __forceinline__ void load_rope_ops(PrologueOps<D> &ops, const Rope &rope, int64_t rope_row, int g) {
  constexpr int KT = D / 32;
  const float *cs = rope.cos + rope_row * rope.row_stride;
  const float *sn = rope.sin + rope_row * rope.row_stride;
  if (rope.pair_stride == 1) {
#pragma unroll
    for (int t = 0; t < KT; ++t) {
      const f32x4u_t cv = *(g_f32x4u_t *)(cs + 16 * t + 4 * g);
      const f32x4u_t sv = *(g_f32x4u_t *)(sn + 16 * t + 4 * g);
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        ops.c[t][q] = cv[q];
        ops.s[t][q] = sv[q];
      }
    }
  } else if (rope.pair_stride == 2 && sn == cs + 1) {
#pragma unroll
    for (int t = 0; t < KT; ++t) {
      const f32x4u_t v0 = *(g_f32x4u_t *)(cs + 32 * t + 8 * g);
      const f32x4u_t v1 = *(g_f32x4u_t *)(cs + 32 * t + 8 * g + 4);
      ops.c[t][0] = v0[0], ops.s[t][0] = v0[1], ops.c[t][1] = v0[2], ops.s[t][1] = v0[3];
      ops.c[t][2] = v1[0], ops.s[t][2] = v1[1], ops.c[t][3] = v1[2], ops.s[t][3] = v1[3];
    }
  } else {
#pragma unroll
    for (int t = 0; t < KT; ++t)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int64_t p = 16 * t + 4 * g + q;
        ops.c[t][q] = *(g_cfloat_t *)(cs + p * rope.pair_stride);
        ops.s[t][q] = *(g_cfloat_t *)(sn + p * rope.pair_stride);
      }
  }
}

// The norm weights of this lane's channels into ops.w. They depend on no row, so a
// caller whose rotary row waits on a loaded position issues them first: they then share
// the first memory round trip instead of adding one after the position arrives.
template <int D>
__device__ __forceinline__ void load_norm_ops(PrologueOps<D> &ops, const float *__restrict__ w, int g) {
  constexpr int KT = D / 32;
#pragma unroll
  for (int t = 0; t < KT; ++t) {
    const f32x4u_t lo = *(g_f32x4u_t *)(w + 32 * t + 8 * g);
    const f32x4u_t hi = *(g_f32x4u_t *)(w + 32 * t + 8 * g + 4);
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      ops.w[t][q] = lo[q];
      ops.w[t][4 + q] = hi[q];
    }
  }
}

template <int D>
__device__ __forceinline__ void load_prologue_ops(PrologueOps<D> &ops, const float *__restrict__ w,
                                                  const Rope &rope, int64_t rope_row, int g) {
  load_norm_ops<D>(ops, w, g);
  load_rope_ops<D>(ops, rope, rope_row, g);
}

// fp32 products, sums and differences each rounded on its own: never contracted into a
// fused multiply-add, whichever kernel inlines them (the prologue's bits must not depend
// on the surrounding code: the fused and the standalone prologue agree bit for bit).
__device__ __forceinline__ float mul_rn(float a, float b) {
#pragma clang fp contract(off)
  return a * b;
}
__device__ __forceinline__ float add_rn(float a, float b) {
#pragma clang fp contract(off)
  return a + b;
}
__device__ __forceinline__ float sub_rn(float a, float b) {
#pragma clang fp contract(off)
  return a - b;
}

// RMSNorm (scale rounded to bf16 before the multiply, product rounded to bf16) then
// interleaved-pair RoPE (fp32 rotate of the bf16 normed values, rounded to bf16) of one
// row held in the row-quad layout. Every lane of the wavefront must call this (the row
// reduction crosses lane groups). The arithmetic is spelled with explicit
// round-to-nearest operations so that every caller computes bit-identical values:
//   r  = 1 / sqrt(sum(x^2) / D + eps)
//   y  = bf16(x * bf16(w * r))
//   e' = bf16(e c - o s),  o' = bf16(o c + e s)       (each product rounded)
// Follows flashmap/modeling_flashmap.py:61-66,79-80 and flashmap/vllm/kernels.py:84-98.
template <int D>
__device__ __forceinline__ void norm_rope_apply(u32x4_t (&x)[D / 32], const PrologueOps<D> &ops,
                                                float eps) {
  constexpr int KT = D / 32;
  float ss = 0.f;
#pragma unroll
  for (int t = 0; t < KT; ++t) {
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const float e = bf16_lo(x[t][q]), o = bf16_hi(x[t][q]);
      ss = add_rn(ss, mul_rn(e, e));
      ss = add_rn(ss, mul_rn(o, o));
    }
  }
  ss = sum_over_groups(ss);
  const float r = __fdiv_rn(1.0f, __fsqrt_rn(add_rn(__fdiv_rn(ss, (float)D), eps)));
#pragma unroll
  for (int t = 0; t < KT; ++t) {
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const float se = round_bf16(mul_rn(ops.w[t][2 * q], r));
      const float so = round_bf16(mul_rn(ops.w[t][2 * q + 1], r));
      const float e = round_bf16(mul_rn(bf16_lo(x[t][q]), se));
      const float o = round_bf16(mul_rn(bf16_hi(x[t][q]), so));
      const float c = ops.c[t][q], s = ops.s[t][q];
      const float e2 = sub_rn(mul_rn(e, c), mul_rn(o, s));
      const float o2 = add_rn(mul_rn(o, c), mul_rn(e, s));
      x[t][q] = pack_bf16x2(e2, o2);
    }
  }
}

// The same RMSNorm + RoPE with the rotated values left in fp32 (the fp8 writers divide
// them by the cache's scale and quantize them directly): y[t][2q], y[t][2q + 1] = the
// rotated pair 16 t + 4 g + q. SGL: the normed value is rounded once, bf16((x r) w), as
// sglang's fp8 pool writer computes it (flashmap/sglang/kernels.py:326-329); otherwise
// bf16(x bf16(w r)) as above (flashmap/vllm/kernels.py:276-290).
template <int D, bool SGL>
__device__ __forceinline__ void norm_rope_f32(const u32x4_t (&x)[D / 32], const PrologueOps<D> &ops, float eps,
                                              float (&y)[D / 32][8]) {
  constexpr int KT = D / 32;
  float ss = 0.f;
#pragma unroll
  for (int t = 0; t < KT; ++t) {
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const float e = bf16_lo(x[t][q]), o = bf16_hi(x[t][q]);
      ss = add_rn(ss, mul_rn(e, e));
      ss = add_rn(ss, mul_rn(o, o));
    }
  }
  ss = sum_over_groups(ss);
  const float r = __fdiv_rn(1.0f, __fsqrt_rn(add_rn(__fdiv_rn(ss, (float)D), eps)));
#pragma unroll
  for (int t = 0; t < KT; ++t) {
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      float e, o;
      if constexpr (SGL) {
        e = round_bf16(mul_rn(mul_rn(bf16_lo(x[t][q]), r), ops.w[t][2 * q]));
        o = round_bf16(mul_rn(mul_rn(bf16_hi(x[t][q]), r), ops.w[t][2 * q + 1]));
      } else {
        e = round_bf16(mul_rn(bf16_lo(x[t][q]), round_bf16(mul_rn(ops.w[t][2 * q], r))));
        o = round_bf16(mul_rn(bf16_hi(x[t][q]), round_bf16(mul_rn(ops.w[t][2 * q + 1], r))));
      }
      const float c = ops.c[t][q], s = ops.s[t][q];
      y[t][2 * q] = sub_rn(mul_rn(e, c), mul_rn(o, s));
      y[t][2 * q + 1] = add_rn(mul_rn(o, c), mul_rn(e, s));
    }
  }
}

// OCP e4m3 (the fp8 KV caches): round to nearest even, saturated to the largest finite
// value +-448 (the conversion the reference's writers use). Byte j of the result holds
// v[j].
__device__ __forceinline__ uint32_t pack_e4m3x4(float v0, float v1, float v2, float v3) {
  auto sat = [](float v) { return v > 448.f ? 448.f : (v < -448.f ? -448.f : v); };  // NaN stays NaN
  int w = __builtin_amdgcn_cvt_pk_fp8_f32(sat(v0), sat(v1), 0, false);
  w = __builtin_amdgcn_cvt_pk_fp8_f32(sat(v2), sat(v3), w, true);
  return (uint32_t)w;
}

template <int D>
__device__ __forceinline__ void norm_rope_row(u32x4_t (&x)[D / 32], const float *__restrict__ w,
                                              float eps, const Rope &rope, int64_t rope_row,
                                              int g) {
  PrologueOps<D> ops;
  load_prologue_ops<D>(ops, w, rope, rope_row, g);
  norm_rope_apply<D>(x, ops, eps);
}

}  // namespace fm
