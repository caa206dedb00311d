// The DiT's residual stream between its sublayers (flashmap/modeling_flashmap.py:102-117,
// 185-192): after a sublayer's output y, the gated residual x' = x + gate * y, then the
// next sublayer's time-modulated LayerNorm h = LN(x') * (1 + scale) + shift. The
// reference runs these as about eight eager bf16 ops per sublayer; here one pass per row
// reads x and y once and writes x' and h.
//
// Rounding points are torch's eager bf16 ones: gate * y, x + (gate * y), LN(x'),
// 1 + scale, LN * (1 + scale) and + shift each round to bf16 (each computed in fp32 from
// bf16 operands, products and sums kept apart so nothing contracts into an FMA). LN is
// without affine weights, (x' - mean) * rsqrt(var + eps) with the biased variance, its
// statistics reduced in fp32 over the row (two passes over the row held in registers).
// The statistics' summation order is the only difference from torch's kernel, so x' is
// bit-exact and h agrees up to an occasional one-ulp flip of the LN rounding.
//
// Layout: rows of `dim` bf16 values with a row stride, one wavefront per row; lane l
// holds the 16-byte chunks l, l + 64, ... of its row (coalesced 1 KiB per wavefront
// load). gate, scale and shift are (dim,) vectors shared by every row: the modulations
// depend on the jump's times only. Two variants serve the folded noise read-out of a
// one-jump draft (flashmap/vllm/model.py:915-925): the gate one bf16 scalar per row, and
// x one (dim,) row shared by all rows (row stride 0).
//
// fm_noise_rows, that read-out's row pass: per row of the fp32 noise z (H values) the
// scale bf16(gain * rsqrt(sum_i z_i^2 lambda_i + eps)) and z rounded to bf16 for the
// folded GEMM; one wavefront per row, 16-byte loads.
#include "fm_device.h"
#include "fm_host.h"

namespace fm {

struct AdalnArgs {
  const uint16_t *x;
  const uint16_t *y;  // NULL: no residual, x' = x
  const uint16_t *gate, *scale, *shift;  // scale NULL: no norm
  int32_t gate_rows;  // nonzero: gate holds one value per row
  uint16_t *x_out;  // NULL: x' not stored
  uint16_t *h_out;
  int64_t rows;
  int64_t xs, ys, xos, hs;  // row strides (elements)
  int32_t dim;
  float eps;
};

__device__ __forceinline__ float wave_sum64(float v) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) v = __fadd_rn(v, __shfl_xor(v, m, 64));
  return v;
}

template <int NCH>
__global__ __launch_bounds__(256) void adaln_residual_kernel(const AdalnArgs a) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * 4 + wave_id();
  if (row >= a.rows) return;  // wave-uniform
  const int chunks = a.dim >> 3;
  u32x4_t r[NCH];
  float sum = 0.f;
#pragma unroll
  for (int i = 0; i < NCH; ++i) {
    const int c = lane + 64 * i;
    if (c < chunks) {
      const u32x4_t xv = load16(a.x + row * a.xs + 8 * c);
      if (a.y != nullptr) {
        const u32x4_t yv = load16(a.y + row * a.ys + 8 * c);
        u32x4_t gv;
        if (a.gate_rows) {
          const uint32_t gr = a.gate[row];
          const uint32_t g2 = gr | (gr << 16);
          gv = u32x4_t{g2, g2, g2, g2};
        } else {
          gv = load16(a.gate + 8 * c);
        }
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const float lo = __fadd_rn(bf16_lo(xv[q]), round_bf16(__fmul_rn(bf16_lo(gv[q]), bf16_lo(yv[q]))));
          const float hi = __fadd_rn(bf16_hi(xv[q]), round_bf16(__fmul_rn(bf16_hi(gv[q]), bf16_hi(yv[q]))));
          r[i][q] = pack_bf16x2(lo, hi);
        }
      } else {
        r[i] = xv;
      }
#pragma unroll
      for (int q = 0; q < 4; ++q) sum = __fadd_rn(sum, __fadd_rn(bf16_lo(r[i][q]), bf16_hi(r[i][q])));
      if (a.x_out != nullptr) store16(a.x_out + row * a.xos + 8 * c, r[i]);
    }
  }
  if (a.scale == nullptr) return;
  const float n = (float)a.dim;
  const float mean = __fdiv_rn(wave_sum64(sum), n);
  float sq = 0.f;
#pragma unroll
  for (int i = 0; i < NCH; ++i) {
    if (lane + 64 * i < chunks) {
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const float dl = __fsub_rn(bf16_lo(r[i][q]), mean), dh = __fsub_rn(bf16_hi(r[i][q]), mean);
        sq = __fadd_rn(sq, __fadd_rn(__fmul_rn(dl, dl), __fmul_rn(dh, dh)));
      }
    }
  }
  const float rstd = rsqrtf(__fadd_rn(__fdiv_rn(wave_sum64(sq), n), a.eps));
#pragma unroll
  for (int i = 0; i < NCH; ++i) {
    const int c = lane + 64 * i;
    if (c < chunks) {
      const u32x4_t sv = load16(a.scale + 8 * c);
      const u32x4_t tv = load16(a.shift + 8 * c);
      u32x4_t h;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        float v[2] = {bf16_lo(r[i][q]), bf16_hi(r[i][q])};
        const float s[2] = {bf16_lo(sv[q]), bf16_hi(sv[q])};
        const float t[2] = {bf16_lo(tv[q]), bf16_hi(tv[q])};
#pragma unroll
        for (int j = 0; j < 2; ++j) {
          const float ln = round_bf16(__fmul_rn(rstd, __fsub_rn(v[j], mean)));
          const float mod = round_bf16(__fmul_rn(ln, round_bf16(__fadd_rn(1.0f, s[j]))));
          v[j] = __fadd_rn(mod, t[j]);
        }
        h[q] = pack_bf16x2(v[0], v[1]);
      }
      store16(a.h_out + row * a.hs + 8 * c, h);
    }
  }
}

// One wavefront per row of z (fp32, H values): lane l holds the 4-value chunks l, l + 64, ...
template <int NCH>
__global__ __launch_bounds__(256) void noise_rows_kernel(const float *__restrict__ z, int64_t rows, int32_t h,
                                                         int64_t zs, const float *__restrict__ lam, float eps,
                                                         float gain, uint16_t *__restrict__ z16, int64_t z16s,
                                                         uint16_t *__restrict__ scale) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * 4 + wave_id();
  if (row >= rows) return;  // wave-uniform
  const int chunks = h >> 2;
  float acc = 0.f;
#pragma unroll
  for (int i = 0; i < NCH; ++i) {
    const int c = lane + 64 * i;
    if (c < chunks) {
      const f32x4_t v = *reinterpret_cast<const f32x4_t *>(z + row * zs + 4 * c);
      const f32x4_t l = *reinterpret_cast<const f32x4_t *>(lam + 4 * c);
#pragma unroll
      for (int q = 0; q < 4; ++q) acc = __builtin_fmaf(__fmul_rn(v[q], v[q]), l[q], acc);
      *reinterpret_cast<u32x2_t *>(z16 + row * z16s + 4 * c) = u32x2_t{pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3])};
    }
  }
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) acc = __fadd_rn(acc, __shfl_xor(acc, m, 64));
  if (lane == 0) {
    const float s = __fmul_rn(gain, rsqrtf(__fadd_rn(acc, eps)));
    scale[row] = (uint16_t)(pack_bf16x2(s, 0.f) & 0xffffu);
  }
}

static bool aligned16(const void *p) { return ((uintptr_t)p & 15) == 0; }

}  // namespace fm

extern "C" int fm_adaln_residual(const void *x, int64_t x_stride, const void *y, int64_t y_stride,
                                 const void *gate, int32_t gate_per_row, const void *scale, const void *shift,
                                 void *x_out, int64_t x_out_stride, void *h_out, int64_t h_out_stride,
                                 int64_t rows, int32_t dim, float eps, void *stream) {
  using namespace fm;
  FM_REQUIRE(rows >= 0 && dim > 0, "bad sizes: rows=%lld dim=%d", (long long)rows, dim);
  if (rows == 0) return FM_OK;
  if (dim % 8 != 0 || dim > 8192)
    return fail(FM_ERR_UNSUPPORTED, "dim %d not supported (a multiple of 8, at most 8192)", dim);
  FM_REQUIRE(x != nullptr, "NULL x");
  FM_REQUIRE(y == nullptr || gate != nullptr, "a residual needs its gate");
  FM_REQUIRE(scale == nullptr || (shift != nullptr && h_out != nullptr), "a norm needs shift and h_out");
  FM_REQUIRE(scale != nullptr || x_out != nullptr, "nothing to write: neither x_out nor a norm");
  const void *ptrs[7] = {x, y, gate, scale, shift, x_out, h_out};
  for (const void *p : ptrs) FM_REQUIRE(p == nullptr || aligned16(p), "tensors must be 16-byte aligned");
  FM_REQUIRE(x_stride % 8 == 0 && y_stride % 8 == 0 && x_out_stride % 8 == 0 && h_out_stride % 8 == 0,
             "row strides must be multiples of 8 elements");
  FM_REQUIRE((x_stride == 0 || x_stride >= dim) && (y == nullptr || y_stride >= dim) &&
                 (x_out == nullptr || x_out_stride >= dim) && (h_out == nullptr || h_out_stride >= dim),
             "row strides must cover a row of %d (x may also be one shared row, stride 0)", dim);
  FM_REQUIRE(x_stride != 0 || x_out != x, "a shared x row cannot be written in place");
  const int64_t blocks = (rows + 3) / 4;
  FM_REQUIRE(blocks < (1ll << 31), "too many rows");
  AdalnArgs a{(const uint16_t *)x,     (const uint16_t *)y,     (const uint16_t *)gate,
              (const uint16_t *)scale, (const uint16_t *)shift, gate_per_row,
              (uint16_t *)x_out,       (uint16_t *)h_out,       rows,
              x_stride,                y_stride,                x_out_stride,
              h_out_stride,            dim,                     eps};
  hipStream_t s = (hipStream_t)stream;
  const int per_lane = (dim / 8 + 63) / 64;
  const dim3 grid((unsigned)blocks), block(256);
  if (per_lane <= 1)
    adaln_residual_kernel<1><<<grid, block, 0, s>>>(a);
  else if (per_lane <= 2)
    adaln_residual_kernel<2><<<grid, block, 0, s>>>(a);
  else if (per_lane <= 4)
    adaln_residual_kernel<4><<<grid, block, 0, s>>>(a);
  else if (per_lane <= 8)
    adaln_residual_kernel<8><<<grid, block, 0, s>>>(a);
  else
    adaln_residual_kernel<16><<<grid, block, 0, s>>>(a);
  FM_CHECK_HIP(hipGetLastError());
  return FM_OK;
}

extern "C" int fm_noise_rows(const float *z, int64_t rows, int32_t hidden, int64_t z_stride, const float *eigvals,
                             float eps, float gain, void *z_bf16, int64_t z_bf16_stride, void *scale,
                             void *stream) {
  using namespace fm;
  FM_REQUIRE(rows >= 0 && hidden > 0, "bad sizes: rows=%lld hidden=%d", (long long)rows, hidden);
  if (rows == 0) return FM_OK;
  if (hidden % 4 != 0 || hidden > 16384)
    return fail(FM_ERR_UNSUPPORTED, "hidden %d not supported (a multiple of 4, at most 16384)", hidden);
  FM_REQUIRE(z && eigvals && z_bf16 && scale, "NULL tensor pointer");
  FM_REQUIRE(aligned16(z) && aligned16(eigvals) && ((uintptr_t)z_bf16 & 7) == 0,
             "z / eigvals must be 16-byte aligned, z_bf16 8-byte aligned");
  FM_REQUIRE(z_stride % 4 == 0 && z_stride >= hidden && z_bf16_stride % 4 == 0 && z_bf16_stride >= hidden,
             "row strides must be multiples of 4 covering a row");
  const int64_t blocks = (rows + 3) / 4;
  FM_REQUIRE(blocks < (1ll << 31), "too many rows");
  hipStream_t s = (hipStream_t)stream;
  const int per_lane = (hidden / 4 + 63) / 64;
  const dim3 grid((unsigned)blocks), block(256);
  uint16_t *zo = (uint16_t *)z_bf16, *so = (uint16_t *)scale;
  if (per_lane <= 8)
    noise_rows_kernel<8><<<grid, block, 0, s>>>(z, rows, hidden, z_stride, eigvals, eps, gain, zo, z_bf16_stride, so);
  else if (per_lane <= 16)
    noise_rows_kernel<16><<<grid, block, 0, s>>>(z, rows, hidden, z_stride, eigvals, eps, gain, zo, z_bf16_stride, so);
  else
    noise_rows_kernel<64><<<grid, block, 0, s>>>(z, rows, hidden, z_stride, eigvals, eps, gain, zo, z_bf16_stride, so);
  FM_CHECK_HIP(hipGetLastError());
  return FM_OK;
}
