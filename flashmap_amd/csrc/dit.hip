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

// The several-jump draft's state over the vocabulary (flashmap/vllm/model.py:944-956,
// 1031-1036): softmaxes over rows of up to ~10^5 fp32 values, one workgroup per row.
// The row is read twice: once for its statistics (max and sum of exponentials, online
// per thread, merged over the workgroup), once for the outputs (each thread re-reads the
// 16-byte chunks it read the first time; a row is small enough to be served from the
// cache the second time). Exponentials are expf; the division and the update use torch's
// rounding points.
constexpr int STATE_THREADS = 256;

struct RowStats {
  float m, s;  // max and sum of exp(x - m)
};

__device__ __forceinline__ RowStats merge_stats(RowStats a, RowStats b) {
  const float m = fmaxf(a.m, b.m);
  if (m == -INFINITY) return RowStats{m, 0.f};
  const float sa = a.m == -INFINITY ? 0.f : __fmul_rn(a.s, expf(__fsub_rn(a.m, m)));
  const float sb = b.m == -INFINITY ? 0.f : __fmul_rn(b.s, expf(__fsub_rn(b.m, m)));
  return RowStats{m, __fadd_rn(sa, sb)};
}

__device__ __forceinline__ void add_chunk(RowStats &st, const float (&x)[4]) {
  const float mx = fmaxf(fmaxf(x[0], x[1]), fmaxf(x[2], x[3]));
  if (mx == -INFINITY) return;  // nothing to add (and no exp(-inf - -inf))
  if (mx > st.m) {
    st.s = st.m == -INFINITY ? 0.f : __fmul_rn(st.s, expf(__fsub_rn(st.m, mx)));
    st.m = mx;
  }
#pragma unroll
  for (int q = 0; q < 4; ++q) st.s = __fadd_rn(st.s, expf(__fsub_rn(x[q], st.m)));
}

// The workgroup's statistics from each thread's.
__device__ __forceinline__ RowStats block_stats(RowStats st) {
  __shared__ RowStats part[STATE_THREADS / 64];
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) {
    const RowStats other{__shfl_xor(st.m, o, 64), __shfl_xor(st.s, o, 64)};
    st = merge_stats(st, other);
  }
  if ((threadIdx.x & 63) == 0) part[wave_id()] = st;
  __syncthreads();
  RowStats r = part[0];
#pragma unroll
  for (int w = 1; w < STATE_THREADS / 64; ++w) r = merge_stats(r, part[w]);
  return r;
}

// POST: rows r < rows of out get bf16(softmax(evidence * state[r])) and rows rows + r
// bf16(state[r]); otherwise out holds the state rows only (one read of the row).
template <bool POST>
__global__ __launch_bounds__(STATE_THREADS) void state_embed_rows_kernel(const float *__restrict__ state,
                                                                         int64_t vocab, int64_t ss, float evidence,
                                                                         uint16_t *__restrict__ out, int64_t os,
                                                                         int64_t rows) {
  const int64_t row = blockIdx.x;
  const float *x = state + row * ss;
  const int64_t chunks = vocab >> 2;
  if constexpr (!POST) {
    uint16_t *raw = out + row * os;
#pragma unroll 4
    for (int64_t c = threadIdx.x; c < chunks; c += STATE_THREADS) {
      const f32x4_t v = *reinterpret_cast<const f32x4_t *>(x + 4 * c);
      *reinterpret_cast<u32x2_t *>(raw + 4 * c) = u32x2_t{pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3])};
    }
    for (int64_t i = 4 * chunks + threadIdx.x; i < vocab; i += STATE_THREADS)
      raw[i] = (uint16_t)(pack_bf16x2(x[i], 0.f) & 0xffffu);
    return;
  }
  RowStats st{-INFINITY, 0.f};
#pragma unroll 4
  for (int64_t c = threadIdx.x; c < chunks; c += STATE_THREADS) {
    const f32x4_t v = *reinterpret_cast<const f32x4_t *>(x + 4 * c);
    const float e[4] = {__fmul_rn(v[0], evidence), __fmul_rn(v[1], evidence), __fmul_rn(v[2], evidence),
                        __fmul_rn(v[3], evidence)};
    add_chunk(st, e);
  }
  for (int64_t i = 4 * chunks + threadIdx.x; i < vocab; i += STATE_THREADS) {  // the tail (vocab % 4)
    const float e[4] = {__fmul_rn(x[i], evidence), -INFINITY, -INFINITY, -INFINITY};
    add_chunk(st, e);
  }
  const RowStats t = block_stats(st);
  uint16_t *post = out + row * os, *raw = out + (rows + row) * os;
#pragma unroll 4
  for (int64_t c = threadIdx.x; c < chunks; c += STATE_THREADS) {
    const f32x4_t v = *reinterpret_cast<const f32x4_t *>(x + 4 * c);
    float p[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) p[q] = __fdiv_rn(expf(__fsub_rn(__fmul_rn(v[q], evidence), t.m)), t.s);
    *reinterpret_cast<u32x2_t *>(post + 4 * c) = u32x2_t{pack_bf16x2(p[0], p[1]), pack_bf16x2(p[2], p[3])};
    *reinterpret_cast<u32x2_t *>(raw + 4 * c) = u32x2_t{pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3])};
  }
  for (int64_t i = 4 * chunks + threadIdx.x; i < vocab; i += STATE_THREADS) {
    const float p = __fdiv_rn(expf(__fsub_rn(__fmul_rn(x[i], evidence), t.m)), t.s);
    post[i] = (uint16_t)(pack_bf16x2(p, 0.f) & 0xffffu);
    raw[i] = (uint16_t)(pack_bf16x2(x[i], 0.f) & 0xffffu);
  }
}

// state[r] = (c_keep * state[r] + c_new * softmax(logits[r])) / c_div in place, logits bf16.
__global__ __launch_bounds__(STATE_THREADS) void state_update_kernel(float *__restrict__ state, int64_t vocab,
                                                                     int64_t ss, const uint16_t *__restrict__ logits,
                                                                     int64_t ls, float c_keep, float c_new,
                                                                     float c_div) {
  const int64_t row = blockIdx.x;
  float *x = state + row * ss;
  const uint16_t *lg = logits + row * ls;
  const int64_t chunks = vocab >> 2;
  RowStats st{-INFINITY, 0.f};
#pragma unroll 4
  for (int64_t c = threadIdx.x; c < chunks; c += STATE_THREADS) {
    const u32x2_t w = *reinterpret_cast<const u32x2_t *>(lg + 4 * c);
    const float e[4] = {bf16_lo(w[0]), bf16_hi(w[0]), bf16_lo(w[1]), bf16_hi(w[1])};
    add_chunk(st, e);
  }
  for (int64_t i = 4 * chunks + threadIdx.x; i < vocab; i += STATE_THREADS) {
    const float e[4] = {__uint_as_float((uint32_t)lg[i] << 16), -INFINITY, -INFINITY, -INFINITY};
    add_chunk(st, e);
  }
  const RowStats t = block_stats(st);
  auto upd = [&](float s, float l) {
    const float d = __fdiv_rn(expf(__fsub_rn(l, t.m)), t.s);
    return __fdiv_rn(__fadd_rn(__fmul_rn(c_keep, s), __fmul_rn(c_new, d)), c_div);
  };
#pragma unroll 4
  for (int64_t c = threadIdx.x; c < chunks; c += STATE_THREADS) {
    const u32x2_t w = *reinterpret_cast<const u32x2_t *>(lg + 4 * c);
    f32x4_t v = *reinterpret_cast<const f32x4_t *>(x + 4 * c);
    v[0] = upd(v[0], bf16_lo(w[0]));
    v[1] = upd(v[1], bf16_hi(w[0]));
    v[2] = upd(v[2], bf16_lo(w[1]));
    v[3] = upd(v[3], bf16_hi(w[1]));
    *reinterpret_cast<f32x4_t *>(x + 4 * c) = v;
  }
  for (int64_t i = 4 * chunks + threadIdx.x; i < vocab; i += STATE_THREADS)
    x[i] = upd(x[i], __uint_as_float((uint32_t)lg[i] << 16));
}

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

extern "C" int fm_state_embed_rows(const float *state, int64_t rows, int64_t vocab, int64_t state_stride,
                                   float evidence, int32_t posterior, void *out, int64_t out_stride, void *stream) {
  using namespace fm;
  FM_REQUIRE(rows >= 0 && vocab > 0, "bad sizes: rows=%lld vocab=%lld", (long long)rows, (long long)vocab);
  if (rows == 0) return FM_OK;
  FM_REQUIRE(state && out, "NULL tensor pointer");
  FM_REQUIRE(rows < (1ll << 31), "too many rows");
  FM_REQUIRE(aligned16(state) && state_stride % 4 == 0 && state_stride >= vocab,
             "state must be 16-byte aligned with a row stride that is a multiple of 4 covering a row");
  FM_REQUIRE(((uintptr_t)out & 7) == 0 && out_stride % 4 == 0 && out_stride >= vocab,
             "out must be 8-byte aligned with a row stride that is a multiple of 4 covering a row");
  const dim3 grid((unsigned)rows), block(STATE_THREADS);
  if (posterior)
    state_embed_rows_kernel<true><<<grid, block, 0, (hipStream_t)stream>>>(state, vocab, state_stride, evidence,
                                                                           (uint16_t *)out, out_stride, rows);
  else
    state_embed_rows_kernel<false><<<grid, block, 0, (hipStream_t)stream>>>(state, vocab, state_stride, evidence,
                                                                            (uint16_t *)out, out_stride, rows);
  FM_CHECK_HIP(hipGetLastError());
  return FM_OK;
}

extern "C" int fm_state_update(float *state, int64_t rows, int64_t vocab, int64_t state_stride, const void *logits,
                               int64_t logits_stride, double start, double end, void *stream) {
  using namespace fm;
  FM_REQUIRE(rows >= 0 && vocab > 0, "bad sizes: rows=%lld vocab=%lld", (long long)rows, (long long)vocab);
  if (rows == 0) return FM_OK;
  FM_REQUIRE(state && logits, "NULL tensor pointer");
  FM_REQUIRE(rows < (1ll << 31), "too many rows");
  FM_REQUIRE(start < 1.0 && end >= start, "jump times must satisfy start <= end, start < 1 (got %g, %g)", start, end);
  FM_REQUIRE(aligned16(state) && state_stride % 4 == 0 && state_stride >= vocab,
             "state must be 16-byte aligned with a row stride that is a multiple of 4 covering a row");
  FM_REQUIRE(((uintptr_t)logits & 7) == 0 && logits_stride % 4 == 0 && logits_stride >= vocab,
             "logits must be 8-byte aligned with a row stride that is a multiple of 4 covering a row");
  // The scalars as torch takes Python floats into a float32 op: computed in double, then
  // rounded to float.
  const float c_keep = (float)(1.0 - end), c_new = (float)(end - start), c_div = (float)(1.0 - start);
  state_update_kernel<<<dim3((unsigned)rows), dim3(STATE_THREADS), 0, (hipStream_t)stream>>>(
      state, vocab, state_stride, (const uint16_t *)logits, logits_stride, c_keep, c_new, c_div);
  FM_CHECK_HIP(hipGetLastError());
  return FM_OK;
}
