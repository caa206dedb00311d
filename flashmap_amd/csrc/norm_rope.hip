// a2/a3: the Q prologue as its own launch, QK-RMSNorm + interleaved RoPE of every
// (token, head) row. One wavefront transforms 16 rows held in the row-quad layout
// (fm_device.h), the same code path the fused attention prologue runs, so the
// standalone and fused prologues produce bit-identical bf16 values.
#include "fm_device.h"
#include "fm_host.h"

namespace fm {

template <int D>
__global__ __launch_bounds__(256) void rms_norm_rope_kernel(
    const uint16_t *__restrict__ x, uint16_t *__restrict__ out, int64_t rows, int32_t heads,
    int64_t xs_t, int64_t xs_h, int64_t os_t, int64_t os_h, const float *__restrict__ w,
    Rope rope, const int64_t *__restrict__ positions, float eps) {
  constexpr int KT = D / 32;
  const int lane = threadIdx.x & 63, wave = wave_id();
  const int n = lane & 15, g = lane >> 4;
  const int64_t row = ((int64_t)blockIdx.x * 4 + wave) * 16 + n;
  const bool valid = row < rows;
  const int64_t token = valid ? row / heads : 0;
  const int64_t head = valid ? row % heads : 0;
  u32x4_t v[KT];
  const uint16_t *src = x + token * xs_t + head * xs_h + 8 * g;
#pragma unroll
  for (int t = 0; t < KT; ++t) v[t] = valid ? load16(src + 32 * t) : u32x4_t{0, 0, 0, 0};
  const int64_t rr = clamp_row(rope, valid ? (positions ? positions[token] : token) : 0);
  norm_rope_row<D>(v, w, eps, rope, rr, g);
  if (valid) {
    uint16_t *dst = out + token * os_t + head * os_h + 8 * g;
#pragma unroll
    for (int t = 0; t < KT; ++t) store16(dst + 32 * t, v[t]);
  }
}

static bool aligned16(const void *p) { return ((uintptr_t)p & 15) == 0; }

}  // namespace fm

extern "C" int fm_rms_norm_rope(const void *x, void *out, int64_t tokens, int32_t heads,
                                int32_t head_dim, int64_t x_stride_token, int64_t x_stride_head,
                                int64_t out_stride_token, int64_t out_stride_head,
                                const float *weight, const float *rope_cos, const float *rope_sin,
                                int64_t rope_row_stride, int64_t rope_pair_stride,
                                int64_t rope_rows, const int64_t *positions, float eps,
                                void *stream) {
  using namespace fm;
  FM_REQUIRE(tokens >= 0 && heads > 0, "bad sizes: tokens=%lld heads=%d", (long long)tokens, heads);
  if (tokens == 0) return FM_OK;
  if (head_dim != 64 && head_dim != 128)
    return fail(FM_ERR_UNSUPPORTED, "head_dim %d not supported (64 or 128)", head_dim);
  FM_REQUIRE(x && out && weight && rope_cos && rope_sin, "NULL tensor pointer");
  FM_REQUIRE(aligned16(x) && aligned16(out), "x/out must be 16-byte aligned");
  FM_REQUIRE(x_stride_token % 8 == 0 && x_stride_head % 8 == 0 && out_stride_token % 8 == 0 &&
                 out_stride_head % 8 == 0,
             "token/head strides must be multiples of 8 elements");
  const int64_t rows = tokens * heads;
  const int64_t blocks = (rows + 63) / 64;
  FM_REQUIRE(blocks < (1ll << 31), "too many rows");
  Rope rope{rope_cos, rope_sin, rope_row_stride, rope_pair_stride, rope_rows};
  hipStream_t s = (hipStream_t)stream;
  const uint16_t *xp = (const uint16_t *)x;
  uint16_t *op = (uint16_t *)out;
  if (head_dim == 128)
    rms_norm_rope_kernel<128><<<dim3((unsigned)blocks), dim3(256), 0, s>>>(
        xp, op, rows, heads, x_stride_token, x_stride_head, out_stride_token, out_stride_head,
        weight, rope, positions, eps);
  else
    rms_norm_rope_kernel<64><<<dim3((unsigned)blocks), dim3(256), 0, s>>>(
        xp, op, rows, heads, x_stride_token, x_stride_head, out_stride_token, out_stride_head,
        weight, rope, positions, eps);
  FM_CHECK_HIP(hipGetLastError());
  return FM_OK;
}
