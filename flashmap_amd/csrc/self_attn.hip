// a8: self-attention within each draft block, with the q/k RMSNorms and RoPE fused.
// One wavefront per (block, head): the block's T <= 16 slots are the 16 rows of the
// row-quad layout (fm_device.h), so q and k are normed and rotated by the same code
// as the cross-attention prologue, then
//   S^T = K Q^T                 v_mfma_f32_16x16x32_bf16 (4 k-steps at head_dim 128)
//   P   = exp(S * scale - max)  per query column (lane), summed into the denominator
//   O^T = V^T P^T               v_mfma_f32_16x16x16bf16_1k, V^T read from LDS
//   out = O / denom             rounded to bf16 once
// Follows flashmap/vllm/kernels.py:127-191 and flashmap/sglang/kernels.py:18-75
// (P rounded to bf16 before P.V, fp32 denominator).
#include <math.h>

#include "fm_device.h"
#include "fm_host.h"

namespace fm {

template <int D>
__global__ __launch_bounds__(256) void block_self_attn_kernel(
    const uint16_t *__restrict__ qkv, uint16_t *__restrict__ out, int64_t pairs, int32_t T,
    int32_t H, const float *__restrict__ qn_w, const float *__restrict__ kn_w, Rope rope,
    const int64_t *__restrict__ positions, float eps, float scale) {
  constexpr int KT = D / 32, DB = D / 16, VP = D + 4;
  __shared__ __attribute__((aligned(16))) uint16_t vstage[4][16 * VP];
  const int lane = threadIdx.x & 63, wave = wave_id();
  const int n = lane & 15, g = lane >> 4;
  const int64_t pair = (int64_t)blockIdx.x * 4 + wave;
  if (pair >= pairs) return;  // wave-uniform; no block-wide barrier follows
  const int64_t blk = pair / H;
  const int h = (int)(pair - blk * H);
  const bool valid = n < T;
  const int64_t tok = blk * T + (valid ? n : 0);
  const int64_t row_stride = 3ll * H * D;
  const uint16_t *qrow = qkv + tok * row_stride + (int64_t)h * D + 8 * g;
  u32x4_t qf[KT], kf[KT], vv[KT];
#pragma unroll
  for (int t = 0; t < KT; ++t) {
    qf[t] = valid ? load16(qrow + 32 * t) : u32x4_t{0, 0, 0, 0};
    kf[t] = valid ? load16(qrow + (int64_t)H * D + 32 * t) : u32x4_t{0, 0, 0, 0};
    vv[t] = valid ? load16(qrow + 2ll * H * D + 32 * t) : u32x4_t{0, 0, 0, 0};
  }
  const int64_t rr = clamp_row(rope, valid ? (positions ? positions[tok] : tok) : 0);
  norm_rope_row<D>(qf, qn_w, eps, rope, rr, g);
  norm_rope_row<D>(kf, kn_w, eps, rope, rr, g);

  uint16_t *vs = vstage[wave];
#pragma unroll
  for (int t = 0; t < KT; ++t) {
    uint16_t *dst = vs + n * VP + 32 * t + 8 * g;
    *reinterpret_cast<u32x2_t *>(dst) = u32x2_t{vv[t][0], vv[t][1]};
    *reinterpret_cast<u32x2_t *>(dst + 4) = u32x2_t{vv[t][2], vv[t][3]};
  }

  f32x4_t s = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int t = 0; t < KT; ++t) s = mfma_16x16x32(kf[t], qf[t], s);  // S^T[key 4g+i][query n]
  float p[4];
  float mx = -INFINITY;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    p[i] = (4 * g + i < T) ? s[i] * scale : -INFINITY;
    mx = fmaxf(mx, p[i]);
  }
  mx = max_over_groups(mx);
  float den = 0.f;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    p[i] = __expf(p[i] - mx);
    den += p[i];
  }
  den = sum_over_groups(den);
  const u32x2_t pk = u32x2_t{pack_bf16x2(p[0], p[1]), pack_bf16x2(p[2], p[3])};

  __builtin_amdgcn_wave_barrier();
  const uint16_t *vcol = vs + 4 * g * VP + n;
  const float inv = 1.f / den;
  uint16_t *dst = out + ((blk * T + n) * H + h) * (int64_t)D + 4 * g;
#pragma unroll
  for (int db = 0; db < DB; ++db) {
    const uint16_t *c0 = vcol + 16 * db;
    const u32x2_t vf = u32x2_t{(uint32_t)c0[0] | ((uint32_t)c0[VP] << 16),
                               (uint32_t)c0[2 * VP] | ((uint32_t)c0[3 * VP] << 16)};
    f32x4_t o = {0.f, 0.f, 0.f, 0.f};
    o = mfma_16x16x16(vf, pk, o);  // O^T[d = 16 db + 4 g + i][query n]
    if (valid) {
      o *= inv;
      *reinterpret_cast<u32x2_t *>(dst + 16 * db) = u32x2_t{pack_bf16x2(o[0], o[1]), pack_bf16x2(o[2], o[3])};
    }
  }
}

}  // namespace fm

extern "C" int fm_block_self_attention(const void *qkv, void *out, int64_t blocks,
                                       int32_t block_size, int32_t heads, int32_t head_dim,
                                       const float *q_norm_weight, const float *k_norm_weight,
                                       const float *rope_cos, const float *rope_sin,
                                       int64_t rope_row_stride, int64_t rope_pair_stride,
                                       int64_t rope_rows, const int64_t *positions, float eps,
                                       float softmax_scale, void *stream) {
  using namespace fm;
  FM_REQUIRE(blocks >= 0 && heads > 0 && block_size > 0, "bad sizes");
  if (blocks == 0) return FM_OK;
  if (block_size > 16)
    return fail(FM_ERR_UNSUPPORTED, "block_size %d not supported (at most 16)", block_size);
  if (head_dim != 64 && head_dim != 128)
    return fail(FM_ERR_UNSUPPORTED, "head_dim %d not supported (64 or 128)", head_dim);
  FM_REQUIRE(qkv && out && q_norm_weight && k_norm_weight && rope_cos && rope_sin, "NULL pointer");
  FM_REQUIRE((((uintptr_t)qkv | (uintptr_t)out) & 15) == 0, "qkv/out must be 16-byte aligned");
  const int64_t pairs = blocks * heads;
  const int64_t grid = (pairs + 3) / 4;
  FM_REQUIRE(grid < (1ll << 31), "too many blocks");
  Rope rope{rope_cos, rope_sin, rope_row_stride, rope_pair_stride, rope_rows};
  hipStream_t s = (hipStream_t)stream;
  if (head_dim == 128)
    block_self_attn_kernel<128><<<dim3((unsigned)grid), dim3(256), 0, s>>>(
        (const uint16_t *)qkv, (uint16_t *)out, pairs, block_size, heads, q_norm_weight,
        k_norm_weight, rope, positions, eps, softmax_scale);
  else
    block_self_attn_kernel<64><<<dim3((unsigned)grid), dim3(256), 0, s>>>(
        (const uint16_t *)qkv, (uint16_t *)out, pairs, block_size, heads, q_norm_weight,
        k_norm_weight, rope, positions, eps, softmax_scale);
  FM_CHECK_HIP(hipGetLastError());
  return FM_OK;
}
