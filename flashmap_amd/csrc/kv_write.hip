// a4: the K side of the QK-norm prologue. Every committed context row's keys are
// k-normed and rotated at the row's context position and stored, with its values,
// into the engine's KV layout. One wavefront transforms 16 (token, global head) rows
// in the row-quad layout (fm_device.h), with the same arithmetic as the Q prologue.
//   vLLM:   kv (tokens, layers, 2, heads, D) -> paged caches (blocks, heads, page, 2D)
//           (flashmap/vllm/kernels.py:235-364)
//   SGLang: the same kv rows -> per-layer (pool, heads, D) key/value buffers
//           (sglang's fused_kv_norm_rope_write as flashmap/sglang/model.py:746-766
//           calls it; flashmap/sglang/kernels.py:283-357 is its fp8 twin)
// FP8: e4m3 caches (one byte per element): keys rotated in fp32, both keys and values
// divided by the cache's scale, rounded to nearest even and saturated to +-448 --
// vLLM's per-layer scales (flashmap/vllm/kernels.py:292-299), or the pool writer's
// static scales with its own norm rounding (flashmap/sglang/kernels.py:283-357).
#include "fm_device.h"
#include "fm_host.h"

namespace fm {

struct KvWriteArgs {
  const uint16_t *kv;
  int64_t rows;  // tokens * layers * heads
  int32_t layers, heads;
  const int64_t *positions;
  const float *k_norm;  // (layers, D)
  Rope rope;
  float eps;
  // vLLM destination
  const int64_t *slots;
  const int64_t *cache_ptrs;
  int32_t num_caches, heads_per_cache, page_size;
  int64_t s_block, s_head, s_token, v_offset;
  // SGLang destination
  const int64_t *meta;  // (layers, 4)
  const int64_t *locs;
  const int32_t *commit_lens;
  int64_t row_width;
  // FP8 destinations: per-layer (key, value) scales (vLLM, layers x 2) or one pair.
  const float *scales;
  float k_scale, v_scale;
};

template <int D, bool POOL, bool FP8>
__global__ __launch_bounds__(256) void kv_write_kernel(const KvWriteArgs a) {
  constexpr int KT = D / 32;
  const int lane = threadIdx.x & 63, wave = wave_id();
  const int n = lane & 15, g = lane >> 4;
  const int64_t row = ((int64_t)blockIdx.x * 4 + wave) * 16 + n;
  const int64_t lh = (int64_t)a.layers * a.heads;
  bool live = row < a.rows;
  const int64_t token = live ? row / lh : 0;
  const int gh = live ? (int)(row - token * lh) : 0;
  const int layer = gh / a.heads, h = gh - layer * a.heads;
  int64_t slot = 0;
  if (live) {
    if (POOL) {
      slot = a.locs[token];
      if (a.commit_lens != nullptr) {
        const int64_t rb = token / a.row_width;
        if (token - rb * a.row_width >= (int64_t)a.commit_lens[rb]) live = false;
      }
    } else {
      slot = a.slots[token];
    }
    if (slot < 0) live = false;
  }
  const uint16_t *krow = a.kv + ((token * a.layers + layer) * 2ll * a.heads + h) * D + 8 * g;
  const uint16_t *vrow = krow + (int64_t)a.heads * D;
  u32x4_t kf[KT], vf[KT];
#pragma unroll
  for (int t = 0; t < KT; ++t) {
    kf[t] = live ? load16(krow + 32 * t) : u32x4_t{0, 0, 0, 0};
    vf[t] = live ? load16(vrow + 32 * t) : u32x4_t{0, 0, 0, 0};
  }
  const int64_t rr = clamp_row(a.rope, live ? a.positions[token] : 0);
  if constexpr (FP8) {
    PrologueOps<D> ops;
    load_prologue_ops<D>(ops, a.k_norm + (int64_t)layer * D, a.rope, rr, g);
    float ky[KT][8];
    norm_rope_f32<D, POOL>(kf, ops, a.eps, ky);  // every lane: the norm crosses lanes
    if (!live) return;
    const float ks = POOL ? a.k_scale : a.scales[2 * layer], vs = POOL ? a.v_scale : a.scales[2 * layer + 1];
    uint8_t *kdst, *vdst;
    if (POOL) {
      const int64_t *m = a.meta + 4ll * layer;
      kdst = reinterpret_cast<uint8_t *>(m[0]) + slot * m[2] + (int64_t)h * D;
      vdst = reinterpret_cast<uint8_t *>(m[1]) + slot * m[3] + (int64_t)h * D;
    } else {
      const int cache = gh / a.heads_per_cache, cslot = gh - cache * a.heads_per_cache;
      const int64_t page = slot / a.page_size, in_page = slot - page * a.page_size;
      kdst = reinterpret_cast<uint8_t *>(a.cache_ptrs[cache]) + page * a.s_block + (int64_t)cslot * a.s_head +
             in_page * a.s_token;
      vdst = kdst + a.v_offset;
    }
    typedef __attribute__((address_space(1))) u32x2_t gu32x2_t;
#pragma unroll
    for (int t = 0; t < KT; ++t) {
      float kq[8], vq[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) kq[j] = __fdiv_rn(ky[t][j], ks);
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        vq[2 * q] = __fdiv_rn(bf16_lo(vf[t][q]), vs);
        vq[2 * q + 1] = __fdiv_rn(bf16_hi(vf[t][q]), vs);
      }
      *(gu32x2_t *)(kdst + 32 * t + 8 * g) =
          u32x2_t{pack_e4m3x4(kq[0], kq[1], kq[2], kq[3]), pack_e4m3x4(kq[4], kq[5], kq[6], kq[7])};
      *(gu32x2_t *)(vdst + 32 * t + 8 * g) =
          u32x2_t{pack_e4m3x4(vq[0], vq[1], vq[2], vq[3]), pack_e4m3x4(vq[4], vq[5], vq[6], vq[7])};
    }
    return;
  }
  norm_rope_row<D>(kf, a.k_norm + (int64_t)layer * D, a.eps, a.rope, rr, g);
  if (!live) return;
  uint16_t *kdst;
  uint16_t *vdst;
  if (POOL) {
    const int64_t *m = a.meta + 4ll * layer;
    kdst = reinterpret_cast<uint16_t *>(m[0]) + slot * m[2] + (int64_t)h * D;
    vdst = reinterpret_cast<uint16_t *>(m[1]) + slot * m[3] + (int64_t)h * D;
  } else {
    const int cache = gh / a.heads_per_cache, cslot = gh - cache * a.heads_per_cache;
    const int64_t page = slot / a.page_size, in_page = slot - page * a.page_size;
    kdst = reinterpret_cast<uint16_t *>(a.cache_ptrs[cache]) + page * a.s_block +
           (int64_t)cslot * a.s_head + in_page * a.s_token;
    vdst = kdst + a.v_offset;
  }
#pragma unroll
  for (int t = 0; t < KT; ++t) {
    store16(kdst + 32 * t + 8 * g, kf[t]);
    store16(vdst + 32 * t + 8 * g, vf[t]);
  }
}

template <bool POOL, bool FP8 = false>
static int launch_kv_write(const KvWriteArgs &a, int head_dim, hipStream_t s) {
  const int64_t grid = (a.rows + 63) / 64;
  FM_REQUIRE(grid < (1ll << 31), "too many rows");
  if (head_dim == 128)
    kv_write_kernel<128, POOL, FP8><<<dim3((unsigned)grid), dim3(256), 0, s>>>(a);
  else
    kv_write_kernel<64, POOL, FP8><<<dim3((unsigned)grid), dim3(256), 0, s>>>(a);
  FM_CHECK_HIP(hipGetLastError());
  return FM_OK;
}

}  // namespace fm

using namespace fm;

extern "C" int fm_write_context_kv(const void *kv, int64_t tokens, int32_t layers, int32_t heads,
                                   int32_t head_dim, const int64_t *positions, const int64_t *slots,
                                   const float *k_norm_weight, const float *rope_cos,
                                   const float *rope_sin, int64_t rope_row_stride,
                                   int64_t rope_pair_stride, int64_t rope_rows,
                                   const int64_t *cache_ptrs, int32_t num_caches,
                                   int32_t heads_per_cache, int64_t stride_block,
                                   int64_t stride_head, int64_t stride_token, int64_t v_offset,
                                   int32_t page_size, float eps, void *stream) {
  FM_REQUIRE(tokens >= 0 && layers > 0 && heads > 0, "bad sizes");
  if (tokens == 0) return FM_OK;
  if (head_dim != 64 && head_dim != 128)
    return fail(FM_ERR_UNSUPPORTED, "head_dim %d not supported (64 or 128)", head_dim);
  FM_REQUIRE(kv && positions && slots && k_norm_weight && rope_cos && rope_sin && cache_ptrs,
             "NULL pointer");
  FM_REQUIRE(heads_per_cache > 0 && page_size > 0, "bad cache geometry");
  FM_REQUIRE((int64_t)num_caches * heads_per_cache >= (int64_t)layers * heads,
             "%d caches of %d heads cannot hold %d x %d heads", num_caches, heads_per_cache, layers,
             heads);
  FM_REQUIRE(((uintptr_t)kv & 15) == 0, "kv must be 16-byte aligned");
  FM_REQUIRE(stride_block % 8 == 0 && stride_head % 8 == 0 && stride_token % 8 == 0 &&
                 v_offset % 8 == 0,
             "cache strides must be multiples of 8 elements");
  KvWriteArgs a{};
  a.kv = (const uint16_t *)kv;
  a.rows = tokens * layers * heads;
  a.layers = layers;
  a.heads = heads;
  a.positions = positions;
  a.k_norm = k_norm_weight;
  a.rope = Rope{rope_cos, rope_sin, rope_row_stride, rope_pair_stride, rope_rows};
  a.eps = eps;
  a.slots = slots;
  a.cache_ptrs = cache_ptrs;
  a.num_caches = num_caches;
  a.heads_per_cache = heads_per_cache;
  a.page_size = page_size;
  a.s_block = stride_block;
  a.s_head = stride_head;
  a.s_token = stride_token;
  a.v_offset = v_offset;
  return launch_kv_write<false>(a, head_dim, (hipStream_t)stream);
}

extern "C" int fm_write_context_kv_pool(const void *kv, int64_t tokens, int32_t layers,
                                        int32_t heads, int32_t head_dim, const int64_t *meta,
                                        const float *k_norm_weight, const float *rope_cos,
                                        const float *rope_sin, int64_t rope_row_stride,
                                        int64_t rope_pair_stride, int64_t rope_rows,
                                        const int64_t *positions, const int64_t *locs,
                                        const int32_t *commit_lens, int64_t locs_row_width,
                                        float eps, void *stream) {
  FM_REQUIRE(tokens >= 0 && layers > 0 && heads > 0, "bad sizes");
  if (tokens == 0) return FM_OK;
  if (head_dim != 64 && head_dim != 128)
    return fail(FM_ERR_UNSUPPORTED, "head_dim %d not supported (64 or 128)", head_dim);
  FM_REQUIRE(kv && meta && k_norm_weight && rope_cos && rope_sin && positions && locs,
             "NULL pointer");
  FM_REQUIRE(commit_lens == nullptr || locs_row_width > 0, "commit_lens needs locs_row_width > 0");
  FM_REQUIRE(((uintptr_t)kv & 15) == 0, "kv must be 16-byte aligned");
  KvWriteArgs a{};
  a.kv = (const uint16_t *)kv;
  a.rows = tokens * layers * heads;
  a.layers = layers;
  a.heads = heads;
  a.positions = positions;
  a.k_norm = k_norm_weight;
  a.rope = Rope{rope_cos, rope_sin, rope_row_stride, rope_pair_stride, rope_rows};
  a.eps = eps;
  a.meta = meta;
  a.locs = locs;
  a.commit_lens = commit_lens;
  a.row_width = locs_row_width > 0 ? locs_row_width : 1;
  return launch_kv_write<true>(a, head_dim, (hipStream_t)stream);
}

extern "C" int fm_write_context_kv_fp8(const void *kv, int64_t tokens, int32_t layers, int32_t heads,
                                       int32_t head_dim, const int64_t *positions, const int64_t *slots,
                                       const float *k_norm_weight, const float *rope_cos,
                                       const float *rope_sin, int64_t rope_row_stride,
                                       int64_t rope_pair_stride, int64_t rope_rows,
                                       const int64_t *cache_ptrs, int32_t num_caches,
                                       int32_t heads_per_cache, int64_t stride_block,
                                       int64_t stride_head, int64_t stride_token, int64_t v_offset,
                                       int32_t page_size, const float *scales, float eps, void *stream) {
  FM_REQUIRE(tokens >= 0 && layers > 0 && heads > 0, "bad sizes");
  if (tokens == 0) return FM_OK;
  if (head_dim != 64 && head_dim != 128)
    return fail(FM_ERR_UNSUPPORTED, "head_dim %d not supported (64 or 128)", head_dim);
  FM_REQUIRE(kv && positions && slots && k_norm_weight && rope_cos && rope_sin && cache_ptrs && scales,
             "NULL pointer");
  FM_REQUIRE(heads_per_cache > 0 && page_size > 0, "bad cache geometry");
  FM_REQUIRE((int64_t)num_caches * heads_per_cache >= (int64_t)layers * heads,
             "%d caches of %d heads cannot hold %d x %d heads", num_caches, heads_per_cache, layers,
             heads);
  FM_REQUIRE(((uintptr_t)kv & 15) == 0, "kv must be 16-byte aligned");
  FM_REQUIRE(stride_block % 8 == 0 && stride_head % 8 == 0 && stride_token % 8 == 0 &&
                 v_offset % 8 == 0,
             "cache strides must be multiples of 8 elements");
  KvWriteArgs a{};
  a.kv = (const uint16_t *)kv;
  a.rows = tokens * layers * heads;
  a.layers = layers;
  a.heads = heads;
  a.positions = positions;
  a.k_norm = k_norm_weight;
  a.rope = Rope{rope_cos, rope_sin, rope_row_stride, rope_pair_stride, rope_rows};
  a.eps = eps;
  a.slots = slots;
  a.cache_ptrs = cache_ptrs;
  a.num_caches = num_caches;
  a.heads_per_cache = heads_per_cache;
  a.page_size = page_size;
  a.s_block = stride_block;
  a.s_head = stride_head;
  a.s_token = stride_token;
  a.v_offset = v_offset;
  a.scales = scales;
  return launch_kv_write<false, true>(a, head_dim, (hipStream_t)stream);
}

extern "C" int fm_write_context_kv_pool_fp8(const void *kv, int64_t tokens, int32_t layers,
                                            int32_t heads, int32_t head_dim, const int64_t *meta,
                                            const float *k_norm_weight, const float *rope_cos,
                                            const float *rope_sin, int64_t rope_row_stride,
                                            int64_t rope_pair_stride, int64_t rope_rows,
                                            const int64_t *positions, const int64_t *locs,
                                            const int32_t *commit_lens, int64_t locs_row_width,
                                            float k_scale, float v_scale, float eps, void *stream) {
  FM_REQUIRE(tokens >= 0 && layers > 0 && heads > 0, "bad sizes");
  if (tokens == 0) return FM_OK;
  if (head_dim != 64 && head_dim != 128)
    return fail(FM_ERR_UNSUPPORTED, "head_dim %d not supported (64 or 128)", head_dim);
  FM_REQUIRE(kv && meta && k_norm_weight && rope_cos && rope_sin && positions && locs,
             "NULL pointer");
  FM_REQUIRE(commit_lens == nullptr || locs_row_width > 0, "commit_lens needs locs_row_width > 0");
  FM_REQUIRE(((uintptr_t)kv & 15) == 0, "kv must be 16-byte aligned");
  FM_REQUIRE(k_scale > 0.f && v_scale > 0.f, "scales must be positive");
  KvWriteArgs a{};
  a.kv = (const uint16_t *)kv;
  a.rows = tokens * layers * heads;
  a.layers = layers;
  a.heads = heads;
  a.positions = positions;
  a.k_norm = k_norm_weight;
  a.rope = Rope{rope_cos, rope_sin, rope_row_stride, rope_pair_stride, rope_rows};
  a.eps = eps;
  a.meta = meta;
  a.locs = locs;
  a.commit_lens = commit_lens;
  a.row_width = locs_row_width > 0 ? locs_row_width : 1;
  a.k_scale = k_scale;
  a.v_scale = v_scale;
  return launch_kv_write<true, true>(a, head_dim, (hipStream_t)stream);
}
