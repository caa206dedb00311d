// a4: the K side of the QK-norm prologue. Every committed context row's keys are
// k-normed and rotated at the row's context position and stored, with its values,
// into the engine's KV layout. One wavefront transforms 16 (token, global head) rows
// in the row-quad layout (fm_device.h), with the same arithmetic as the Q prologue.
//   vLLM:   kv (tokens, layers, 2, heads, D) -> paged caches (blocks, heads, page, 2D)
//           (flashmap/vllm/kernels.py:235-364)
//   SGLang: the same kv rows -> per-layer (pool, heads, D) key/value buffers
//           (sglang's fused_kv_norm_rope_write as flashmap/sglang/model.py:746-766
//           calls it; flashmap/sglang/kernels.py:283-357 is its fp8 twin)
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
};

template <int D, bool POOL>
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

template <bool POOL>
static int launch_kv_write(const KvWriteArgs &a, int head_dim, hipStream_t s) {
  const int64_t grid = (a.rows + 63) / 64;
  FM_REQUIRE(grid < (1ll << 31), "too many rows");
  if (head_dim == 128)
    kv_write_kernel<128, POOL><<<dim3((unsigned)grid), dim3(256), 0, s>>>(a);
  else
    kv_write_kernel<64, POOL><<<dim3((unsigned)grid), dim3(256), 0, s>>>(a);
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
