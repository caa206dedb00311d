// The draft step's token selection and noise:
//   - argmax over the vocabulary per row, the first index among equals
//     (flashmap/vllm/fold.py:117-128, split_argmax);
//   - the fused sampler: per row the argmax of its logits (greedy rows) or of
//     logit / T - log(-log u) (Gumbel-max, a sample of softmax(logits / T)) with u from
//     Philox at offset row * V + col (flashmap/sglang/kernels.py:195-247, sample_rows);
//   - keyed standard normals, row i keyed by seeds[rows[i]] * 1000003 + positions[i]
//     (flashmap/vllm/kernels.py:367-410, seeded_normal).
//
// The random stream is Triton's tl.rand / tl.randn, word for word: Philox-4x32 with 10
// rounds (Salmon et al., SC 2011) keyed by the seed's low and high words, counter
// (offset, 0, 0, 0) for the int32 offsets both kernels use; a word x maps to
// (x as int32, negatives folded by ~x) * 4.6566127342e-10f; a normal is
// sqrt(-2 log(max(u1, 1e-7))) * cos(6.2831855f * u2) of the first two words.
//
// Selection: one 256-thread workgroup per (tile of logits, row) streams the tile with
// 16-byte loads, keys it in registers (no noise buffer) and reduces (key, index) over the
// wavefront and then the workgroup; a one-wavefront-per-row pass merges the tiles. Tiles
// are 16384 logits for the argmax and 8192 for the sampler (SEL_TILE_*, below). NaN
// counts as the largest key, the first NaN winning (torch.argmax's rule).
#include <math.h>
#include <stdint.h>

#include "fm_device.h"
#include "fm_host.h"

namespace fm {

constexpr int SEL_THREADS = 256;
// Logits per workgroup. The argmax is HBM-bound: 64 per thread keep more bytes in flight
// per wavefront (1024 x 151936 bf16 logits in 64 us against 71 us with 32 per thread). The
// sampler is bound by Philox's ALU work and gains from more workgroups: 32 per thread
// (364 us against 437 us with 64).
constexpr int SEL_TILE_ARGMAX = 16384;
constexpr int SEL_TILE_SAMPLE = 8192;
__host__ __device__ constexpr int sel_tile(bool sample) { return sample ? SEL_TILE_SAMPLE : SEL_TILE_ARGMAX; }
constexpr int NOISE_COLS = 1024;  // columns per workgroup of seeded normals (4 per thread)

enum LogitType { LOGITS_BF16 = 0, LOGITS_F16 = 1, LOGITS_F32 = 2 };

__device__ __forceinline__ void philox4x32_10(uint32_t (&c)[4], uint32_t k0, uint32_t k1) {
#pragma unroll
  for (int r = 0; r < 10; ++r) {
    const uint64_t p0 = (uint64_t)0xD2511F53u * c[0];
    const uint64_t p1 = (uint64_t)0xCD9E8D57u * c[2];
    const uint32_t n0 = (uint32_t)(p1 >> 32) ^ c[1] ^ k0;
    const uint32_t n2 = (uint32_t)(p0 >> 32) ^ c[3] ^ k1;
    c[0] = n0;
    c[1] = (uint32_t)p1;
    c[2] = n2;
    c[3] = (uint32_t)p0;
    k0 += 0x9E3779B9u;
    k1 += 0xBB67AE85u;
  }
}

__device__ __forceinline__ float word_to_uniform(uint32_t w) {
  const int32_t i = (int32_t)w;
  return (float)(i < 0 ? ~i : i) * 4.6566127342e-10f;
}

// (key, index) order: NaN above everything (the first NaN wins), else larger key, then
// smaller index.
__device__ __forceinline__ bool better(float k, int32_t i, float bk, int32_t bi) {
  if (k != k) return bk == bk || i < bi;
  if (bk != bk) return false;
  return k > bk || (k == bk && i < bi);
}

__device__ __forceinline__ void wave_best(float &bk, int32_t &bi) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    const float k2 = __shfl_xor(bk, o);
    const int32_t i2 = __shfl_xor(bi, o);
    if (better(k2, i2, bk, bi)) bk = k2, bi = i2;
  }
}

template <int TY>
__device__ __forceinline__ float logit_at(const char *row, int64_t col) {
  if (TY == LOGITS_BF16) return bf16_to_f32(reinterpret_cast<const uint16_t *>(row)[col]);
  if (TY == LOGITS_F16) return (float)reinterpret_cast<const _Float16 *>(row)[col];
  return reinterpret_cast<const float *>(row)[col];
}

// Eight consecutive logits starting at col (16-byte aligned for 2-byte types, two
// 16-byte loads for float32).
template <int TY>
__device__ __forceinline__ void logits8(const char *row, int64_t col, float (&x)[8]) {
  if (TY == LOGITS_F32) {
    const u32x4_t a = load16(row + col * 4), b = load16(row + col * 4 + 16);
#pragma unroll
    for (int j = 0; j < 4; ++j) x[j] = __uint_as_float(a[j]), x[4 + j] = __uint_as_float(b[j]);
  } else {
    const u32x4_t a = load16(row + col * 2);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      if (TY == LOGITS_BF16) {
        x[2 * j] = bf16_lo(a[j]);
        x[2 * j + 1] = __uint_as_float(a[j] & 0xFFFF0000u);
      } else {
        // through the by-value helpers: a bit cast applied to the vector element a[j]
        // itself is lowered as a cast of a[0]
        x[2 * j] = f16_lo(a[j]);
        x[2 * j + 1] = f16_hi(a[j]);
      }
    }
  }
}

struct SelectArgs {
  const char *logits;
  int64_t row_bytes;  // row stride in bytes
  int64_t vocab;
  int32_t n_tiles, vec;  // vec: rows 16-byte aligned, 8-logit chunks may be loaded whole
  const float *temps;    // sampling only
  const uint8_t *greedy;
  const int64_t *seed;
  float *best;     // (rows, n_tiles)
  int32_t *index;  // (rows, n_tiles)
};

// Per (tile, row): the tile's best key and its first index.
template <int TY, bool SAMPLE>
__global__ __launch_bounds__(SEL_THREADS) void select_tiles_kernel(const SelectArgs a) {
  const int tile = blockIdx.x;
  const int64_t row = blockIdx.y;
  const char *src = a.logits + row * a.row_bytes;
  bool noisy = false;
  float temp = 1.f;
  uint32_t k0 = 0, k1 = 0;
  if (SAMPLE) {
    noisy = a.greedy[row] == 0;
    temp = a.temps[row];
    const uint64_t s = (uint64_t)a.seed[0];
    k0 = (uint32_t)s;
    k1 = (uint32_t)(s >> 32);
  }
  // int32 offsets row * V + col, as the reference's kernel forms them
  const uint32_t row_off = (uint32_t)row * (uint32_t)a.vocab;
  float bk = -INFINITY;
  int32_t bi = INT32_MAX;
  auto visit = [&](int64_t col, float x) {
    float key = x;
    if (SAMPLE && noisy) {
      uint32_t c[4] = {row_off + (uint32_t)col, 0u, 0u, 0u};
      philox4x32_10(c, k0, k1);
      const float u = word_to_uniform(c[0]);
      key = x / temp - logf(-logf(u));
    }
    // A thread visits its logits in increasing index order: a strictly larger key, the
    // first one, or a first NaN over a number takes the place (branch-free); the full
    // order settles ties between threads.
    const bool take = key > bk || bi == INT32_MAX || (key != key && bk == bk);
    bk = take ? key : bk;
    bi = take ? (int32_t)col : bi;
  };
  constexpr int TILE = sel_tile(SAMPLE);
  const int64_t base = (int64_t)tile * TILE;
  constexpr int IT = TILE / (8 * SEL_THREADS);
  if (a.vec && base + TILE <= a.vocab) {  // a whole tile: every load in flight first
    float x[IT][8];
#pragma unroll
    for (int it = 0; it < IT; ++it) logits8<TY>(src, base + 8 * ((int64_t)it * SEL_THREADS + threadIdx.x), x[it]);
#pragma unroll
    for (int it = 0; it < IT; ++it)
#pragma unroll
      for (int j = 0; j < 8; ++j) visit(base + 8 * ((int64_t)it * SEL_THREADS + threadIdx.x) + j, x[it][j]);
  } else {  // the vocabulary's last, partial tile (or unaligned rows)
#pragma unroll
    for (int it = 0; it < IT; ++it) {
      const int64_t col0 = base + 8 * ((int64_t)it * SEL_THREADS + threadIdx.x);
      if (col0 >= a.vocab) break;
      if (a.vec && col0 + 8 <= a.vocab) {
        float x[8];
        logits8<TY>(src, col0, x);
#pragma unroll
        for (int j = 0; j < 8; ++j) visit(col0 + j, x[j]);
      } else {
        for (int j = 0; j < 8 && col0 + j < a.vocab; ++j) visit(col0 + j, logit_at<TY>(src, col0 + j));
      }
    }
  }
  wave_best(bk, bi);
  __shared__ float sk[SEL_THREADS / 64];
  __shared__ int32_t si[SEL_THREADS / 64];
  const int w = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) sk[w] = bk, si[w] = bi;
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int v = 1; v < SEL_THREADS / 64; ++v)
      if (better(sk[v], si[v], bk, bi)) bk = sk[v], bi = si[v];
    a.best[row * a.n_tiles + tile] = bk;
    a.index[row * a.n_tiles + tile] = bi;
  }
}

// Per row (one wavefront): the best of its tiles.
__global__ __launch_bounds__(64) void select_rows_kernel(const float *best, const int32_t *index, int32_t n_tiles,
                                                         int64_t *out) {
  const int64_t row = blockIdx.x;
  float bk = -INFINITY;
  int32_t bi = INT32_MAX;
  for (int t = threadIdx.x; t < n_tiles; t += 64) {
    const float k = best[row * n_tiles + t];
    const int32_t i = index[row * n_tiles + t];
    if (better(k, i, bk, bi)) bk = k, bi = i;
  }
  wave_best(bk, bi);
  if (threadIdx.x == 0) out[row] = bi;
}

struct NoiseArgs {
  const int64_t *seeds;
  const void *rows;
  const void *positions;
  int32_t rows_64, pos_64;  // index widths: int64 (1) or int32 (0)
  int64_t n_cols, out_stride;
  float scale;
  float *out;
};

__global__ __launch_bounds__(256) void seeded_normal_kernel(const NoiseArgs a) {
  const int64_t row = blockIdx.y;
  const int64_t state = a.rows_64 ? reinterpret_cast<const int64_t *>(a.rows)[row]
                                  : (int64_t)reinterpret_cast<const int32_t *>(a.rows)[row];
  const int64_t pos = a.pos_64 ? reinterpret_cast<const int64_t *>(a.positions)[row]
                               : (int64_t)reinterpret_cast<const int32_t *>(a.positions)[row];
  const uint64_t seed = state >= 0 ? (uint64_t)a.seeds[state] : 0ull;
  const uint64_t key = seed * 1000003ull + (uint64_t)pos;  // int64 arithmetic, wrapping
  const uint32_t k0 = (uint32_t)key, k1 = (uint32_t)(key >> 32);
  float *dst = a.out + row * a.out_stride;
#pragma unroll
  for (int k = 0; k < NOISE_COLS / 256; ++k) {
    const int64_t col = (int64_t)blockIdx.x * NOISE_COLS + k * 256 + threadIdx.x;
    if (col >= a.n_cols) break;
    uint32_t c[4] = {(uint32_t)col, 0u, 0u, 0u};
    philox4x32_10(c, k0, k1);
    const float u1 = fmaxf(1.0e-7f, word_to_uniform(c[0]));
    const float u2 = word_to_uniform(c[1]);
    const float r = sqrtf(-2.0f * logf(u1));
    dst[col] = r * cosf(6.2831855f * u2) * a.scale;
  }
}

static size_t select_ws_offset(int64_t rows, int64_t n_tiles) {
  return ((size_t)(rows * n_tiles) * sizeof(float) + 255) & ~(size_t)255;
}

static int64_t select_tiles(int64_t vocab, bool sample) { return (vocab + sel_tile(sample) - 1) / sel_tile(sample); }

static int run_select(const void *logits, int32_t dtype, int64_t rows, int64_t vocab, int64_t row_stride,
                      const float *temps, const uint8_t *greedy, const int64_t *seed, int64_t *out, void *ws,
                      size_t ws_bytes, void *stream) {
  FM_REQUIRE(rows >= 0 && vocab >= 0, "bad sizes");
  if (rows == 0) return FM_OK;
  FM_REQUIRE(vocab > 0, "an empty vocabulary has no argmax");
  FM_REQUIRE(vocab <= INT32_MAX, "vocabulary of %lld above 2^31 - 1", (long long)vocab);
  FM_REQUIRE(rows <= 65535, "at most 65535 rows per call, got %lld", (long long)rows);
  FM_REQUIRE(logits && out && ws, "NULL logits/out/workspace");
  FM_REQUIRE(dtype == LOGITS_BF16 || dtype == LOGITS_F16 || dtype == LOGITS_F32, "unknown logits dtype %d", dtype);
  FM_REQUIRE(row_stride >= vocab, "row stride %lld below the vocabulary %lld", (long long)row_stride,
             (long long)vocab);
  const bool sample = temps != nullptr;
  const int64_t n_tiles = select_tiles(vocab, sample);
  const size_t need = select_ws_offset(rows, n_tiles) + (size_t)(rows * n_tiles) * sizeof(int32_t);
  if (ws_bytes < need) return fail(FM_ERR_WORKSPACE, "workspace of %zu bytes, %zu needed", ws_bytes, need);
  const int es = dtype == LOGITS_F32 ? 4 : 2;
  SelectArgs a{};
  a.logits = (const char *)logits;
  a.row_bytes = row_stride * es;
  a.vocab = vocab;
  a.n_tiles = (int32_t)n_tiles;
  a.vec = ((uintptr_t)logits % 16 == 0 && a.row_bytes % 16 == 0) ? 1 : 0;
  a.temps = temps;
  a.greedy = greedy;
  a.seed = seed;
  a.best = (float *)ws;
  a.index = (int32_t *)((char *)ws + select_ws_offset(rows, n_tiles));
  hipStream_t s = (hipStream_t)stream;
  const dim3 grid((unsigned)n_tiles, (unsigned)rows);
#define FM_SEL(TY)                                                                          \
  do {                                                                                      \
    if (sample)                                                                             \
      hipLaunchKernelGGL((select_tiles_kernel<TY, true>), grid, dim3(SEL_THREADS), 0, s, a);  \
    else                                                                                    \
      hipLaunchKernelGGL((select_tiles_kernel<TY, false>), grid, dim3(SEL_THREADS), 0, s, a); \
  } while (0)
  if (dtype == LOGITS_BF16)
    FM_SEL(LOGITS_BF16);
  else if (dtype == LOGITS_F16)
    FM_SEL(LOGITS_F16);
  else
    FM_SEL(LOGITS_F32);
#undef FM_SEL
  FM_CHECK_HIP(hipGetLastError());
  hipLaunchKernelGGL(select_rows_kernel, dim3((unsigned)rows), dim3(64), 0, s, a.best, a.index, a.n_tiles, out);
  FM_CHECK_HIP(hipGetLastError());
  return FM_OK;
}

}  // namespace fm

using namespace fm;

extern "C" size_t fm_select_workspace_bytes(int64_t rows, int64_t vocab) {
  if (rows <= 0 || vocab <= 0) return 0;
  const int64_t n_tiles = select_tiles(vocab, true);  // the finer tiling: enough for both
  return select_ws_offset(rows, n_tiles) + (size_t)(rows * n_tiles) * sizeof(int32_t);
}

extern "C" int fm_argmax_rows(const void *logits, int32_t dtype, int64_t rows, int64_t vocab, int64_t row_stride,
                              int64_t *out, void *workspace, size_t workspace_bytes, void *stream) {
  clear_error();
  return run_select(logits, dtype, rows, vocab, row_stride, nullptr, nullptr, nullptr, out, workspace,
                    workspace_bytes, stream);
}

extern "C" int fm_sample_rows(const void *logits, int32_t dtype, int64_t rows, int64_t vocab, int64_t row_stride,
                              const float *temperatures, const uint8_t *greedy, const int64_t *seed, int64_t *out,
                              void *workspace, size_t workspace_bytes, void *stream) {
  clear_error();
  FM_REQUIRE(rows == 0 || (temperatures && greedy && seed), "NULL temperatures/greedy/seed");
  return run_select(logits, dtype, rows, vocab, row_stride, temperatures, greedy, seed, out, workspace,
                    workspace_bytes, stream);
}

extern "C" int fm_seeded_normal(const int64_t *seeds, const void *rows, int32_t rows_int64, const void *positions,
                                int32_t positions_int64, int64_t num_rows, int64_t n_cols, float scale, float *out,
                                int64_t out_row_stride, void *stream) {
  clear_error();
  FM_REQUIRE(num_rows >= 0 && n_cols >= 0, "bad sizes");
  if (num_rows == 0 || n_cols == 0) return FM_OK;
  FM_REQUIRE(seeds && rows && positions && out, "NULL seeds/rows/positions/out");
  FM_REQUIRE(num_rows <= 65535, "at most 65535 rows per call, got %lld", (long long)num_rows);
  FM_REQUIRE(out_row_stride >= n_cols, "output row stride below n_cols");
  NoiseArgs a{seeds, rows, positions, rows_int64 ? 1 : 0, positions_int64 ? 1 : 0, n_cols, out_row_stride, scale, out};
  const dim3 grid((unsigned)((n_cols + NOISE_COLS - 1) / NOISE_COLS), (unsigned)num_rows);
  hipLaunchKernelGGL(seeded_normal_kernel, grid, dim3(256), 0, (hipStream_t)stream, a);
  FM_CHECK_HIP(hipGetLastError());
  return FM_OK;
}
