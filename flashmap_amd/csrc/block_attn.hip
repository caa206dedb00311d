// a5/a6/a7: block attention of the K draft slots onto the context keys/values, for
// contiguous (FlashMapCache), block-paged (vLLM) and token-paged (SGLang) KV.
//
// Work decomposition (split-KV, "stream-K" style). A unit is (sequence b, KV head h,
// row group rg): the G query heads sharing KV head h times the q_len draft rows,
// packed into 16-row MFMA blocks (row r = query head h*G + r / q_len at token
// r % q_len, the GQA row convention of flashmap/sglang/verify_attention.py:77-79).
// Each unit's context is cut into tiles of 32 positions; all units' tiles form one
// line (sequence-major, then head, then row group) that is cut into num_wg equal
// shares, one per workgroup of the persistent grid. A workgroup walks its share unit
// by unit (a "segment" per unit); its four wavefronts take the segment's tiles in
// turn. A unit wholly inside one share is finished in place (bf16 out); a unit cut
// between shares leaves one fp32 partial (normalized O and log-sum-exp) per share and
// is merged by attn_combine_kernel (the LSE merge of
// flashmap/sglang/verify_attention.py:184-233). Only the first and last segment of a
// share can be cut, so two partial slots per workgroup suffice.
//
// Per tile and wavefront (16-row blocks rb, 16-position halves pb):
//   S^T[pos][row] = K Q^T     (v_mfma_f32_16x16x32_bf16, A = K rows straight from HBM,
//                              B = Q rows in registers)
//   online softmax on S^T: each lane owns one row (lane % 16), so the running max,
//   sum and rescale are lane-local; only the max crosses the 4 lane groups.
//   O^T[d][row] += V^T P^T    (B = P^T is exactly the S^T accumulator layout rounded
//                              to bf16; A = V^T is read transposed out of LDS, where
//                              the V tile was staged with 16-byte loads)
// K is read from HBM with 16-byte loads in MFMA operand layout (64 contiguous bytes
// per row per instruction); V with fully contiguous 16-byte loads. The next tile's K
// and V are loaded while the current one is computed (register double buffer).
#include <math.h>

#include <mutex>

#include "fm_device.h"
#include "fm_host.h"

namespace fm {

constexpr int TILE = 32;   // context positions per tile
constexpr int WAVES = 4;   // wavefronts per workgroup
constexpr int NRB_MAX = 5; // 16-row blocks per unit

enum Layout { CONTIG = 0, PAGED16 = 1, PAGED = 2 };

struct AttnArgs {
  const uint16_t *q;
  int64_t q_sb, q_st, q_sh;
  uint16_t *o;
  int64_t o_sb, o_st, o_sh;
  const int32_t *cu_q;
  int32_t q_len;  // rows per query head (max_seqlen_q)
  const uint16_t *k;
  const uint16_t *v;
  int64_t k_s0, k_s1, k_s2;  // CONTIG: batch, head, position; paged: page, head, token
  int64_t v_s0, v_s1, v_s2;
  const int32_t *table;
  int64_t table_stride, table_width, num_pages;
  int32_t page_size, page_shift;
  const int32_t *seqlens;  // NULL: every sequence has uniform_len positions
  int32_t uniform_len, uniform_tiles;
  int32_t batch, hkv, group, rgroups;
  float scale_log2;
  const float *qn_w;  // non-NULL: fused Q prologue
  Rope rope;
  const int64_t *q_pos;
  float eps;
  const int32_t *plan;  // tile prefix over sequences (NULL with seqlens == NULL)
  int32_t num_wg;
  float *part_o;
  float *part_lse;
};

__device__ __forceinline__ int32_t seq_len(const AttnArgs &a, int b) {
  if (a.seqlens == nullptr) return a.uniform_len;
  const int32_t L = a.seqlens[b];
  return L > 0 ? L : 0;
}
__device__ __forceinline__ int64_t tile_prefix(const AttnArgs &a, int b) {
  return a.plan ? (int64_t)a.plan[b] : (int64_t)b * a.uniform_tiles;
}
__device__ __forceinline__ int32_t q_rows_of(const AttnArgs &a, int b) {
  if (a.cu_q == nullptr) return a.q_len;
  const int32_t r = a.cu_q[b + 1] - a.cu_q[b];
  return r < a.q_len ? r : a.q_len;
}
// Element offset of query/output row (b, t, head) and the varlen row index of (b, t).
__device__ __forceinline__ int64_t q_token_index(const AttnArgs &a, int b, int t) {
  return a.cu_q ? (int64_t)a.cu_q[b] + t : (int64_t)b * a.q_len + t;
}

// The share [T0, T1) of workgroup w over `total` tiles, and the workgroup owning tile x.
__device__ __forceinline__ int64_t share_start(int64_t w, int64_t total, int64_t nw) {
  return w * total / nw;
}
__device__ __forceinline__ int64_t share_of(int64_t x, int64_t total, int64_t nw) {
  return ((x + 1) * nw - 1) / total;
}

// Offsets (elements) of the context rows of one 16-position half tile: rows
// p0 .. p0+15 clamped to the last valid position L-1, so padding positions re-read a
// valid row (their scores are masked) and table lookups stay inside the sequence.
template <int LAYOUT>
struct HalfRows {
  int64_t kbase, vbase;  // PAGED16 / CONTIG: offset of the half's first valid row
  int32_t lim;           // last valid row index inside the half
};

template <int LAYOUT>
__device__ __forceinline__ HalfRows<LAYOUT> half_rows(const AttnArgs &a, int b, int h, int p0,
                                                      int L) {
  HalfRows<LAYOUT> r;
  const int pe = p0 < L ? p0 : L - 1;
  r.lim = L - 1 - pe;
  if (LAYOUT == CONTIG) {
    r.kbase = (int64_t)b * a.k_s0 + (int64_t)h * a.k_s1 + (int64_t)pe * a.k_s2;
    r.vbase = (int64_t)b * a.v_s0 + (int64_t)h * a.v_s1 + (int64_t)pe * a.v_s2;
  } else if (LAYOUT == PAGED16) {
    int64_t col = pe >> a.page_shift;
    col = col < a.table_width ? col : a.table_width - 1;
    int64_t page = a.table[(int64_t)b * a.table_stride + col];
    page = page < 0 ? 0 : (page >= a.num_pages ? a.num_pages - 1 : page);
    const int64_t in_page = pe & (a.page_size - 1);
    r.kbase = page * a.k_s0 + (int64_t)h * a.k_s1 + in_page * a.k_s2;
    r.vbase = page * a.v_s0 + (int64_t)h * a.v_s1 + in_page * a.v_s2;
  } else {
    r.kbase = 0;
    r.vbase = 0;
  }
  return r;
}

// Offsets of one context position for the generic paged layout (any page size,
// including SGLang's page size 1).
__device__ __forceinline__ void paged_row(const AttnArgs &a, int b, int h, int p, int64_t &ko,
                                          int64_t &vo) {
  int64_t col = a.page_size == 1 ? p : p / a.page_size;
  col = col < a.table_width ? col : a.table_width - 1;
  int64_t page = a.table[(int64_t)b * a.table_stride + col];
  page = page < 0 ? 0 : (page >= a.num_pages ? a.num_pages - 1 : page);
  const int64_t in_page = a.page_size == 1 ? 0 : p - col * a.page_size;
  ko = page * a.k_s0 + (int64_t)h * a.k_s1 + in_page * a.k_s2;
  vo = page * a.v_s0 + (int64_t)h * a.v_s1 + in_page * a.v_s2;
}

template <int D>
struct TileRegs {
  u32x4_t kf[2][D / 32];  // K operand: half pb, k-step t: row 16 pb + n, channels 32t+8g..
  u32x4_t vr[D / 16];     // V rows for the LDS stage: load i covers rows RPL*i + lane/LPR
};

// Issue the loads of tile `lt` (positions 32*lt ..) of unit (b, h) into `r`.
template <int LAYOUT, int D>
__device__ __forceinline__ void issue_tile(const AttnArgs &a, TileRegs<D> &r, int b, int h,
                                           int lt, int L, int lane) {
  constexpr int KT = D / 32, VL = D / 16;
  constexpr int LPR = D / 8;     // lanes per V row (16-byte chunks per row)
  constexpr int RPL = 64 / LPR;  // V rows per load
  const int n = lane & 15, g = lane >> 4;
  const int base = lt * TILE;
  if (LAYOUT == PAGED) {
#pragma unroll
    for (int pb = 0; pb < 2; ++pb) {
      int p = base + 16 * pb + n;
      p = p < L ? p : L - 1;
      int64_t ko, vo;
      paged_row(a, b, h, p, ko, vo);
      const uint16_t *kp = a.k + ko + 8 * g;
#pragma unroll
      for (int t = 0; t < KT; ++t) r.kf[pb][t] = load16(kp + 32 * t);
    }
#pragma unroll
    for (int i = 0; i < VL; ++i) {
      int p = base + RPL * i + lane / LPR;
      p = p < L ? p : L - 1;
      int64_t ko, vo;
      paged_row(a, b, h, p, ko, vo);
      r.vr[i] = load16(a.v + vo + 8 * (lane % LPR));
    }
  } else {
    HalfRows<LAYOUT> hr[2];
    hr[0] = half_rows<LAYOUT>(a, b, h, base, L);
    hr[1] = half_rows<LAYOUT>(a, b, h, base + 16, L);
#pragma unroll
    for (int pb = 0; pb < 2; ++pb) {
      const int row = n < hr[pb].lim ? n : hr[pb].lim;
      const uint16_t *kp = a.k + hr[pb].kbase + (int64_t)row * a.k_s2 + 8 * g;
#pragma unroll
      for (int t = 0; t < KT; ++t) r.kf[pb][t] = load16(kp + 32 * t);
    }
#pragma unroll
    for (int i = 0; i < VL; ++i) {
      const int rv = RPL * i + lane / LPR;  // 0..31
      const int pb = rv >> 4;
      int row = rv & 15;
      row = row < hr[pb].lim ? row : hr[pb].lim;
      r.vr[i] = load16(a.v + hr[pb].vbase + (int64_t)row * a.v_s2 + 8 * (lane % LPR));
    }
  }
}

// Load the unit's query rows into MFMA operand registers (row-quad layout), applying
// the fused QK-RMSNorm + RoPE when requested. Rows past the unit's valid rows are 0.
template <int NRB, int D>
__device__ __forceinline__ void load_queries(const AttnArgs &a, u32x4_t (&qf)[NRB][D / 32], int b,
                                             int h, int rg, int lane) {
  constexpr int KT = D / 32;
  const int n = lane & 15, g = lane >> 4;
  const int qlen_b = q_rows_of(a, b);
#pragma unroll
  for (int rb = 0; rb < NRB; ++rb) {
    const int R = (rg * NRB + rb) * 16 + n;
    const int gq = R / a.q_len, tq = R - gq * a.q_len;
    const bool valid = gq < a.group && tq < qlen_b;
    const int64_t tok = q_token_index(a, b, valid ? tq : 0);
    const int64_t head = (int64_t)h * a.group + (valid ? gq : 0);
    const uint16_t *src =
        a.q + (a.cu_q ? tok * a.q_st : (int64_t)b * a.q_sb + (int64_t)tq * a.q_st) + head * a.q_sh +
        8 * g;
#pragma unroll
    for (int t = 0; t < KT; ++t) qf[rb][t] = valid ? load16(src + 32 * t) : u32x4_t{0, 0, 0, 0};
    if (a.qn_w != nullptr) {
      const int64_t rr = clamp_row(a.rope, valid ? (a.q_pos ? a.q_pos[tok] : tok) : 0);
      norm_rope_row<D>(qf[rb], a.qn_w, a.eps, a.rope, rr, g);
    }
  }
}

template <int NRB, int D>
struct WaveState {
  f32x4_t acc[NRB][D / 16];  // O^T[d = 16 db + 4 g + i][row = 16 rb + n]
  float m[NRB];              // running max (log2 domain), uniform over lane groups
  float l[NRB];              // running sum, lane-partial (this lane's positions)
};

// One tile: stage V in LDS, S^T = K Q^T, online softmax, O^T += V^T P^T.
template <int NRB, int D>
__device__ __forceinline__ void compute_tile(const AttnArgs &a, const TileRegs<D> &r,
                                             const u32x4_t (&qf)[NRB][D / 32],
                                             WaveState<NRB, D> &st, uint16_t *vs, int tile_base,
                                             int L, int lane) {
  constexpr int KT = D / 32, DB = D / 16, VL = D / 16;
  constexpr int LPR = D / 8, RPL = 64 / LPR;
  constexpr int VP = D + 4;  // LDS row pitch (elements): conflict-free transposed reads
  const int n = lane & 15, g = lane >> 4;

  // V rows into this wavefront's LDS stage.
#pragma unroll
  for (int i = 0; i < VL; ++i) {
    const int rv = RPL * i + lane / LPR;
    uint16_t *dst = vs + rv * VP + 8 * (lane % LPR);
    *reinterpret_cast<u32x2_t *>(dst) = u32x2_t{r.vr[i][0], r.vr[i][1]};
    *reinterpret_cast<u32x2_t *>(dst + 4) = u32x2_t{r.vr[i][2], r.vr[i][3]};
  }

  // S^T = K Q^T for both halves and every row block.
  f32x4_t s[2][NRB];
#pragma unroll
  for (int pb = 0; pb < 2; ++pb) {
#pragma unroll
    for (int rb = 0; rb < NRB; ++rb) {
      f32x4_t c = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int t = 0; t < KT; ++t) c = mfma_16x16x32(r.kf[pb][t], qf[rb][t], c);
      s[pb][rb] = c;
    }
  }
  if (tile_base + TILE > L) {
#pragma unroll
    for (int pb = 0; pb < 2; ++pb)
#pragma unroll
      for (int i = 0; i < 4; ++i)
        if (tile_base + 16 * pb + 4 * g + i >= L)
#pragma unroll
          for (int rb = 0; rb < NRB; ++rb) s[pb][rb][i] = -INFINITY;
  }

  // Online softmax (log2 domain) and P^T as the bf16 B operand.
  u32x4_t pk[NRB];
#pragma unroll
  for (int rb = 0; rb < NRB; ++rb) {
    float mx = s[0][rb][0];
#pragma unroll
    for (int pb = 0; pb < 2; ++pb)
#pragma unroll
      for (int i = 0; i < 4; ++i) mx = fmaxf(mx, s[pb][rb][i]);
    mx = max_over_groups(mx);
    const float mnew = fmaxf(st.m[rb], mx * a.scale_log2);
    const float alpha = __builtin_amdgcn_exp2f(st.m[rb] - mnew);
    st.m[rb] = mnew;
    float p[2][4];
    float ps = 0.f;
#pragma unroll
    for (int pb = 0; pb < 2; ++pb)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        p[pb][i] = __builtin_amdgcn_exp2f(fmaf(s[pb][rb][i], a.scale_log2, -mnew));
        ps += p[pb][i];
      }
    st.l[rb] = st.l[rb] * alpha + ps;
    pk[rb] = u32x4_t{pack_bf16x2(p[0][0], p[0][1]), pack_bf16x2(p[0][2], p[0][3]),
                     pack_bf16x2(p[1][0], p[1][1]), pack_bf16x2(p[1][2], p[1][3])};
#pragma unroll
    for (int db = 0; db < DB; ++db) st.acc[rb][db] *= alpha;
  }

  __builtin_amdgcn_wave_barrier();
  // O^T += V^T P^T: A operand row d = 16 db + n, reduction positions
  // {4g, 4g+1, 4g+2, 4g+3, 16+4g, .., 16+4g+3} (the S^T accumulator positions).
  const uint16_t *vcol = vs + 4 * g * VP + n;
#pragma unroll
  for (int db = 0; db < DB; ++db) {
    const uint16_t *c0 = vcol + 16 * db;
    u32x4_t vf;
    vf[0] = (uint32_t)c0[0 * VP] | ((uint32_t)c0[1 * VP] << 16);
    vf[1] = (uint32_t)c0[2 * VP] | ((uint32_t)c0[3 * VP] << 16);
    vf[2] = (uint32_t)c0[16 * VP] | ((uint32_t)c0[17 * VP] << 16);
    vf[3] = (uint32_t)c0[18 * VP] | ((uint32_t)c0[19 * VP] << 16);
#pragma unroll
    for (int rb = 0; rb < NRB; ++rb) st.acc[rb][db] = mfma_16x16x32(vf, pk[rb], st.acc[rb][db]);
  }
  __builtin_amdgcn_wave_barrier();
}

template <int NRB, int D>
constexpr int smem_bytes() {
  constexpr int stage = WAVES * TILE * (D + 4) * 2;
  constexpr int combine = 2 * NRB * (D / 16) * 64 * 16 + 2 * WAVES * NRB * 16 * 4;
  return stage > combine ? stage : combine;
}

template <int LAYOUT, int NRB, int D>
__global__ __launch_bounds__(256, 1) void attn_fwd_kernel(const AttnArgs a) {
  constexpr int DB = D / 16;
  constexpr int ROWS = NRB * 16;
  __shared__ __attribute__((aligned(16))) char smem[smem_bytes<NRB, D>()];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int n = lane & 15, g = lane >> 4;

  const int64_t ups = (int64_t)a.hkv * a.rgroups;
  const int64_t total = ups * tile_prefix(a, a.batch);
  const int64_t nw = a.num_wg;
  const int64_t T0 = share_start(blockIdx.x, total, nw);
  const int64_t T1 = share_start((int64_t)blockIdx.x + 1, total, nw);
  if (T0 >= T1) return;

  // Sequence of the first tile: the largest b with ups * prefix(b) <= T0.
  int b = 0;
  {
    int lo = 0, hi = a.batch;
    while (hi - lo > 1) {
      const int mid = (lo + hi) >> 1;
      if (ups * tile_prefix(a, mid) <= T0)
        lo = mid;
      else
        hi = mid;
    }
    b = lo;
  }

  uint16_t *vstage = reinterpret_cast<uint16_t *>(smem) + wave * TILE * (D + 4);
  float *obuf = reinterpret_cast<float *>(smem);                       // [2][NRB][DB][64][4]
  float *m_s = obuf + 2 * NRB * DB * 64 * 4;                           // [WAVES][ROWS]
  float *l_s = m_s + WAVES * ROWS;                                      // [WAVES][ROWS]

  int64_t t = T0;
  int seg = 0;
  while (t < T1) {
    while (b + 1 < a.batch && ups * tile_prefix(a, b + 1) <= t) ++b;
    const int64_t sb = ups * tile_prefix(a, b);
    const int tiles_b = (int)(tile_prefix(a, b + 1) - tile_prefix(a, b));
    const int64_t off = t - sb;
    const int ul = (int)(off / tiles_b);
    const int lt0 = (int)(off - (int64_t)ul * tiles_b);
    const int64_t rem = T1 - t;
    const int lt1 = (int64_t)(tiles_b - lt0) < rem ? tiles_b : lt0 + (int)rem;
    const int h = ul / a.rgroups, rg = ul - h * a.rgroups;
    const int L = seq_len(a, b);

    u32x4_t qf[NRB][D / 32];
    load_queries<NRB, D>(a, qf, b, h, rg, lane);

    WaveState<NRB, D> st;
#pragma unroll
    for (int rb = 0; rb < NRB; ++rb) {
      st.m[rb] = -INFINITY;
      st.l[rb] = 0.f;
#pragma unroll
      for (int db = 0; db < DB; ++db) st.acc[rb][db] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    }

    // This wavefront's tiles: lt0 + wave, + WAVES, ... (register double buffer).
    TileRegs<D> buf0, buf1;
    int lt = lt0 + wave;
    if (lt < lt1) issue_tile<LAYOUT, D>(a, buf0, b, h, lt, L, lane);
    while (lt < lt1) {
      int ltn = lt + WAVES;
      if (ltn < lt1) issue_tile<LAYOUT, D>(a, buf1, b, h, ltn, L, lane);
      compute_tile<NRB, D>(a, buf0, qf, st, vstage, lt * TILE, L, lane);
      lt = ltn;
      if (lt >= lt1) break;
      ltn = lt + WAVES;
      if (ltn < lt1) issue_tile<LAYOUT, D>(a, buf0, b, h, ltn, L, lane);
      compute_tile<NRB, D>(a, buf1, qf, st, vstage, lt * TILE, L, lane);
      lt = ltn;
    }

    // Merge the four wavefronts: common max, rescale, tree-sum of O^T in LDS.
#pragma unroll
    for (int rb = 0; rb < NRB; ++rb) st.l[rb] = sum_over_groups(st.l[rb]);
    __syncthreads();  // every wavefront is done with its V stage (aliased below)
    if (g == 0) {
#pragma unroll
      for (int rb = 0; rb < NRB; ++rb) {
        m_s[wave * ROWS + rb * 16 + n] = st.m[rb];
        l_s[wave * ROWS + rb * 16 + n] = st.l[rb];
      }
    }
    __syncthreads();
    float inv_l[NRB], lse[NRB];
#pragma unroll
    for (int rb = 0; rb < NRB; ++rb) {
      const int row = rb * 16 + n;
      float M = m_s[row];
#pragma unroll
      for (int w = 1; w < WAVES; ++w) M = fmaxf(M, m_s[w * ROWS + row]);
      float Lt = 0.f;
#pragma unroll
      for (int w = 0; w < WAVES; ++w) {
        const float mw = m_s[w * ROWS + row];
        Lt += mw == -INFINITY ? 0.f : l_s[w * ROWS + row] * __builtin_amdgcn_exp2f(mw - M);
      }
      const float f = st.m[rb] == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(st.m[rb] - M);
#pragma unroll
      for (int db = 0; db < DB; ++db) st.acc[rb][db] *= f;
      inv_l[rb] = Lt > 0.f ? 1.f / Lt : 0.f;
      lse[rb] = M + log2f(Lt);
    }
    f32x4_t *ob = reinterpret_cast<f32x4_t *>(obuf);
    if (wave >= 2) {
#pragma unroll
      for (int rb = 0; rb < NRB; ++rb)
#pragma unroll
        for (int db = 0; db < DB; ++db) ob[(((wave - 2) * NRB + rb) * DB + db) * 64 + lane] = st.acc[rb][db];
    }
    __syncthreads();
    if (wave < 2) {
#pragma unroll
      for (int rb = 0; rb < NRB; ++rb)
#pragma unroll
        for (int db = 0; db < DB; ++db) st.acc[rb][db] += ob[((wave * NRB + rb) * DB + db) * 64 + lane];
    }
    __syncthreads();
    if (wave == 1) {
#pragma unroll
      for (int rb = 0; rb < NRB; ++rb)
#pragma unroll
        for (int db = 0; db < DB; ++db) ob[(rb * DB + db) * 64 + lane] = st.acc[rb][db];
    }
    __syncthreads();
    if (wave == 0) {
#pragma unroll
      for (int rb = 0; rb < NRB; ++rb)
#pragma unroll
        for (int db = 0; db < DB; ++db) st.acc[rb][db] += ob[(rb * DB + db) * 64 + lane];
    }
    __syncthreads();  // LDS is free for the next segment's V stage

    if (wave == 0) {
      const bool whole = lt0 == 0 && lt1 == tiles_b;
      const int qlen_b = q_rows_of(a, b);
      const int64_t slot = 2 * (int64_t)blockIdx.x + (seg == 0 ? 0 : 1);
#pragma unroll
      for (int rb = 0; rb < NRB; ++rb) {
        const int R = (rg * NRB + rb) * 16 + n;
        const int gq = R / a.q_len, tq = R - gq * a.q_len;
        if (gq >= a.group || tq >= qlen_b) continue;
        if (whole) {
          const int64_t head = (int64_t)h * a.group + gq;
          uint16_t *dst = a.o +
                          (a.cu_q ? q_token_index(a, b, tq) * a.o_st
                                  : (int64_t)b * a.o_sb + (int64_t)tq * a.o_st) +
                          head * a.o_sh + 4 * g;
#pragma unroll
          for (int db = 0; db < DB; ++db) {
            const f32x4_t v = st.acc[rb][db] * inv_l[rb];
            *reinterpret_cast<u32x2_t *>(dst + 16 * db) =
                u32x2_t{pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3])};
          }
        } else {
          const int64_t prow = slot * ROWS + rb * 16 + n;
          float *dst = a.part_o + prow * D + 4 * g;
#pragma unroll
          for (int db = 0; db < DB; ++db)
            *reinterpret_cast<f32x4_t *>(dst + 16 * db) = st.acc[rb][db] * inv_l[rb];
          if (g == 0) a.part_lse[prow] = lse[rb];
        }
      }
    }
    t += lt1 - lt0;
    ++seg;
  }
}

// Merge the partials of units cut between workgroups; zero-fill empty sequences.
template <int D>
__global__ __launch_bounds__(256) void attn_combine_kernel(const AttnArgs a, int nrb) {
  const int rows = nrb * 16;
  const int64_t ups = (int64_t)a.hkv * a.rgroups;
  const int64_t unit = blockIdx.x;
  const int b = (int)(unit / ups);
  const int ul = (int)(unit - (int64_t)b * ups);
  const int h = ul / a.rgroups, rg = ul - h * a.rgroups;
  const int64_t pre = tile_prefix(a, b);
  const int tiles_b = (int)(tile_prefix(a, b + 1) - pre);
  const int qlen_b = q_rows_of(a, b);
  const int64_t total = ups * tile_prefix(a, a.batch);
  const int64_t nw = a.num_wg;
  int64_t wa = 0, wb = 0, U0 = 0;
  if (tiles_b > 0) {
    U0 = ups * pre + (int64_t)ul * tiles_b;
    wa = share_of(U0, total, nw);
    wb = share_of(U0 + tiles_b - 1, total, nw);
    if (wa == wb) return;  // finished in place by its workgroup
  }
  const bool a_first = tiles_b > 0 && U0 == share_start(wa, total, nw);
  constexpr int C = D / 4;  // float4 chunks per row
  for (int idx = threadIdx.x; idx < rows * C; idx += blockDim.x) {
    const int r = idx / C, c = idx - r * C;
    const int R = rg * rows + r;
    const int gq = R / a.q_len, tq = R - gq * a.q_len;
    if (gq >= a.group || tq >= qlen_b) continue;
    f32x4_t acc = {0.f, 0.f, 0.f, 0.f};
    if (tiles_b > 0) {
      float M = -INFINITY;
      for (int64_t w = wa; w <= wb; ++w) {
        const int64_t slot = (w == wa && !a_first) ? 2 * w + 1 : 2 * w;
        M = fmaxf(M, a.part_lse[slot * rows + r]);
      }
      float den = 0.f;
      for (int64_t w = wa; w <= wb; ++w) {
        const int64_t slot = (w == wa && !a_first) ? 2 * w + 1 : 2 * w;
        const float lw = a.part_lse[slot * rows + r];
        if (lw == -INFINITY) continue;
        const float f = __builtin_amdgcn_exp2f(lw - M);
        acc += f * *reinterpret_cast<const f32x4_t *>(a.part_o + (slot * rows + r) * D + 4 * c);
        den += f;
      }
      acc *= den > 0.f ? 1.f / den : 0.f;
    }
    const int64_t head = (int64_t)h * a.group + gq;
    uint16_t *dst = a.o +
                    (a.cu_q ? q_token_index(a, b, tq) * a.o_st
                            : (int64_t)b * a.o_sb + (int64_t)tq * a.o_st) +
                    head * a.o_sh + 4 * c;
    *reinterpret_cast<u32x2_t *>(dst) = u32x2_t{pack_bf16x2(acc[0], acc[1]), pack_bf16x2(acc[2], acc[3])};
  }
}

// plan[0] = 0, plan[b + 1] = plan[b] + ceil(max(seqlens[b], 0) / TILE).
__global__ __launch_bounds__(1024) void attn_plan_kernel(const int32_t *__restrict__ seqlens,
                                                         int32_t batch, int32_t *__restrict__ plan) {
  __shared__ int32_t buf[1024];
  int32_t carry = 0;
  if (threadIdx.x == 0) plan[0] = 0;
  for (int base = 0; base < batch; base += 1024) {
    const int i = base + threadIdx.x;
    int32_t L = i < batch ? seqlens[i] : 0;
    L = L > 0 ? L : 0;
    buf[threadIdx.x] = (L + TILE - 1) / TILE;
    __syncthreads();
    for (int off = 1; off < 1024; off <<= 1) {
      const int32_t add = threadIdx.x >= (unsigned)off ? buf[threadIdx.x - off] : 0;
      __syncthreads();
      buf[threadIdx.x] += add;
      __syncthreads();
    }
    if (i < batch) plan[i + 1] = carry + buf[threadIdx.x];
    carry += buf[1023];
    __syncthreads();
  }
}

// ---------------------------------------------------------------------------------
// Host side: grid sizing, workspace layout, dispatch.

typedef void (*AttnKernel)(const AttnArgs);

template <int LAYOUT, int D>
static AttnKernel pick_kernel(int nrb) {
  switch (nrb) {
    case 1: return attn_fwd_kernel<LAYOUT, 1, D>;
    case 2: return attn_fwd_kernel<LAYOUT, 2, D>;
    case 3: return attn_fwd_kernel<LAYOUT, 3, D>;
    case 4: return attn_fwd_kernel<LAYOUT, 4, D>;
    default: return attn_fwd_kernel<LAYOUT, 5, D>;
  }
}

static AttnKernel select_kernel(int layout, int d, int nrb) {
  if (d == 128) {
    if (layout == CONTIG) return pick_kernel<CONTIG, 128>(nrb);
    if (layout == PAGED16) return pick_kernel<PAGED16, 128>(nrb);
    return pick_kernel<PAGED, 128>(nrb);
  }
  if (layout == CONTIG) return pick_kernel<CONTIG, 64>(nrb);
  if (layout == PAGED16) return pick_kernel<PAGED16, 64>(nrb);
  return pick_kernel<PAGED, 64>(nrb);
}

struct RowPlan {
  int nrb;      // 16-row blocks per unit
  int rgroups;  // units per KV head
};

static RowPlan row_plan(int group, int q_len) {
  const int total = (group * q_len + 15) / 16;
  RowPlan p;
  if (total <= NRB_MAX) {
    p.rgroups = 1;
    p.nrb = total;
  } else {
    p.rgroups = (total + 3) / 4;
    p.nrb = (total + p.rgroups - 1) / p.rgroups;
  }
  return p;
}

static int env_int(const char *name, int dflt) {
  const char *v = getenv(name);
  if (v == nullptr || *v == 0) return dflt;
  return atoi(v);
}

// Workgroups resident per CU for a kernel (cached).
static int occupancy(AttnKernel k) {
  static std::mutex mu;
  static std::vector<std::pair<AttnKernel, int>> cache;
  std::lock_guard<std::mutex> lock(mu);
  for (auto &e : cache)
    if (e.first == k) return e.second;
  int blocks = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&blocks, reinterpret_cast<const void *>(k), 256,
                                                   0) != hipSuccess ||
      blocks < 1)
    blocks = 1;
  cache.push_back({k, blocks});
  return blocks;
}

struct Sizing {
  RowPlan rp;
  int num_wg;
  size_t plan_off, lse_off, o_off, bytes;
};

static size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

static int sizing(int layout, int batch, int q_len, int hq, int hkv, int d, int max_k,
                  bool need_plan, Sizing *sz) {
  DeviceInfo info;
  int rc = device_info(&info);
  if (rc != FM_OK) return rc;
  sz->rp = row_plan(hq / hkv, q_len);
  AttnKernel k = select_kernel(layout, d, sz->rp.nrb);
  const int64_t ups = (int64_t)hkv * sz->rp.rgroups;
  const int64_t tiles_bound = ups * batch * (((int64_t)max_k + TILE - 1) / TILE);
  const int min_tiles = env_int("FLASHMAP_SPLITKV_MIN_TILES", 8) > 0 ? env_int("FLASHMAP_SPLITKV_MIN_TILES", 8) : 1;
  int64_t nw = (int64_t)info.cus * occupancy(k);
  const int cap = env_int("FLASHMAP_SPLITKV_WORKGROUPS", 0);
  if (cap > 0) nw = cap;
  const int64_t want = (tiles_bound + min_tiles - 1) / min_tiles;
  if (want < nw) nw = want;
  if (nw < 1) nw = 1;
  sz->num_wg = (int)nw;
  const int64_t rows = (int64_t)sz->rp.nrb * 16;
  size_t off = 0;
  sz->plan_off = off;
  if (need_plan) off = align256(off + sizeof(int32_t) * ((size_t)batch + 1));
  sz->lse_off = off;
  off = align256(off + sizeof(float) * 2 * (size_t)nw * rows);
  sz->o_off = off;
  off = align256(off + sizeof(float) * 2 * (size_t)nw * rows * d);
  sz->bytes = off;
  return FM_OK;
}

static bool al16(const void *p) { return ((uintptr_t)p & 15) == 0; }

struct CommonIn {
  const void *q;
  int64_t q_sb, q_st, q_sh;
  void *out;
  int64_t o_sb, o_st, o_sh;
  const int32_t *cu_q;
  int32_t batch, q_len, max_k, hq, hkv, d;
  float scale;
  const float *qn_w, *rope_cos, *rope_sin;
  int64_t rope_rs, rope_ps, rope_rows;
  const int64_t *q_pos;
  float eps;
  const int32_t *plan;
  void *ws;
  size_t ws_bytes;
  hipStream_t stream;
};

static int run_attention(const CommonIn &c, int layout, AttnArgs a) {
  FM_REQUIRE(c.batch >= 0 && c.q_len >= 0 && c.hq > 0 && c.hkv > 0, "bad sizes");
  if (c.batch == 0 || c.q_len == 0) return FM_OK;
  if (c.d != 64 && c.d != 128) return fail(FM_ERR_UNSUPPORTED, "head_dim %d not supported (64 or 128)", c.d);
  FM_REQUIRE(c.hq % c.hkv == 0, "num_q_heads %d is not a multiple of num_kv_heads %d", c.hq, c.hkv);
  FM_REQUIRE(c.q && c.out, "NULL query/output");
  FM_REQUIRE(al16(c.q) && al16(c.out) && al16(a.k) && al16(a.v), "q/out/k/v must be 16-byte aligned");
  FM_REQUIRE(c.q_sb % 8 == 0 && c.q_st % 8 == 0 && c.q_sh % 8 == 0 && c.o_sb % 8 == 0 &&
                 c.o_st % 8 == 0 && c.o_sh % 8 == 0,
             "query/output strides must be multiples of 8 elements");
  FM_REQUIRE(a.k_s0 % 8 == 0 && a.k_s1 % 8 == 0 && a.k_s2 % 8 == 0 && a.v_s0 % 8 == 0 &&
                 a.v_s1 % 8 == 0 && a.v_s2 % 8 == 0,
             "key/value strides must be multiples of 8 elements");
  if (c.qn_w) FM_REQUIRE(c.rope_cos && c.rope_sin, "fused prologue needs the rotary table");
  const bool need_plan = a.seqlens != nullptr && c.plan == nullptr;
  Sizing sz;
  int rc = sizing(layout, c.batch, c.q_len, c.hq, c.hkv, c.d, c.max_k, need_plan, &sz);
  if (rc != FM_OK) return rc;
  if (c.ws == nullptr || c.ws_bytes < sz.bytes)
    return fail(FM_ERR_WORKSPACE, "workspace of %zu bytes, need %zu", c.ws_bytes, sz.bytes);
  FM_REQUIRE(al16(c.ws), "workspace must be 16-byte aligned");

  a.q = (const uint16_t *)c.q;
  a.q_sb = c.q_sb, a.q_st = c.q_st, a.q_sh = c.q_sh;
  a.o = (uint16_t *)c.out;
  a.o_sb = c.o_sb, a.o_st = c.o_st, a.o_sh = c.o_sh;
  a.cu_q = c.cu_q;
  a.q_len = c.q_len;
  a.batch = c.batch;
  a.hkv = c.hkv;
  a.group = c.hq / c.hkv;
  a.rgroups = sz.rp.rgroups;
  a.scale_log2 = c.scale * 1.4426950408889634f;
  a.qn_w = c.qn_w;
  a.rope = Rope{c.rope_cos, c.rope_sin, c.rope_rs, c.rope_ps, c.rope_rows};
  a.q_pos = c.q_pos;
  a.eps = c.eps;
  a.num_wg = sz.num_wg;
  char *ws = (char *)c.ws;
  a.part_lse = (float *)(ws + sz.lse_off);
  a.part_o = (float *)(ws + sz.o_off);
  if (a.seqlens != nullptr) {
    if (need_plan) {
      int32_t *plan = (int32_t *)(ws + sz.plan_off);
      attn_plan_kernel<<<1, 1024, 0, c.stream>>>(a.seqlens, c.batch, plan);
      FM_CHECK_HIP(hipGetLastError());
      a.plan = plan;
    } else {
      a.plan = c.plan;
    }
  } else {
    a.plan = nullptr;
    a.uniform_tiles = (a.uniform_len + TILE - 1) / TILE;
  }
  AttnKernel k = select_kernel(layout, c.d, sz.rp.nrb);
  void *kargs[] = {&a};
  profile_before(c.stream);
  const hipError_t lerr = hipLaunchKernel(reinterpret_cast<const void *>(k), dim3(sz.num_wg), dim3(256),
                                          kargs, 0, c.stream);
  profile_after(c.stream);
  if (lerr != hipSuccess) return fail(FM_ERR_HIP, "attention launch failed: %s", hipGetErrorString(lerr));
  const int64_t units = (int64_t)c.batch * c.hkv * sz.rp.rgroups;
  // With uniform lengths the host knows whether a unit is cut between workgroups (or
  // empty and in need of zeros); otherwise the combine kernel decides per unit.
  bool need_combine = true;
  if (a.seqlens == nullptr) {
    const int64_t total = units * a.uniform_tiles;
    need_combine = total == 0;
    for (int64_t w = 1; w < sz.num_wg && !need_combine; ++w) {
      const int64_t t0 = w * total / sz.num_wg;
      if (t0 % a.uniform_tiles != 0) need_combine = true;
    }
  }
  if (need_combine) {
    FM_REQUIRE(units < (1ll << 31), "too many units");
    if (c.d == 128)
      attn_combine_kernel<128><<<dim3((unsigned)units), dim3(256), 0, c.stream>>>(a, sz.rp.nrb);
    else
      attn_combine_kernel<64><<<dim3((unsigned)units), dim3(256), 0, c.stream>>>(a, sz.rp.nrb);
    FM_CHECK_HIP(hipGetLastError());
  }
  return FM_OK;
}

}  // namespace fm

using namespace fm;

extern "C" size_t fm_attn_plan_bytes(int32_t batch) {
  return sizeof(int32_t) * ((size_t)(batch < 0 ? 0 : batch) + 1);
}

extern "C" int fm_attn_plan(const int32_t *seqlens, int32_t batch, int32_t *plan, void *stream) {
  FM_REQUIRE(batch >= 0, "bad batch");
  FM_REQUIRE(plan != nullptr && (batch == 0 || seqlens != nullptr), "NULL pointer");
  attn_plan_kernel<<<1, 1024, 0, (hipStream_t)stream>>>(seqlens, batch, plan);
  FM_CHECK_HIP(hipGetLastError());
  return FM_OK;
}

extern "C" size_t fm_attn_workspace_bytes(int32_t batch, int32_t max_seqlen_q, int32_t num_q_heads,
                                          int32_t num_kv_heads, int32_t head_dim,
                                          int32_t max_seqlen_k, int device) {
  if (batch <= 0 || max_seqlen_q <= 0 || num_kv_heads <= 0 || num_q_heads % num_kv_heads != 0 ||
      (head_dim != 64 && head_dim != 128))
    return 256;
  int prev = 0;
  if (hipGetDevice(&prev) != hipSuccess) return 0;
  if (device != prev && hipSetDevice(device) != hipSuccess) return 0;
  // The largest need over the three layouts (their occupancy, hence grid, may differ),
  // with room for an in-call plan.
  size_t bytes = 0;
  int rc = FM_OK;
  for (int layout = CONTIG; layout <= PAGED && rc == FM_OK; ++layout) {
    Sizing sz;
    rc = sizing(layout, batch, max_seqlen_q, num_q_heads, num_kv_heads, head_dim, max_seqlen_k,
                true, &sz);
    if (rc == FM_OK && sz.bytes > bytes) bytes = sz.bytes;
  }
  if (device != prev) hipSetDevice(prev);
  return rc == FM_OK ? bytes : 0;
}

extern "C" int fm_block_attn_contig(
    const void *q, int64_t q_stride_batch, int64_t q_stride_token, int64_t q_stride_head, void *out,
    int64_t out_stride_batch, int64_t out_stride_token, int64_t out_stride_head,
    const int32_t *cu_seqlens_q, const void *k, int64_t k_stride_batch, int64_t k_stride_head,
    int64_t k_stride_pos, const void *v, int64_t v_stride_batch, int64_t v_stride_head,
    int64_t v_stride_pos, const int32_t *seqlens_k, int32_t kv_len, int32_t batch,
    int32_t max_seqlen_q, int32_t num_q_heads, int32_t num_kv_heads, int32_t head_dim,
    float softmax_scale, const float *q_norm_weight, const float *rope_cos, const float *rope_sin,
    int64_t rope_row_stride, int64_t rope_pair_stride, int64_t rope_rows,
    const int64_t *q_positions, float eps, const int32_t *plan, void *workspace,
    size_t workspace_bytes, void *stream) {
  FM_REQUIRE(k && v, "NULL key/value");
  FM_REQUIRE(kv_len >= 0, "bad kv_len");
  CommonIn c{q, q_stride_batch, q_stride_token, q_stride_head, out, out_stride_batch,
             out_stride_token, out_stride_head, cu_seqlens_q, batch, max_seqlen_q,
             kv_len, num_q_heads, num_kv_heads, head_dim, softmax_scale,
             q_norm_weight, rope_cos, rope_sin, rope_row_stride, rope_pair_stride, rope_rows,
             q_positions, eps, plan, workspace, workspace_bytes, (hipStream_t)stream};
  AttnArgs a{};
  a.k = (const uint16_t *)k;
  a.v = (const uint16_t *)v;
  a.k_s0 = k_stride_batch, a.k_s1 = k_stride_head, a.k_s2 = k_stride_pos;
  a.v_s0 = v_stride_batch, a.v_s1 = v_stride_head, a.v_s2 = v_stride_pos;
  a.seqlens = seqlens_k;
  a.uniform_len = kv_len;
  return run_attention(c, CONTIG, a);
}

extern "C" int fm_block_attn_paged(
    const void *q, int64_t q_stride_batch, int64_t q_stride_token, int64_t q_stride_head, void *out,
    int64_t out_stride_batch, int64_t out_stride_token, int64_t out_stride_head,
    const int32_t *cu_seqlens_q, const void *kv_cache, int64_t num_blocks, int64_t stride_block,
    int64_t stride_head, int64_t stride_token, int64_t v_offset, int32_t page_size,
    const int32_t *block_table, int64_t block_table_stride, int64_t block_table_width,
    const int32_t *seqused_k, int32_t batch, int32_t max_seqlen_q, int32_t max_seqlen_k,
    int32_t num_q_heads, int32_t num_kv_heads, int32_t head_dim, float softmax_scale,
    const float *q_norm_weight, const float *rope_cos, const float *rope_sin,
    int64_t rope_row_stride, int64_t rope_pair_stride, int64_t rope_rows,
    const int64_t *q_positions, float eps, const int32_t *plan, void *workspace,
    size_t workspace_bytes, void *stream) {
  FM_REQUIRE(kv_cache && block_table && seqused_k, "NULL cache/block table/seqused_k");
  FM_REQUIRE(page_size > 0 && num_blocks > 0 && block_table_width > 0, "bad page geometry");
  FM_REQUIRE(v_offset % 8 == 0, "v_offset must be a multiple of 8 elements");
  const bool pow2 = (page_size & (page_size - 1)) == 0;
  const int layout = (pow2 && page_size % 16 == 0) ? PAGED16 : PAGED;
  CommonIn c{q, q_stride_batch, q_stride_token, q_stride_head, out, out_stride_batch,
             out_stride_token, out_stride_head, cu_seqlens_q, batch, max_seqlen_q, max_seqlen_k,
             num_q_heads, num_kv_heads, head_dim, softmax_scale, q_norm_weight, rope_cos,
             rope_sin, rope_row_stride, rope_pair_stride, rope_rows, q_positions, eps, plan,
             workspace, workspace_bytes, (hipStream_t)stream};
  AttnArgs a{};
  a.k = (const uint16_t *)kv_cache;
  a.v = (const uint16_t *)kv_cache + v_offset;
  a.k_s0 = stride_block, a.k_s1 = stride_head, a.k_s2 = stride_token;
  a.v_s0 = stride_block, a.v_s1 = stride_head, a.v_s2 = stride_token;
  a.table = block_table;
  a.table_stride = block_table_stride;
  a.table_width = block_table_width;
  a.num_pages = num_blocks;
  a.page_size = page_size;
  a.page_shift = pow2 ? __builtin_ctz((unsigned)page_size) : 0;
  a.seqlens = seqused_k;
  return run_attention(c, layout, a);
}

extern "C" int fm_block_attn_token_paged(
    const void *q, int64_t q_stride_batch, int64_t q_stride_token, int64_t q_stride_head, void *out,
    int64_t out_stride_batch, int64_t out_stride_token, int64_t out_stride_head,
    const int32_t *cu_seqlens_q, const void *key_buffer, const void *value_buffer,
    int64_t pool_size, int64_t k_stride_slot, int64_t k_stride_head, int64_t v_stride_slot,
    int64_t v_stride_head, const int32_t *page_table, int64_t page_table_stride,
    int64_t page_table_width, const int32_t *cache_seqlens, int32_t batch, int32_t max_seqlen_q,
    int32_t max_seqlen_k, int32_t num_q_heads, int32_t num_kv_heads, int32_t head_dim,
    float softmax_scale, const float *q_norm_weight, const float *rope_cos, const float *rope_sin,
    int64_t rope_row_stride, int64_t rope_pair_stride, int64_t rope_rows,
    const int64_t *q_positions, float eps, const int32_t *plan, void *workspace,
    size_t workspace_bytes, void *stream) {
  FM_REQUIRE(key_buffer && value_buffer && page_table && cache_seqlens, "NULL pool/page table/seqlens");
  FM_REQUIRE(pool_size > 0 && page_table_width > 0, "bad pool geometry");
  CommonIn c{q, q_stride_batch, q_stride_token, q_stride_head, out, out_stride_batch,
             out_stride_token, out_stride_head, cu_seqlens_q, batch, max_seqlen_q, max_seqlen_k,
             num_q_heads, num_kv_heads, head_dim, softmax_scale, q_norm_weight, rope_cos,
             rope_sin, rope_row_stride, rope_pair_stride, rope_rows, q_positions, eps, plan,
             workspace, workspace_bytes, (hipStream_t)stream};
  AttnArgs a{};
  a.k = (const uint16_t *)key_buffer;
  a.v = (const uint16_t *)value_buffer;
  a.k_s0 = k_stride_slot, a.k_s1 = k_stride_head, a.k_s2 = 0;
  a.v_s0 = v_stride_slot, a.v_s1 = v_stride_head, a.v_s2 = 0;
  a.table = page_table;
  a.table_stride = page_table_stride;
  a.table_width = page_table_width;
  a.num_pages = pool_size;
  a.page_size = 1;
  a.page_shift = 0;
  a.seqlens = cache_seqlens;
  return run_attention(c, PAGED, a);
}
