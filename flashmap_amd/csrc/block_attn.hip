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
// Workgroup = one wavefront per 16-row block of the unit (4 at GQA 4 x 16 rows). All
// wavefronts walk the share's tiles together: K/V tiles stream from HBM straight into
// an LDS ring of STAGES tiles with LDS-DMA (global_load_lds_dwordx4, no registers in
// flight), each wavefront issuing an equal part of every tile's 16-byte loads; tile i
// is consumed after a hand-counted s_waitcnt vmcnt and a barrier while tiles
// i+1 .. i+STAGES-1 are in flight. K lands in LDS already in MFMA operand order.
// Per tile, wavefront w (its 16 rows r):
//   S^T[pos][r] = K Q^T       v_mfma_f32_16x16x32_bf16, A = K from LDS, B = Q in registers
//   online softmax on S^T:    each lane owns one row (lane % 16): the running max, sum
//                             and rescale are lane-local; the max crosses 4 lane groups
//   O^T[d][r] += V^T P^T      B = P^T is the S^T accumulator rounded to bf16 as is;
//                             A = V^T is read transposed out of LDS (16-bit reads)
// so no wavefront exchanges data with another and each writes its own rows.
#include <math.h>

#include <mutex>

#include "fm_device.h"
#include "fm_host.h"

namespace fm {

constexpr int TILE = 32;    // context positions per tile
constexpr int NRB_MAX = 8;  // wavefronts (16-row blocks) per unit
constexpr int STAGES = 4;   // LDS ring depth (tiles)

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
  int32_t pos_cap;  // CONTIG: positions the K/V tensors hold (reads are clamped below it)
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

// LDS geometry of one tile stage (bytes). K is stored in MFMA fragment order: block
// (pb, t) of 1 KB holds, at lane*16, the 8 channels 32t+8g.. of row 16pb+n, i.e. what
// lane (n, g) feeds to the MFMA. V is stored by rows, RPB rows per 1 KB block, blocks
// padded by 32 bytes so the transposed 16-bit reads of the P.V operand hit 32 distinct
// banks.
template <int D>
struct Geo {
  static constexpr int KT = D / 32;            // k-steps over head_dim
  static constexpr int DB = D / 16;            // 16-channel blocks of O^T
  static constexpr int KFRAGS = 2 * KT;        // 1 KB K blocks per tile
  static constexpr int LPR = D / 8;            // 16-byte chunks per row
  static constexpr int RPB = 64 / LPR;         // V rows per 1 KB block
  static constexpr int VBLKS = TILE / RPB;     // V blocks per tile
  static constexpr int VPITCH = 1024 + 32;     // bytes per V block (with pad)
  static constexpr int NI = KFRAGS + VBLKS;    // 16-byte LDS-DMA loads per lane per tile
  static constexpr int KBYTES = KFRAGS * 1024;
  static constexpr int VBYTES = VBLKS * VPITCH;
  static constexpr int TBYTES = 128;           // page ids of the tile (generic paging)
  static constexpr int STAGE = KBYTES + VBYTES + TBYTES;
  static constexpr int SMEM = STAGES * STAGE;
};

__device__ __forceinline__ int64_t share_start(int64_t w, int64_t total, int64_t nw) {
  return w * total / nw;
}
__device__ __forceinline__ int64_t share_of(int64_t x, int64_t total, int64_t nw) {
  return ((x + 1) * nw - 1) / total;
}

// Read-only per-sequence metadata (uniform loads: scalar when the pointers are noalias).
struct Meta {
  const int32_t *__restrict__ plan;
  const int32_t *__restrict__ seqlens;
  const int32_t *__restrict__ table;
  const int32_t *__restrict__ cu_q;
};

// Scalar (SMEM) load of a wave-uniform int32 that no kernel of this call writes
// (plans, lengths, tables). Completion is awaited inside, on lgkmcnt, so it never
// joins the vmcnt-ordered stream of LDS-DMA loads whose waits are counted by hand.
__device__ __forceinline__ int32_t sload(const int32_t *p) {
  int32_t v;
  // Both halves of the address are zero-extended (readfirstlane returns a signed int).
  const uint64_t addr = reinterpret_cast<uint64_t>(p);
  const uint32_t lo = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)addr);
  const uint32_t hi = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)(addr >> 32));
  const int32_t *u = reinterpret_cast<const int32_t *>(((uint64_t)hi << 32) | (uint64_t)lo);
  asm volatile("s_load_dword %0, %1, 0x0\n\ts_waitcnt lgkmcnt(0)" : "=s"(v) : "s"(u));
  return v;
}

__device__ __forceinline__ int64_t tile_prefix(const AttnArgs &a, const Meta &m, int b) {
  return m.plan ? (int64_t)sload(m.plan + b) : (int64_t)b * a.uniform_tiles;
}
__device__ __forceinline__ int32_t seq_len(const AttnArgs &a, const Meta &m, int b) {
  if (m.seqlens == nullptr) return a.uniform_len;
  const int32_t L = sload(m.seqlens + b);
  return L > 0 ? L : 0;
}
__device__ __forceinline__ int32_t q_rows_of(const AttnArgs &a, const Meta &m, int b) {
  if (m.cu_q == nullptr) return a.q_len;
  const int32_t r = sload(m.cu_q + b + 1) - sload(m.cu_q + b);
  return r < a.q_len ? r : a.q_len;
}
__device__ __forceinline__ int64_t q_token_index(const AttnArgs &a, const Meta &m, int b, int t) {
  return m.cu_q ? (int64_t)sload(m.cu_q + b) + t : (int64_t)b * a.q_len + t;
}

// Position on the workgroup's line of tiles: sequence b, unit ul (= head * rgroups +
// row group), tile lt of the unit; tiles / L of sequence b.
struct Cursor {
  int b, ul, lt, tiles, L;
};

__device__ __forceinline__ void cursor_load(const AttnArgs &a, const Meta &m, Cursor &c) {
  c.tiles = (int)(tile_prefix(a, m, c.b + 1) - tile_prefix(a, m, c.b));
  c.L = seq_len(a, m, c.b);
}

__device__ __forceinline__ void cursor_next(const AttnArgs &a, const Meta &m, Cursor &c, int ups) {
  if (++c.lt < c.tiles) return;
  c.lt = 0;
  if (++c.ul < ups) return;
  c.ul = 0;
  do {
    ++c.b;
  } while (c.b < a.batch && tile_prefix(a, m, c.b + 1) == tile_prefix(a, m, c.b));
  if (c.b < a.batch) cursor_load(a, m, c);
}

__device__ __forceinline__ Cursor cursor_at(const AttnArgs &a, const Meta &m, int64_t t, int64_t ups) {
  int lo = 0, hi = a.batch;  // largest b with ups * prefix(b) <= t
  while (hi - lo > 1) {
    const int mid = (lo + hi) >> 1;
    if (ups * tile_prefix(a, m, mid) <= t)
      lo = mid;
    else
      hi = mid;
  }
  Cursor c;
  c.b = lo;
  cursor_load(a, m, c);
  const int64_t off = t - ups * tile_prefix(a, m, lo);
  c.ul = (int)(off / c.tiles);
  c.lt = (int)(off - (int64_t)c.ul * c.tiles);
  return c;
}

typedef __attribute__((address_space(3))) void *lds_ptr_t;

__device__ __forceinline__ void dma16(const void *g, void *l) {
  __builtin_amdgcn_global_load_lds(g, (lds_ptr_t)l, 16, 0, 0);
}

// s_waitcnt vmcnt(n) lgkmcnt(0): this wavefront's older LDS-DMA loads but the last n
// are complete, and its LDS reads are done (before a workgroup barrier).
__device__ __forceinline__ void wait_vm_lgkm0(int n) {
#define FM_W(N) \
  case N:       \
    __builtin_amdgcn_s_waitcnt(((N)&15) | (((N) >> 4) << 14) | (7 << 4)); \
    break;
  switch (n) {
    FM_W(0) FM_W(1) FM_W(2) FM_W(3) FM_W(4) FM_W(5) FM_W(6) FM_W(7) FM_W(8) FM_W(9)
    FM_W(10) FM_W(11) FM_W(12) FM_W(13) FM_W(14) FM_W(15) FM_W(16) FM_W(17) FM_W(18)
    FM_W(19) FM_W(20) FM_W(21) FM_W(22) FM_W(23) FM_W(24) FM_W(25) FM_W(26) FM_W(27)
    FM_W(28) FM_W(29) FM_W(30) FM_W(31) FM_W(32) FM_W(33) FM_W(34) FM_W(35) FM_W(36)
    FM_W(37) FM_W(38) FM_W(39) FM_W(40) FM_W(41) FM_W(42) FM_W(43) FM_W(44) FM_W(45)
    FM_W(46) FM_W(47)
    default:
      __builtin_amdgcn_s_waitcnt((7 << 4));  // vmcnt(0) lgkmcnt(0)
  }
#undef FM_W
}

__device__ __forceinline__ void block_sync() {
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
}

// Page id of a position for the 16-aligned paged layout (uniform: scalar loads).
__device__ __forceinline__ int64_t page_of(const AttnArgs &a, const Meta &m, int b, int pos) {
  int64_t col = pos >> a.page_shift;
  col = col < a.table_width ? col : a.table_width - 1;
  int64_t page = sload(m.table + (int64_t)b * a.table_stride + col);
  return page < 0 ? 0 : (page >= a.num_pages ? a.num_pages - 1 : page);
}

// Generic paging: DMA the page ids of the tile's 32 positions (clamped to the
// sequence) into the stage's table slot. Issued by wavefront 0 only (one instruction).
template <int D>
__device__ __forceinline__ void issue_table(const AttnArgs &a, const Meta &m, const Cursor &c,
                                            char *stage, int lane) {
  using G = Geo<D>;
  if (lane < 32) {
    int p = c.lt * TILE + lane;
    p = p < c.L ? p : c.L - 1;
    int64_t col = a.page_size == 1 ? p : p / a.page_size;
    col = col < a.table_width ? col : a.table_width - 1;
    __builtin_amdgcn_global_load_lds(m.table + (int64_t)c.b * a.table_stride + col,
                                     (lds_ptr_t)(stage + G::KBYTES + G::VBYTES), 4, 0, 0);
  }
}

// This wavefront's share of the K/V LDS-DMA loads of tile c into `stage`:
// load i = wave, wave + W, ... of the tile's NI loads (K blocks first, then V blocks).
template <int LAYOUT, int D, int W>
__device__ __forceinline__ void issue_kv(const AttnArgs &a, const Meta &m, const Cursor &c,
                                         char *stage, int wave, int lane) {
  using G = Geo<D>;
  const int n = lane & 15, g = lane >> 4;
  const int h = c.ul / a.rgroups;
  const int pos0 = c.lt * TILE;
  int last = c.L - 1 - pos0;  // last valid row of the tile
  last = last > 0 ? last : 0;  // (never negative, even for a plan that disagrees with L)
  int64_t page0 = 0, page1 = 0;
  if (LAYOUT == PAGED16) {
    page0 = page_of(a, m, c.b, pos0);
    page1 = page_of(a, m, c.b, pos0 + 16 <= c.L - 1 ? pos0 + 16 : c.L - 1);
  }
  const int32_t *tbl = reinterpret_cast<const int32_t *>(stage + G::KBYTES + G::VBYTES);
#pragma unroll
  for (int k = 0; k < (G::NI + W - 1) / W; ++k) {
    const int i = wave + k * W;
    if (i >= G::NI) break;
    const bool isk = i < G::KFRAGS;
    int row, coff;
    char *dst;
    if (isk) {
      const int pb = i / G::KT, t = i - (i / G::KT) * G::KT;
      row = 16 * pb + n;
      coff = 32 * t + 8 * g;
      dst = stage + i * 1024;
    } else {
      const int vb = i - G::KFRAGS;
      row = G::RPB * vb + lane / G::LPR;
      coff = 8 * (lane % G::LPR);
      dst = stage + G::KBYTES + vb * G::VPITCH;
    }
    row = row < last ? row : last;
    const int64_t s0 = isk ? a.k_s0 : a.v_s0, s1 = isk ? a.k_s1 : a.v_s1, s2 = isk ? a.k_s2 : a.v_s2;
    const uint16_t *base = isk ? a.k : a.v;
    int64_t off;
    if (LAYOUT == CONTIG) {
      const int p = pos0 + row < a.pos_cap ? pos0 + row : a.pos_cap - 1;
      off = (int64_t)c.b * s0 + (int64_t)h * s1 + (int64_t)p * s2;
    } else if (LAYOUT == PAGED16) {
      const int64_t page = row >= 16 ? page1 : page0;
      off = page * s0 + (int64_t)h * s1 + (int64_t)((pos0 + row) & (a.page_size - 1)) * s2;
    } else {
      int64_t page = tbl[row];
      page = page < 0 ? 0 : (page >= a.num_pages ? a.num_pages - 1 : page);
      const int p = pos0 + row;
      const int in_page = a.page_size == 1 ? 0 : p - (p / a.page_size) * a.page_size;
      off = page * s0 + (int64_t)h * s1 + (int64_t)in_page * s2;
    }
    dma16(base + off + coff, dst);
  }
}

// Query rows of this wavefront (row block `wave` of unit (b, h, rg)) as the MFMA B
// operand, with the fused QK-RMSNorm + RoPE when requested. Invalid rows are 0.
template <int D, int W>
__device__ __forceinline__ void load_queries(const AttnArgs &a, const Meta &m, u32x4_t (&qf)[D / 32],
                                             int b, int h, int rg, int wave, int lane) {
  constexpr int KT = D / 32;
  const int n = lane & 15, g = lane >> 4;
  const int R = (rg * W + wave) * 16 + n;
  const int gq = R / a.q_len, tq = R - gq * a.q_len;
  const bool valid = gq < a.group && tq < q_rows_of(a, m, b);
  const int64_t tok = q_token_index(a, m, b, valid ? tq : 0);
  const int64_t head = (int64_t)h * a.group + (valid ? gq : 0);
  const uint16_t *src = a.q + (m.cu_q ? tok * a.q_st : (int64_t)b * a.q_sb + (int64_t)tq * a.q_st) +
                        head * a.q_sh + 8 * g;
#pragma unroll
  for (int t = 0; t < KT; ++t) qf[t] = valid ? load16(src + 32 * t) : u32x4_t{0, 0, 0, 0};
  if (a.qn_w != nullptr) {
    const int64_t rr = clamp_row(a.rope, valid ? (a.q_pos ? a.q_pos[tok] : tok) : 0);
    norm_rope_row<D>(qf, a.qn_w, a.eps, a.rope, rr, g);
  }
  // Settle the query registers here, at the segment start: their loads are then no
  // longer pending anywhere in the tile loop, so the compiler does not drain the
  // LDS-DMA pipeline (vmcnt(0)) before each tile's first MFMA.
#pragma unroll
  for (int t = 0; t < KT; ++t) asm volatile("" : "+v"(qf[t]));
}

// One tile for this wavefront's 16 rows: S^T = K Q^T, online softmax, O^T += V^T P^T.
template <int D>
__device__ __forceinline__ void compute_tile(const AttnArgs &a, const char *stage,
                                             const u32x4_t (&qf)[D / 32], f32x4_t (&acc)[D / 16],
                                             float &m, float &l, int pos0, int L, int lane) {
  using G = Geo<D>;
  const int n = lane & 15, g = lane >> 4;
  f32x4_t s[2];
#pragma unroll
  for (int pb = 0; pb < 2; ++pb) {
    f32x4_t c = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int t = 0; t < G::KT; ++t) {
      const u32x4_t kf = *reinterpret_cast<const u32x4_t *>(stage + (pb * G::KT + t) * 1024 + lane * 16);
      c = mfma_16x16x32(kf, qf[t], c);
    }
    s[pb] = c;  // S^T[pos 16 pb + 4 g + i][row n]
  }
  if (pos0 + TILE > L) {
#pragma unroll
    for (int pb = 0; pb < 2; ++pb)
#pragma unroll
      for (int i = 0; i < 4; ++i)
        if (pos0 + 16 * pb + 4 * g + i >= L) s[pb][i] = -INFINITY;
  }
  float mx = fmaxf(fmaxf(fmaxf(s[0][0], s[0][1]), fmaxf(s[0][2], s[0][3])),
                   fmaxf(fmaxf(s[1][0], s[1][1]), fmaxf(s[1][2], s[1][3])));
  mx = max_over_groups(mx);
  const float mnew = fmaxf(m, mx * a.scale_log2);
  const float alpha = __builtin_amdgcn_exp2f(m - mnew);
  m = mnew;
  float p[2][4];
  float ps = 0.f;
#pragma unroll
  for (int pb = 0; pb < 2; ++pb)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      p[pb][i] = __builtin_amdgcn_exp2f(fmaf(s[pb][i], a.scale_log2, -mnew));
      ps += p[pb][i];
    }
  l = l * alpha + ps;
  const u32x4_t pk = {pack_bf16x2(p[0][0], p[0][1]), pack_bf16x2(p[0][2], p[0][3]),
                      pack_bf16x2(p[1][0], p[1][1]), pack_bf16x2(p[1][2], p[1][3])};
  // V^T operand: row d = 16 db + n, reduction positions pos(g, j) = 4g + j (j < 4) and
  // 16 + 4g + j - 4 (j >= 4), the positions of this lane's S^T values.
  const uint16_t *vs = reinterpret_cast<const uint16_t *>(stage + G::KBYTES);
  int vo[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const int pos = j < 4 ? 4 * g + j : 16 + 4 * g + (j - 4);
    vo[j] = (pos / G::RPB) * (G::VPITCH / 2) + (pos % G::RPB) * D + n;
  }
#pragma unroll
  for (int db = 0; db < G::DB; ++db) {
    const uint16_t *c0 = vs + 16 * db;
    u32x4_t vf;
    vf[0] = (uint32_t)c0[vo[0]] | ((uint32_t)c0[vo[1]] << 16);
    vf[1] = (uint32_t)c0[vo[2]] | ((uint32_t)c0[vo[3]] << 16);
    vf[2] = (uint32_t)c0[vo[4]] | ((uint32_t)c0[vo[5]] << 16);
    vf[3] = (uint32_t)c0[vo[6]] | ((uint32_t)c0[vo[7]] << 16);
    acc[db] = mfma_16x16x32(vf, pk, acc[db] * alpha);
  }
}

template <int LAYOUT, int W, int D>
__global__ __launch_bounds__(64 * W) void attn_fwd_kernel(
    const AttnArgs a, const int32_t *__restrict__ plan, const int32_t *__restrict__ seqlens,
    const int32_t *__restrict__ table, const int32_t *__restrict__ cu_q) {
  using G = Geo<D>;
  __shared__ __attribute__((aligned(1024))) char smem[G::SMEM];
  const Meta mt{plan, seqlens, table, cu_q};
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int n = lane & 15, g = lane >> 4;
  const int ups = a.hkv * a.rgroups;
  const int64_t total = (int64_t)ups * tile_prefix(a, mt, a.batch);
  const int64_t T0 = share_start(blockIdx.x, total, a.num_wg);
  const int64_t T1 = share_start((int64_t)blockIdx.x + 1, total, a.num_wg);
  if (T0 >= T1) return;
  const int ntiles = (int)(T1 - T0);
  // Loads this wavefront issues per tile, and per tile for wavefront 0's page ids.
  const int ipw = (G::NI - wave + W - 1) / W;
  constexpr bool TBL = LAYOUT == PAGED;

  Cursor cc = cursor_at(a, mt, T0, ups);  // tile being computed (i)
  Cursor ci = cc;                         // tile being loaded (i + STAGES - 1)
  Cursor ct = cc;                         // tile whose page ids are loaded (i + STAGES)
  if (TBL) {
    for (int j = 0; j < STAGES && j < ntiles; ++j) {
      if (wave == 0) issue_table<D>(a, mt, ct, smem + j * G::STAGE, lane);
      if (j + 1 < ntiles) cursor_next(a, mt, ct, ups);
    }
    wait_vm_lgkm0(0);
    block_sync();
  }
  for (int j = 0; j < STAGES - 1 && j < ntiles; ++j) {
    issue_kv<LAYOUT, D, W>(a, mt, ci, smem + j * G::STAGE, wave, lane);
    if (j + 1 < ntiles) cursor_next(a, mt, ci, ups);
  }

  u32x4_t qf[D / 32];
  f32x4_t acc[D / 16];
  float m = -INFINITY, l = 0.f;
  int seg = 0, lt_first = 0;
  for (int i = 0; i < ntiles; ++i) {
    // Tile i is complete once every later load of this wavefront is allowed to be
    // outstanding: the K/V loads of tiles i+1 .. i+STAGES-2 (and, on wavefront 0,
    // the page-id loads issued after tile i's).
    {
      const int later = min(STAGES - 2, ntiles - 1 - i);
      int nwait = ipw * (later > 0 ? later : 0);
      if (TBL && wave == 0) {
        const int lo = max(i + 2, STAGES), hi = min(i + STAGES - 1, ntiles - 1);
        nwait += hi >= lo ? hi - lo + 1 : 0;
        // page ids of tile i + STAGES - 1 (issued last iteration, before its K/V loads)
        if (i >= 1 && i + STAGES - 1 < ntiles) nwait = min(nwait, i + STAGES - 2 < ntiles ? ipw : 0);
      }
      wait_vm_lgkm0(nwait);
    }
    block_sync();
    if (TBL && i + STAGES < ntiles) {
      if (wave == 0) issue_table<D>(a, mt, ct, smem + ((i + STAGES) % STAGES) * G::STAGE, lane);
      cursor_next(a, mt, ct, ups);
    }
    if (i + STAGES - 1 < ntiles) {
      issue_kv<LAYOUT, D, W>(a, mt, ci, smem + ((i + STAGES - 1) % STAGES) * G::STAGE, wave, lane);
      if (i + STAGES < ntiles) cursor_next(a, mt, ci, ups);
    }

    const int h = cc.ul / a.rgroups, rg = cc.ul - h * a.rgroups;
    if (i == 0 || cc.lt == 0) {  // a unit (segment) starts
      load_queries<D, W>(a, mt, qf, cc.b, h, rg, wave, lane);
#pragma unroll
      for (int db = 0; db < D / 16; ++db) acc[db] = f32x4_t{0.f, 0.f, 0.f, 0.f};
      m = -INFINITY;
      l = 0.f;
      lt_first = cc.lt;
    }
    compute_tile<D>(a, smem + (i % STAGES) * G::STAGE, qf, acc, m, l, cc.lt * TILE, cc.L, lane);

    if (cc.lt == cc.tiles - 1 || i == ntiles - 1) {  // the segment ends: write it out
      const float lt_sum = sum_over_groups(l);
      const float inv = lt_sum > 0.f ? 1.f / lt_sum : 0.f;
      const bool whole = lt_first == 0 && cc.lt == cc.tiles - 1;
      const int R = (rg * W + wave) * 16 + n;
      const int gq = R / a.q_len, tq = R - gq * a.q_len;
      if (gq < a.group && tq < q_rows_of(a, mt, cc.b)) {
        if (whole) {
          const int64_t head = (int64_t)h * a.group + gq;
          uint16_t *dst = a.o +
                          (cu_q ? q_token_index(a, mt, cc.b, tq) * a.o_st
                                : (int64_t)cc.b * a.o_sb + (int64_t)tq * a.o_st) +
                          head * a.o_sh + 4 * g;
#pragma unroll
          for (int db = 0; db < D / 16; ++db) {
            const f32x4_t v = acc[db] * inv;
            *reinterpret_cast<u32x2_t *>(dst + 16 * db) =
                u32x2_t{pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3])};
          }
        } else {
          const int64_t slot = 2 * (int64_t)blockIdx.x + (seg == 0 ? 0 : 1);
          const int64_t prow = slot * (16 * W) + wave * 16 + n;
          float *dst = a.part_o + prow * D + 4 * g;
#pragma unroll
          for (int db = 0; db < D / 16; ++db) *reinterpret_cast<f32x4_t *>(dst + 16 * db) = acc[db] * inv;
          if (g == 0) a.part_lse[prow] = m + log2f(lt_sum);
        }
      }
      ++seg;
    }
    if (i + 1 < ntiles) cursor_next(a, mt, cc, ups);
  }
}

// Merge the partials of units cut between workgroups; zero-fill empty sequences.
template <int D>
__global__ __launch_bounds__(256) void attn_combine_kernel(const AttnArgs a, int nrb) {
  const Meta mt{a.plan, a.seqlens, a.table, a.cu_q};
  const int rows = nrb * 16;
  const int64_t ups = (int64_t)a.hkv * a.rgroups;
  const int64_t unit = blockIdx.x;
  const int b = (int)(unit / ups);
  const int ul = (int)(unit - (int64_t)b * ups);
  const int h = ul / a.rgroups, rg = ul - h * a.rgroups;
  const int64_t pre = tile_prefix(a, mt, b);
  const int tiles_b = (int)(tile_prefix(a, mt, b + 1) - pre);
  const int qlen_b = q_rows_of(a, mt, b);
  const int64_t total = ups * tile_prefix(a, mt, a.batch);
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
                    (a.cu_q ? q_token_index(a, mt, b, tq) * a.o_st
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

typedef void (*AttnKernel)(const AttnArgs, const int32_t *, const int32_t *, const int32_t *,
                           const int32_t *);

template <int LAYOUT, int D>
static AttnKernel pick_kernel(int w) {
  switch (w) {
    case 1: return attn_fwd_kernel<LAYOUT, 1, D>;
    case 2: return attn_fwd_kernel<LAYOUT, 2, D>;
    case 3: return attn_fwd_kernel<LAYOUT, 3, D>;
    case 4: return attn_fwd_kernel<LAYOUT, 4, D>;
    case 5: return attn_fwd_kernel<LAYOUT, 5, D>;
    case 6: return attn_fwd_kernel<LAYOUT, 6, D>;
    case 7: return attn_fwd_kernel<LAYOUT, 7, D>;
    default: return attn_fwd_kernel<LAYOUT, 8, D>;
  }
}

static AttnKernel select_kernel(int layout, int d, int w) {
  if (d == 128) {
    if (layout == CONTIG) return pick_kernel<CONTIG, 128>(w);
    if (layout == PAGED16) return pick_kernel<PAGED16, 128>(w);
    return pick_kernel<PAGED, 128>(w);
  }
  if (layout == CONTIG) return pick_kernel<CONTIG, 64>(w);
  if (layout == PAGED16) return pick_kernel<PAGED16, 64>(w);
  return pick_kernel<PAGED, 64>(w);
}

struct RowPlan {
  int nrb;      // 16-row blocks per unit
  int rgroups;  // units per KV head
};

// Row blocks per unit (= wavefronts per workgroup) and row groups per KV head.
static RowPlan row_plan(int group, int q_len) {
  const int total = (group * q_len + 15) / 16;
  RowPlan p;
  p.rgroups = (total + NRB_MAX - 1) / NRB_MAX;
  p.nrb = (total + p.rgroups - 1) / p.rgroups;
  return p;
}

static int env_int(const char *name, int dflt) {
  const char *v = getenv(name);
  if (v == nullptr || *v == 0) return dflt;
  return atoi(v);
}

// Workgroups resident per CU for a kernel (cached).
static int occupancy(AttnKernel k, int block) {
  static std::mutex mu;
  static std::vector<std::pair<AttnKernel, int>> cache;
  std::lock_guard<std::mutex> lock(mu);
  for (auto &e : cache)
    if (e.first == k) return e.second;
  int blocks = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&blocks, reinterpret_cast<const void *>(k), block,
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
  int64_t nw = (int64_t)info.cus * occupancy(k, 64 * sz->rp.nrb);
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
  const int32_t *kplan = a.plan, *kseq = a.seqlens, *ktab = a.table, *kcu = a.cu_q;
  void *kargs[] = {&a, &kplan, &kseq, &ktab, &kcu};
  profile_before(c.stream);
  const hipError_t lerr = hipLaunchKernel(reinterpret_cast<const void *>(k), dim3(sz.num_wg),
                                          dim3(64 * sz.rp.nrb), kargs, 0, c.stream);
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
  // An empty cache: every sequence attends to nothing (zeros), whatever seqlens_k says.
  a.seqlens = kv_len > 0 ? seqlens_k : nullptr;
  a.uniform_len = kv_len;
  a.pos_cap = kv_len;
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
