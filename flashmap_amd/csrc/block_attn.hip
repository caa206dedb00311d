// a5/a6/a7: block attention of the K draft slots onto the context keys/values, for
// contiguous (FlashMapCache), block-paged (vLLM) and token-paged (SGLang) KV.
//
// Work decomposition (split-KV, "stream-K" style). A unit is (sequence b, KV head h,
// row group rg): the G query heads sharing KV head h times the q_len draft rows,
// packed into 16-row MFMA blocks (row r = query head h*G + r / q_len at token
// r % q_len, the GQA row convention of flashmap/sglang/verify_attention.py:77-79).
// Each unit's context is cut into tiles of 32 positions; all units' tiles form one
// line (sequence-major, then head, then row group) that is cut into num_shares equal
// shares, R per workgroup of the persistent grid (see replicas()). A share is walked
// unit by unit, one "segment" per unit it touches, leaving for every segment one fp32
// partial (O normalized by its own softmax sum, and the log-sum-exp) in slot
// unit + share, which is unique along the line. attn_combine_kernel merges each
// unit's partials (the LSE merge of flashmap/sglang/verify_attention.py:184-233) and
// writes the bf16 output.
//
// Three launches per call:
//   pack_queries_kernel  the query rows of every unit, in the order the MFMA blocks
//                        consume them, with the optional QK-RMSNorm + RoPE prologue
//                        applied (invalid rows are zero): the streaming kernel then
//                        addresses a unit's queries as one contiguous block and can
//                        prefetch them ahead of the unit
//   attn_fwd_kernel      the K/V stream and the online softmax
//   attn_combine_kernel  the merge and the scatter into the caller's output layout
//
// Workgroup = one wavefront per 16-row block of the unit (4 at GQA 4 x 16 rows). All
// wavefronts walk the share's tiles together: K/V tiles stream from HBM straight into
// an LDS ring of STAGES tiles with LDS-DMA (global_load_lds_dwordx4, no registers in
// flight), each wavefront issuing an equal part of every tile's 16-byte loads; tile i
// is consumed after a hand-counted s_waitcnt vmcnt and a barrier while tiles
// i+1 .. i+STAGES-1 are in flight. K lands in LDS already in MFMA operand order. The
// query rows of the next unit are loaded with the first tile of that unit, so a unit
// change costs no pipeline drain.
// Per tile, wavefront w (its 16 rows r):
//   S^T[pos][r] = K Q^T       v_mfma_f32_16x16x32_bf16, A = K from LDS, B = Q in registers
//   online softmax on S^T:    each lane owns one row (lane % 16): the running max, sum
//                             and rescale are lane-local; the max crosses 4 lane groups
//   O^T[d][r] += V^T P^T      B = P^T is the S^T accumulator rounded to bf16 as is;
//                             A = V^T is read transposed out of LDS (16-bit reads)
// so no wavefront exchanges data with another and each writes its own rows.
#include <math.h>
#include <stddef.h>

#include <mutex>
#include <type_traits>

#include "fm_device.h"
#include "fm_host.h"

namespace fm {

constexpr int TILE = 32;    // context positions per tile
constexpr int NRB_MAX = 8;  // wavefronts (16-row blocks) per unit
constexpr int STAGES = 3;   // LDS ring depth (tiles)

// Replicas per workgroup: R independent groups of W wavefronts, each streaming its own
// share through its own LDS ring, that meet at one barrier per tile. One workgroup per
// CU (at head_dim 128) then keeps every resident wavefront in lockstep: co-resident
// workgroups would instead be served oldest-first, and with equal static shares the
// youngest would finish last, leaving a tail with a fraction of the loads in flight.
__host__ __device__ constexpr int replicas(int w) { return w <= 6 ? 2 : 1; }

enum Layout { CONTIG = 0, PAGED16 = 1, PAGED = 2 };

// K/V geometry of a unit, read by the streaming kernel in one scalar load whenever its
// K/V stream enters a new unit.
struct UnitArgs {
  const uint16_t *k;
  const uint16_t *v;
  int64_t k_s0, k_s1;  // CONTIG: batch, head; paged: page (slot), head (elements)
  int64_t v_s0, v_s1;
  int64_t table_stride;
  int32_t pos_cap;  // CONTIG: positions the K/V tensors hold (reads are clamped below it)
  int32_t pad;
};
static_assert(sizeof(UnitArgs) == 64, "one s_load_dwordx16");

struct AttnArgs {
  UnitArgs u;  // first: at offset 0 of every kernel's argument segment
  // Per-tile address arithmetic in 32 bits (byte strides; the host checks they fit).
  uint32_t k_tok_b, v_tok_b;    // position / token stride
  uint32_t k_page_b, v_page_b;  // paged: page (slot) stride
  uint32_t page_mask;           // page_size - 1 (power-of-two pages)
  uint32_t col_last, page_last; // table_width - 1, num_pages - 1
  int32_t page_size, page_shift;
  int64_t k_s2, v_s2;           // position strides (elements)
  int64_t table_width, num_pages;
  const int32_t *table;
  const int32_t *plan;     // tile prefix over sequences (NULL with seqlens == NULL)
  const int32_t *seqlens;  // NULL: every sequence has uniform_len positions
  int32_t uniform_len, uniform_tiles;
  int32_t batch, hkv, rgroups, ups;  // ups = hkv * rgroups units per sequence
  int32_t nrb;                       // 16-row blocks (wavefronts) per unit
  int32_t num_shares;  // workgroups x replicas
  float scale_log2;
  const uint16_t *qp;  // packed queries: (units, 16 nrb rows, D) bf16, invalid rows 0
  float *part_o;       // partials: (units + num_shares, 16 nrb, D) fp32
  float *part_lse;     // (units + num_shares, 16 nrb), log2 domain (right after part_o)
  // Query / output side (pack and combine kernels only).
  const uint16_t *q;
  int64_t q_sb, q_st, q_sh;
  uint16_t *o;
  int64_t o_sb, o_st, o_sh;
  const int32_t *cu_q;
  int32_t q_len;  // rows per query head (max_seqlen_q)
  int32_t group;
  const float *qn_w;  // non-NULL: QK-RMSNorm + RoPE prologue on the queries
  Rope rope;
  const int64_t *q_pos;
  float eps;
};

// LDS geometry of one tile stage (bytes). K is stored in MFMA fragment order: block
// (pb, t) of 1 KB holds, at lane*16, the 8 channels 32t+8g.. of row 16pb+n, i.e. what
// lane (n, g) feeds to the MFMA. V is stored by rows, RPB rows per 1 KB block (slot k
// of block v holds row 4*RPB*(v/4) + 4k + v%4), blocks padded by 32 bytes: the four
// consecutive rows one ds_read_b64_tr_b16 of the P.V operand touches then sit in four
// blocks on disjoint banks. The stage ends with the tile's 32 page ids (paged layouts).
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
  static constexpr int QW = KT * 1024;  // one wavefront's 16 query rows, MFMA operand order
};

__device__ __forceinline__ int64_t share_start(int64_t w, int64_t total, int64_t nw) {
  return w * total / nw;
}
__device__ __forceinline__ int64_t share_of(int64_t x, int64_t total, int64_t nw) {
  return ((x + 1) * nw - 1) / total;
}

// The unit block of the arguments, re-read from offset 0 of the kernel argument segment
// in one scalar load (volatile, so the compiler keeps none of it in SGPRs across the
// tile loop).
__device__ __forceinline__ UnitArgs load_unit_args() {
  typedef __attribute__((ext_vector_type(16))) uint32_t u32x16_t;
  const uint64_t base = (uint64_t)__builtin_amdgcn_kernarg_segment_ptr();
  u32x16_t v;
  asm volatile("s_load_dwordx16 %0, %1, 0x0\n\ts_waitcnt lgkmcnt(0)" : "=s"(v) : "s"(base));
  return __builtin_bit_cast(UnitArgs, v);
}

// The partial-output pointers (part_o, part_lse: adjacent fields), re-read the same way
// when a segment ends.
typedef __attribute__((address_space(1))) float gfloat;  // global memory (global_* stores)
struct PartPtrs {
  gfloat *o;
  gfloat *lse;
};
__device__ __forceinline__ PartPtrs load_part_ptrs() {
  typedef __attribute__((ext_vector_type(4))) uint32_t u32x4v_t;
  const uint64_t base = (uint64_t)__builtin_amdgcn_kernarg_segment_ptr();
  u32x4v_t v;
  asm volatile("s_load_dwordx4 %0, %1, %2\n\ts_waitcnt lgkmcnt(0)"
               : "=s"(v)
               : "s"(base), "i"((int)offsetof(AttnArgs, part_o)));
  return __builtin_bit_cast(PartPtrs, v);
}

// Scalar (SMEM) loads of wave-uniform metadata that no kernel of this call writes
// (plans, lengths). Completion is awaited inside, on lgkmcnt, so the values never
// join the vmcnt-ordered stream of LDS-DMA loads whose waits are counted by hand.
__device__ __forceinline__ const int32_t *uniform_ptr(const int32_t *p) {
  // Both halves zero-extended (readfirstlane returns a signed int).
  const uint64_t addr = reinterpret_cast<uint64_t>(p);
  const uint32_t lo = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)addr);
  const uint32_t hi = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)(addr >> 32));
  return reinterpret_cast<const int32_t *>(((uint64_t)hi << 32) | (uint64_t)lo);
}
__device__ __forceinline__ int32_t sload(const int32_t *p) {
  int32_t v;
  asm volatile("s_load_dword %0, %1, 0x0\n\ts_waitcnt lgkmcnt(0)" : "=s"(v) : "s"(uniform_ptr(p)));
  return v;
}
// p[0], p[1] and q[0] in one round trip.
__device__ __forceinline__ void sload3(const int32_t *p, const int32_t *q, int32_t &p0, int32_t &p1,
                                       int32_t &q0) {
  typedef __attribute__((ext_vector_type(2))) int32_t i32x2_t;
  i32x2_t v;
  // Early-clobber outputs: a destination must not share SGPRs with the second load's
  // address, which the first load's data could overwrite before the second issues.
  asm volatile("s_load_dwordx2 %0, %2, 0x0\n\ts_load_dword %1, %3, 0x0\n\ts_waitcnt lgkmcnt(0)"
               : "=&s"(v), "=&s"(q0)
               : "s"(uniform_ptr(p)), "s"(uniform_ptr(q)));
  p0 = v[0];
  p1 = v[1];
}

// Per-sequence metadata (host-side helpers of the pack and combine kernels use plain
// loads; the streaming kernel goes through SeqMeta).
__device__ __forceinline__ int64_t tile_prefix(const AttnArgs &a, const int32_t *__restrict__ plan, int b) {
  return plan ? (int64_t)plan[b] : (int64_t)b * a.uniform_tiles;
}
__device__ __forceinline__ int32_t q_rows_of(const AttnArgs &a, int b) {
  if (a.cu_q == nullptr) return a.q_len;
  const int32_t r = a.cu_q[b + 1] - a.cu_q[b];
  return r < a.q_len ? r : a.q_len;
}
__device__ __forceinline__ int64_t q_token_index(const AttnArgs &a, int b, int t) {
  return a.cu_q ? (int64_t)a.cu_q[b] + t : (int64_t)b * a.q_len + t;
}

// Position on the workgroup's line of tiles: sequence b, KV head h, row group rg and
// tile lt of unit u = b * ups + h * rgroups + rg; tiles / L of sequence b. Advanced
// one tile at a time with compares only (no divisions on the per-tile path).
struct Cursor {
  int b, h, rg, lt, tiles, L, u;
};

// Plan and lengths of the streaming kernel; VAR: known to be per-sequence (the paged
// layouts always are), so the uniform-length fields are never read.
template <bool VAR>
struct SeqMeta {
  const int32_t *plan;
  const int32_t *seqlens;
  __device__ __forceinline__ bool var() const { return VAR || plan != nullptr; }
  __device__ __forceinline__ int64_t prefix(const AttnArgs &a, int b) const {
    return var() ? (int64_t)sload(plan + b) : (int64_t)b * a.uniform_tiles;
  }
  // tiles(b) = prefix(b + 1) - prefix(b) and the length of sequence b, one round trip.
  __device__ __forceinline__ void seq(const AttnArgs &a, int b, int &tiles, int &L) const {
    if (!var()) {
      tiles = a.uniform_tiles;
      L = a.uniform_len;
      return;
    }
    int32_t p0, p1, len;
    sload3(plan + b, seqlens + b, p0, p1, len);
    tiles = p1 - p0;
    L = len > 0 ? len : 0;
  }
};

template <bool VAR>
__device__ __forceinline__ void cursor_load(const AttnArgs &a, const SeqMeta<VAR> &sm, Cursor &c) {
  sm.seq(a, c.b, c.tiles, c.L);
}

// Advance one tile; true when the next tile starts a new unit.
template <bool VAR>
__device__ __forceinline__ bool cursor_next(const AttnArgs &a, const SeqMeta<VAR> &sm, Cursor &c) {
  if (++c.lt < c.tiles) return false;
  c.lt = 0;
  ++c.u;
  if (++c.rg < a.rgroups) return true;
  c.rg = 0;
  if (++c.h < a.hkv) return true;
  c.h = 0;
  // The next sequence with tiles (empty ones have no units).
  for (++c.b; c.b < a.batch; ++c.b) {
    cursor_load(a, sm, c);
    if (c.tiles > 0) break;
  }
  c.u = c.b * a.ups;
  return true;
}

template <bool VAR>
__device__ __forceinline__ Cursor cursor_at(const AttnArgs &a, const SeqMeta<VAR> &sm, int64_t t) {
  int lo = 0, hi = a.batch;  // largest b with ups * prefix(b) <= t
  while (hi - lo > 1) {
    const int mid = (lo + hi) >> 1;
    if ((int64_t)a.ups * sm.prefix(a, mid) <= t)
      lo = mid;
    else
      hi = mid;
  }
  Cursor c;
  c.b = lo;
  cursor_load(a, sm, c);
  const int64_t off = t - (int64_t)a.ups * sm.prefix(a, lo);
  const int ul = (int)(off / c.tiles);
  c.lt = (int)(off - (int64_t)ul * c.tiles);
  c.h = ul / a.rgroups;
  c.rg = ul - c.h * a.rgroups;
  c.u = lo * a.ups + ul;
  return c;
}

typedef __attribute__((address_space(3))) void *lds_ptr_t;

__device__ __forceinline__ void dma16(const void *g, void *l) {
  __builtin_amdgcn_global_load_lds(g, (lds_ptr_t)l, 16, 0, 0);
}

// s_waitcnt vmcnt(N) lgkmcnt(0): this wavefront's vector memory loads but the last N
// are complete, and its LDS reads and scalar loads are done.
template <int N>
__device__ __forceinline__ void wait_vm_lgkm0() {
  static_assert(N >= 0 && N < 64, "vmcnt holds 6 bits");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4));
}

// s_waitcnt lgkmcnt(0) alone: LDS reads (and scalar loads) done, vector loads untouched.
__device__ __forceinline__ void wait_lgkm0() {
  __builtin_amdgcn_s_waitcnt(0xF | (3 << 14) | (7 << 4));  // vmcnt 63, expcnt 7, lgkmcnt 0
}

// The same with a run-time count (generic paging only, where wavefront 0 also has
// page-id loads in flight).
__device__ __forceinline__ void wait_vm_lgkm0(int n) {
#define FM_W(N) \
  case N:       \
    wait_vm_lgkm0<N>(); \
    break;
  switch (n) {
    FM_W(0) FM_W(1) FM_W(2) FM_W(3) FM_W(4) FM_W(5) FM_W(6) FM_W(7) FM_W(8) FM_W(9)
    FM_W(10) FM_W(11) FM_W(12) FM_W(13) FM_W(14) FM_W(15) FM_W(16) FM_W(17) FM_W(18)
    FM_W(19) FM_W(20) FM_W(21) FM_W(22) FM_W(23) FM_W(24) FM_W(25) FM_W(26) FM_W(27)
    FM_W(28) FM_W(29) FM_W(30) FM_W(31) FM_W(32) FM_W(33) FM_W(34) FM_W(35) FM_W(36)
    FM_W(37) FM_W(38) FM_W(39) FM_W(40) FM_W(41) FM_W(42) FM_W(43) FM_W(44) FM_W(45)
    FM_W(46) FM_W(47) FM_W(48) FM_W(49) FM_W(50) FM_W(51) FM_W(52) FM_W(53) FM_W(54)
    FM_W(55) FM_W(56) FM_W(57) FM_W(58) FM_W(59) FM_W(60) FM_W(61) FM_W(62)
    default:
      wait_vm_lgkm0<0>();
  }
#undef FM_W
}

// Wait for tile i's load group when `later` (= tiles after i in the share, at most
// K = STAGES - 2 of them in flight) groups of IPW K/V loads may remain outstanding,
// `e` of which also carry NQ query-row loads. Constant counts in the steady state.
template <int IPW, int NQ, int K, int E>
__device__ __forceinline__ void wait_groups_e(int e) {
  if constexpr (E <= 0) {
    wait_vm_lgkm0<IPW * K>();
  } else {
    if (e >= E)
      wait_vm_lgkm0<IPW * K + NQ * E>();
    else
      wait_groups_e<IPW, NQ, K, E - 1>(e);
  }
}
template <int IPW, int NQ, int K>
__device__ __forceinline__ void wait_groups(int later, int e) {
  if constexpr (K <= 0) {
    wait_vm_lgkm0<0>();
  } else {
    if (later >= K)
      wait_groups_e<IPW, NQ, K, K>(e);
    else
      wait_groups<IPW, NQ, K - 1>(later, e);
  }
}

__device__ __forceinline__ void block_sync() {
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
}

// Generic paging (page size not a multiple of 16, e.g. SGLang's token pool): DMA the
// page ids of the tile's 32 positions (clamped to the sequence) into the stage's table
// slot, one dword per lane, issued by wavefront 0 a tile ahead of the K/V loads.
template <int D>
__device__ __forceinline__ void issue_table(const AttnArgs &a, const int32_t *__restrict__ table,
                                            const Cursor &c, char *stage, int lane) {
  using G = Geo<D>;
  if (lane < 32) {
    int p = c.lt * TILE + lane;
    p = p < c.L ? p : c.L - 1;
    p = p > 0 ? p : 0;
    int64_t col = a.page_size == 1 ? p : p / a.page_size;
    col = col < a.table_width ? col : a.table_width - 1;
    __builtin_amdgcn_global_load_lds(table + (int64_t)c.b * a.u.table_stride + col,
                                     (lds_ptr_t)(stage + G::KBYTES + G::VBYTES), 4, 0, 0);
  }
}

// Scalar state of the K/V stream: the next tile to load, the K/V bases of its unit
// (CONTIG: sequence b, head h at position 0; paged: head h of page 0), the block-table
// row of its sequence and, for 16-aligned pages, the pages of its two 16-position halves
// (plain uniform loads, so scalar, issued a tile before use and clamped into the pool).
struct Loader {
  Cursor c;
  int lim;  // positions of the unit that may be read unclamped (CONTIG: below pos_cap too)
  int cap;  // CONTIG: positions the K/V tensors hold
  const char *kb, *vb;
  const int32_t *trow;
  uint32_t p0, p1;
};

template <int LAYOUT>
__device__ __forceinline__ void loader_unit(const int32_t *__restrict__ table, Loader &ld) {
  const UnitArgs ua = load_unit_args();
  const int64_t h = ld.c.h;
  if (LAYOUT == CONTIG) {
    ld.cap = ua.pos_cap;
    ld.lim = ld.c.L < ua.pos_cap ? ld.c.L : ua.pos_cap;
    ld.kb = reinterpret_cast<const char *>(ua.k + (int64_t)ld.c.b * ua.k_s0 + h * ua.k_s1);
    ld.vb = reinterpret_cast<const char *>(ua.v + (int64_t)ld.c.b * ua.v_s0 + h * ua.v_s1);
  } else {
    ld.lim = ld.c.L;
    ld.kb = reinterpret_cast<const char *>(ua.k + h * ua.k_s1);
    ld.vb = reinterpret_cast<const char *>(ua.v + h * ua.v_s1);
    ld.trow = table + (int64_t)ld.c.b * ua.table_stride;
  }
}

template <int LAYOUT>
__device__ __forceinline__ void loader_pages(const AttnArgs &a, Loader &ld) {
  if (LAYOUT != PAGED16) return;
  const int pos0 = ld.c.lt * TILE;
  const int last = ld.c.L - 1 > 0 ? ld.c.L - 1 : 0;
  const uint32_t pa = (uint32_t)(pos0 < last ? pos0 : last);
  const uint32_t pb = (uint32_t)(pos0 + 16 < last ? pos0 + 16 : last);
  const uint32_t ca = min(pa >> a.page_shift, a.col_last), cb = min(pb >> a.page_shift, a.col_last);
  // The block table is read-only during the call: read through the constant address
  // space, the loads are scalar and their wait is left to the first use (next tile).
  typedef const __attribute__((address_space(4))) int32_t cint32_t;
  cint32_t *row = (cint32_t *)ld.trow;
  ld.p0 = (uint32_t)row[ca];  // clamped where used (next tile)
  ld.p1 = (uint32_t)row[cb];
}

template <int LAYOUT>
__device__ __forceinline__ void loader_advance(const AttnArgs &a, const SeqMeta<LAYOUT != CONTIG> &sm,
                                               const int32_t *__restrict__ table, Loader &ld) {
  if (cursor_next(a, sm, ld.c)) loader_unit<LAYOUT>(table, ld);
  loader_pages<LAYOUT>(a, ld);
}

// Row (within the tile) and channel offset of this lane's k-th load of a tile, and
// whether it is a K load. Load i = wave + k*W of the NI loads (K blocks, then V blocks).
template <int D>
__device__ __forceinline__ void load_slot(int i, int lane, int &row, int &coff, bool &isk, int &dst) {
  using G = Geo<D>;
  const int n = lane & 15, g = lane >> 4;
  isk = i < G::KFRAGS;
  if (isk) {
    const int pb = i / G::KT, t = i - (i / G::KT) * G::KT;
    row = 16 * pb + n;
    coff = 32 * t + 8 * g;
    dst = i * 1024;
  } else {
    const int vb = i - G::KFRAGS;
    row = 4 * G::RPB * (vb / 4) + 4 * (lane / G::LPR) + (vb % 4);
    coff = 8 * (lane % G::LPR);
    dst = G::KBYTES + vb * G::VPITCH;
  }
}

template <int LAYOUT, int D, int W>
__device__ __forceinline__ void issue_kv(const AttnArgs &a, const Loader &ld, char *stage, int wave,
                                         int lane, const uint32_t (&loff)[(Geo<D>::NI + W - 1) / W]) {
  using G = Geo<D>;
  constexpr int KPW = (G::NI + W - 1) / W;
  const int pos0 = ld.c.lt * TILE;
  if (LAYOUT != PAGED && pos0 + TILE <= ld.lim) {
    const char *kh[2], *vh[2];  // first rows of the two halves
    if (LAYOUT == CONTIG) {
      kh[0] = ld.kb + (uint64_t)(uint32_t)pos0 * a.k_tok_b;
      vh[0] = ld.vb + (uint64_t)(uint32_t)pos0 * a.v_tok_b;
      kh[1] = kh[0] + 16 * a.k_tok_b;
      vh[1] = vh[0] + 16 * a.v_tok_b;
    } else {
      const uint32_t in0 = (uint32_t)pos0 & a.page_mask, in1 = (uint32_t)(pos0 + 16) & a.page_mask;
      const uint32_t p0 = min(ld.p0, a.page_last), p1 = min(ld.p1, a.page_last);  // negative ids wrap high
      kh[0] = ld.kb + (uint64_t)p0 * a.k_page_b + in0 * a.k_tok_b;
      vh[0] = ld.vb + (uint64_t)p0 * a.v_page_b + in0 * a.v_tok_b;
      kh[1] = ld.kb + (uint64_t)p1 * a.k_page_b + in1 * a.k_tok_b;
      vh[1] = ld.vb + (uint64_t)p1 * a.v_page_b + in1 * a.v_tok_b;
    }
#pragma unroll
    for (int k = 0; k < KPW; ++k) {
      const int i = wave + k * W;
      if (i >= G::NI) break;
      int row, coff, dst;
      bool isk;
      load_slot<D>(i, lane, row, coff, isk, dst);
      const int hp = row >> 4;  // uniform except for head_dim 64's V blocks
      const char *base = isk ? (hp ? kh[1] : kh[0]) : (hp ? vh[1] : vh[0]);
      dma16(base + loff[k], stage + dst);
    }
    return;
  }
  int last = ld.c.L - 1 - pos0;  // last valid row of the tile
  last = last > 0 ? last : 0;     // (never negative, even for a plan that disagrees with L)
  const int32_t *tbl = reinterpret_cast<const int32_t *>(stage + G::KBYTES + G::VBYTES);
#pragma unroll
  for (int k = 0; k < KPW; ++k) {
    const int i = wave + k * W;
    if (i >= G::NI) break;
    int row, coff, dst;
    bool isk;
    load_slot<D>(i, lane, row, coff, isk, dst);
    row = row < last ? row : last;
    const char *base = isk ? ld.kb : ld.vb;
    const uint32_t tok_b = isk ? a.k_tok_b : a.v_tok_b;
    const int p = pos0 + row;
    uint64_t off;
    if (LAYOUT == CONTIG) {
      const int pc = p < ld.cap ? p : ld.cap - 1;
      off = (uint64_t)(uint32_t)pc * tok_b;
    } else if (LAYOUT == PAGED16) {
      const uint32_t page = min(row >= 16 ? ld.p1 : ld.p0, a.page_last);
      off = (uint64_t)page * (isk ? a.k_page_b : a.v_page_b) + ((uint32_t)p & a.page_mask) * tok_b;
    } else {
      const uint32_t page = min((uint32_t)tbl[row], a.page_last);
      const uint32_t in_page = a.page_size == 1 ? 0u : (uint32_t)(p - (p / a.page_size) * a.page_size);
      off = (uint64_t)page * (isk ? a.k_page_b : a.v_page_b) + in_page * tok_b;
    }
    dma16(base + off + 2 * coff, stage + dst);
  }
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
  mx = max_over_groups(mx) * a.scale_log2;
  // Lazy rescale: the reference max m moves only when a row's tile max exceeds it by
  // more than 8 (log2 units), so P <= 2^8 in between and O^T/l are rescaled rarely. This
  // is exact: O and l share the reference, and the output is O / l.
  if (__builtin_amdgcn_ballot_w64(mx > m + 8.f) != 0) {
    const float mnew = fmaxf(m, mx);
    const float alpha = __builtin_amdgcn_exp2f(m - mnew);  // 0 on the first tile (m = -inf)
    m = mnew;
    l *= alpha;
#pragma unroll
    for (int db = 0; db < G::DB; ++db) acc[db] *= alpha;
  }
  float p[2][4];
  float ps = 0.f;
#pragma unroll
  for (int pb = 0; pb < 2; ++pb)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      p[pb][i] = __builtin_amdgcn_exp2f(fmaf(s[pb][i], a.scale_log2, -m));
      ps += p[pb][i];
    }
  l += ps;
  const u32x4_t pk = {pack_bf16x2(p[0][0], p[0][1]), pack_bf16x2(p[0][2], p[0][3]),
                      pack_bf16x2(p[1][0], p[1][1]), pack_bf16x2(p[1][2], p[1][3])};
  // V^T operand: row d = 16 db + n, reduction positions pos(g, j) = 4g + j (j < 4) and
  // 16 + 4g + j - 4 (j >= 4), the positions of this lane's S^T values. Two
  // ds_read_b64_tr_b16 per operand: within each 16-lane group, lane l receives slot j
  // from element l % 4 of the 8 bytes lane 4j + l / 4 addressed; so lane s addresses
  // row 16h + 4g + s/4 at channels 16db + 4(s%4) .. +3.
  const int s4 = n >> 2, c4 = n & 3;
  int vb[2];
#pragma unroll
  for (int hh = 0; hh < 2; ++hh) {
    const int r = 16 * hh + 4 * g + s4;
    const int blk = (r & 3) + 4 * (r / (4 * G::RPB)), slot = (r % (4 * G::RPB)) >> 2;
    vb[hh] = G::KBYTES + blk * G::VPITCH + slot * (2 * D) + 8 * c4;
  }
  // The reads are issued as inline asm with their own lgkmcnt wait: through the
  // builtin, the compiler cannot tell them apart from the LDS-DMA writes still in
  // flight for later tiles and drains those (vmcnt(0)) before every tile's P.V.
  typedef __attribute__((address_space(3))) const char lds_char_t;
  const uint32_t a0 = (uint32_t)(uintptr_t)(lds_char_t *)(stage + vb[0]);
  const uint32_t a1 = (uint32_t)(uintptr_t)(lds_char_t *)(stage + vb[1]);
  u32x2_t w[2][G::DB];
#pragma unroll
  for (int db = 0; db < G::DB; ++db) {
    asm volatile("ds_read_b64_tr_b16 %0, %1 offset:%2" : "=v"(w[0][db]) : "v"(a0), "i"(32 * db));
    asm volatile("ds_read_b64_tr_b16 %0, %1 offset:%2" : "=v"(w[1][db]) : "v"(a1), "i"(32 * db));
  }
  static_assert(G::DB == 8 || G::DB == 4, "head_dim 128 or 64");
  if constexpr (G::DB == 8) {
    asm volatile("s_waitcnt lgkmcnt(0)"
                 : "+v"(w[0][0]), "+v"(w[1][0]), "+v"(w[0][1]), "+v"(w[1][1]), "+v"(w[0][2]),
                   "+v"(w[1][2]), "+v"(w[0][3]), "+v"(w[1][3]), "+v"(w[0][4]), "+v"(w[1][4]),
                   "+v"(w[0][5]), "+v"(w[1][5]), "+v"(w[0][6]), "+v"(w[1][6]), "+v"(w[0][7]),
                   "+v"(w[1][7]));
  } else {
    asm volatile("s_waitcnt lgkmcnt(0)"
                 : "+v"(w[0][0]), "+v"(w[1][0]), "+v"(w[0][1]), "+v"(w[1][1]), "+v"(w[0][2]),
                   "+v"(w[1][2]), "+v"(w[0][3]), "+v"(w[1][3]));
  }
#pragma unroll
  for (int db = 0; db < G::DB; ++db) {
    const u32x4_t vf = {w[0][db][0], w[0][db][1], w[1][db][0], w[1][db][1]};
    acc[db] = mfma_16x16x32(vf, pk, acc[db]);
  }
}

// The query rows of every unit in MFMA-block order: row r of unit (b, h, rg) is query
// head h*G + R / q_len at draft token R % q_len, R = rg * 16 nrb + r, rows beyond the
// group or the sequence's draft rows are zero. With the prologue requested, each row
// is QK-RMSNormed and rotated at its position (the code the standalone prologue runs,
// so the values are bit-identical to it). One wavefront per 16-row block.
template <int D>
__global__ __launch_bounds__(256) void pack_queries_kernel(const AttnArgs a) {
  constexpr int KT = D / 32;
  const int lane = threadIdx.x & 63, n = lane & 15, g = lane >> 4;
  const int64_t blk = (int64_t)blockIdx.x * 4 + wave_id();  // (unit, row block)
  const int64_t units = (int64_t)a.batch * a.ups;
  if (blk >= units * a.nrb) return;  // wave-uniform; no barrier follows
  const int64_t unit = blk / a.nrb;
  const int rb = (int)(blk - unit * a.nrb);
  const int b = (int)(unit / a.ups);
  const int ul = (int)(unit - (int64_t)b * a.ups);
  const int h = ul / a.rgroups, rg = ul - h * a.rgroups;
  const int r = rb * 16 + n;
  const int R = rg * 16 * a.nrb + r;
  const int gq = R / a.q_len, tq = R - gq * a.q_len;
  const bool valid = gq < a.group && tq < q_rows_of(a, b);
  const int64_t tok = q_token_index(a, b, valid ? tq : 0);
  const int64_t head = (int64_t)h * a.group + (valid ? gq : 0);
  const uint16_t *src = a.q + (a.cu_q ? tok * a.q_st : (int64_t)b * a.q_sb + (int64_t)(valid ? tq : 0) * a.q_st) +
                        head * a.q_sh + 8 * g;
  u32x4_t qf[KT];
#pragma unroll
  for (int t = 0; t < KT; ++t) qf[t] = valid ? load16(src + 32 * t) : u32x4_t{0, 0, 0, 0};
  if (a.qn_w != nullptr) {
    const int64_t rr = clamp_row(a.rope, valid ? (a.q_pos ? a.q_pos[tok] : tok) : 0);
    norm_rope_row<D>(qf, a.qn_w, a.eps, a.rope, rr, g);
  }
  uint16_t *dst = const_cast<uint16_t *>(a.qp) + (unit * 16 * a.nrb + r) * D + 8 * g;
#pragma unroll
  for (int t = 0; t < KT; ++t) store16(dst + 32 * t, valid ? qf[t] : u32x4_t{0, 0, 0, 0});
}

template <int LAYOUT, int W, int D>
__global__ __launch_bounds__(64 * W * replicas(W)) void attn_fwd_kernel(const AttnArgs a,
                                                          const int32_t *__restrict__ table,
                                                          const int32_t *__restrict__ plan,
                                                          const int32_t *__restrict__ seqlens) {
  using G = Geo<D>;
  constexpr int KT = D / 32;
  constexpr int KPW = (G::NI + W - 1) / W;
  // K/V loads per tile of wavefront w: IPW + 1 for w < NHI, else IPW.
  constexpr int IPW = G::NI / W, NHI = G::NI % W;
  constexpr int NQ = KT;            // query-row loads per lane for a segment
  constexpr int UNIT_Q = 16 * W * D * 2;  // bytes of a unit's packed query rows
  constexpr bool TBL = LAYOUT == PAGED;
  constexpr int R = replicas(W);
  static_assert(STAGES >= 3, "the wait schedule keeps two tiles apart");
  // Per replica: the K/V ring, then one query slot per wavefront.
  constexpr int RBYTES = G::SMEM + W * G::QW;
  __shared__ __attribute__((aligned(1024))) char smem_all[R * RBYTES];
  const SeqMeta<LAYOUT != CONTIG> sm{plan, seqlens};
  const int lane = threadIdx.x & 63, wv = wave_id();
  const int rep = wv / W, wave = wv - rep * W;  // replica, wavefront within it
  // (lets the compiler prove every wavefront issues all of its K/V loads per tile)
  __builtin_assume(wave >= 0 && wave < W && rep >= 0 && rep < R);
  const int n = lane & 15, g = lane >> 4;
  char *const smem = smem_all + rep * RBYTES;
  char *const qslot = smem + G::SMEM + wave * G::QW;
  const int64_t total = (int64_t)a.ups * sm.prefix(a, a.batch);
  const int share = (int)blockIdx.x * R + rep;
  const int64_t T0 = share_start(share, total, a.num_shares);
  const int ntiles = (int)(share_start(share + 1, total, a.num_shares) - T0);
  // Iterations of the workgroup: the largest share among its replicas (every wavefront
  // takes part in every barrier; a replica past its share only waits at them).
  int nloop = 0;
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int64_t sr = (int64_t)blockIdx.x * R + r;
    const int nr = (int)(share_start(sr + 1, total, a.num_shares) - share_start(sr, total, a.num_shares));
    nloop = nr > nloop ? nr : nloop;
  }

  // This lane's byte offsets inside a half tile for each of its loads (fast path).
  uint32_t loff[KPW];
#pragma unroll
  for (int k = 0; k < KPW; ++k) {
    const int i = wave + k * W;
    int row = 0, coff = 0, dst = 0;
    bool isk = true;
    if (i < G::NI) load_slot<D>(i, lane, row, coff, isk, dst);
    loff[k] = (uint32_t)(row & 15) * (isk ? a.k_tok_b : a.v_tok_b) + 2u * (uint32_t)coff;
  }
  // This lane's query channels inside a unit's packed rows.
  const char *qbase = reinterpret_cast<const char *>(a.qp) + ((wave * 16 + n) * D + 8 * g) * 2;

  Loader ld;  // next tile to load (i + STAGES - 1)
  ld.c = Cursor{0, 0, 0, 0, 0, 0, 0};
  if (ntiles > 0) {
    ld.c = cursor_at(a, sm, T0);
    loader_unit<LAYOUT>(table, ld);
    loader_pages<LAYOUT>(a, ld);
  }
  Cursor cc = ld.c;  // tile being computed (i)
  Cursor ct = ld.c;  // generic paging: next tile whose page ids are loaded (i + STAGES)
  if (TBL) {
    for (int j = 0; j < STAGES && j < ntiles; ++j) {
      if (wave == 0) issue_table<D>(a, table, ct, smem + j * G::STAGE, lane);
      if (j + 1 < ntiles) cursor_next(a, sm, ct);
    }
    wait_vm_lgkm0<0>();
    block_sync();
  }

  // Query rows of the next segment: LDS-DMA'd into this wavefront's query slot with
  // the first tile of their unit (the KT loads join that tile's group, so the group
  // wait covers them; loads into registers would make the compiler, which cannot
  // follow that wait across iterations, drain every load in flight before using
  // them). One unit at a time: a unit whose rows could not be prefetched (the slot
  // still unread) loads them when it starts.
  int qn_unit = -1;     // unit whose rows the slot holds or receives, -1: none pending
  uint32_t qflags = 0;  // bit j: the load group of tile i + j holds query rows
  auto prefetch_q = [&](int j) {
    if (qn_unit < 0) {
      const char *src = qbase + (uint64_t)(uint32_t)ld.c.u * UNIT_Q;
#pragma unroll
      for (int t = 0; t < KT; ++t) dma16(src + 64 * t, qslot + t * 1024);
      qn_unit = ld.c.u;
      qflags |= 1u << j;
    }
  };

  for (int j = 0; j < STAGES - 1 && j < ntiles; ++j) {
    if (j == 0 || ld.c.lt == 0) prefetch_q(j);
    issue_kv<LAYOUT, D, W>(a, ld, smem + j * G::STAGE, wave, lane, loff);
    if (j + 1 < ntiles) loader_advance<LAYOUT>(a, sm, table, ld);
  }

  u32x4_t qf[KT];
  f32x4_t acc[G::DB];
  float m = -INFINITY, l = 0.f;
  // Output of the segment ended last iteration, stored after the next wait so that its
  // stores do not sit in the vector memory queue in front of that wait.
  bool pend = false;
  float pend_inv = 0.f, pend_lse = 0.f;
  gfloat *pend_o = nullptr, *pend_l = nullptr;
  int cur = 0;                        // LDS offset of tile i's stage
  int nxt = (STAGES - 1) * G::STAGE;  // LDS offset of the stage of tile i + STAGES - 1
  for (int i = 0; i < nloop; ++i) {
    // Tile i's group is complete once every later load of this wavefront is allowed to
    // be outstanding: the groups of tiles i+1 .. i+STAGES-2 (and, on wavefront 0 with
    // generic paging, the page-id loads issued after tile i's).
    const int later = ntiles - 1 - i;
    const int e = __builtin_popcount(qflags & (((1u << (STAGES - 2)) - 1) << 1));
    if (i >= ntiles) {
      // past this replica's share: only the barrier
    } else if (TBL && wave == 0) {
      const int ipw = IPW + (0 < NHI ? 1 : 0);
      int nwait = ipw * min(STAGES - 2, later) + NQ * e;
      const int lo = max(i + 2, STAGES), hi = min(i + STAGES - 1, ntiles - 1);
      nwait += hi >= lo ? hi - lo + 1 : 0;
      // page ids of tile i + STAGES - 1 (issued last iteration, before its loads)
      if (i >= 1 && i + STAGES - 1 < ntiles) nwait = min(nwait, ipw + ((qflags >> (STAGES - 2)) & 1) * NQ);
      wait_vm_lgkm0(nwait);
    } else if (NHI == 0 || wave >= NHI) {
      wait_groups<IPW, NQ, STAGES - 2>(later, e);
    } else {
      wait_groups<IPW + 1, NQ, STAGES - 2>(later, e);
    }
    block_sync();
    if (i >= ntiles) continue;
    if (pend) {
#pragma unroll
      for (int db = 0; db < G::DB; ++db)
        *reinterpret_cast<__attribute__((address_space(1))) f32x4_t *>(pend_o + 16 * db) = acc[db] * pend_inv;
      if (g == 0) *pend_l = pend_lse;
      pend = false;
    }
    if (i == 0 || cc.lt == 0) {  // a segment starts: its query rows
      if (qn_unit == cc.u) {
        qn_unit = -1;
#pragma unroll
        for (int t = 0; t < KT; ++t) qf[t] = *reinterpret_cast<const u32x4_t *>(qslot + t * 1024 + lane * 16);
        // the slot may be refilled later in this iteration: the reads complete first
        wait_lgkm0();
      } else {
        // Not prefetched (units shorter than the ring; the slot may hold a later unit's
        // rows in flight): straight into registers, drained here.
        const char *src = qbase + (uint64_t)(uint32_t)cc.u * UNIT_Q;
#pragma unroll
        for (int t = 0; t < KT; ++t) qf[t] = load16(src + 64 * t);
        wait_vm_lgkm0<0>();
      }
#pragma unroll
      for (int t = 0; t < KT; ++t) asm volatile("" : "+v"(qf[t]));
#pragma unroll
      for (int db = 0; db < G::DB; ++db) acc[db] = f32x4_t{0.f, 0.f, 0.f, 0.f};
      m = -INFINITY;
      l = 0.f;
    }
    if (TBL && i + STAGES < ntiles) {
      if (wave == 0) issue_table<D>(a, table, ct, smem + cur, lane);  // tile i + STAGES
      cursor_next(a, sm, ct);
    }
    if (i + STAGES - 1 < ntiles) {
      if (ld.c.lt == 0) prefetch_q(STAGES - 1);
      issue_kv<LAYOUT, D, W>(a, ld, smem + nxt, wave, lane, loff);
    }

    compute_tile<D>(a, smem + cur, qf, acc, m, l, cc.lt * TILE, cc.L, lane);

    // The loader moves on after the tile's LDS reads: its page-id loads (scalar, on
    // the lgkm counter like LDS reads) then complete behind the P.V products.
    if (i + STAGES < ntiles) loader_advance<LAYOUT>(a, sm, table, ld);

    if (cc.lt == cc.tiles - 1 || i == ntiles - 1) {  // the segment ends
      const float lt_sum = sum_over_groups(l);
      pend = true;
      pend_inv = lt_sum > 0.f ? 1.f / lt_sum : 0.f;
      pend_lse = m + log2f(lt_sum);
      const int64_t row = ((int64_t)cc.u + (int)(blockIdx.x * R) + rep) * (16 * W) + wave * 16 + n;
      const PartPtrs pp = load_part_ptrs();
      pend_o = pp.o + row * D + 4 * g;
      pend_l = pp.lse + row;
    }
    if (i + 1 < ntiles) cursor_next(a, sm, cc);
    qflags >>= 1;
    cur = cur + G::STAGE == G::SMEM ? 0 : cur + G::STAGE;
    nxt = nxt + G::STAGE == G::SMEM ? 0 : nxt + G::STAGE;
  }
  if (pend) {
#pragma unroll
    for (int db = 0; db < G::DB; ++db)
      *reinterpret_cast<__attribute__((address_space(1))) f32x4_t *>(pend_o + 16 * db) = acc[db] * pend_inv;
    if (g == 0) *pend_l = pend_lse;
  }
}

// Merge each unit's partials (one per workgroup its tiles fell to, in slots unit + w)
// and write the bf16 output; units of empty sequences get zeros. One thread per
// (row, 4 channels): a unit's rows * D / 4 items fill whole workgroups of 256 threads,
// so the unit, and with it the sequence metadata, is uniform per workgroup.
template <int D>
__global__ __launch_bounds__(256) void attn_combine_kernel(const AttnArgs a) {
  constexpr int C = D / 4;  // float4 chunks per row
  const int rows = a.nrb * 16;
  const int64_t per_unit = (int64_t)rows * C;  // a multiple of 256
  const int64_t unit = (int64_t)blockIdx.x * 256 / per_unit;
  const int item = (int)((int64_t)blockIdx.x * 256 - unit * per_unit) + threadIdx.x;
  const int r = item / C, c = item - (item / C) * C;
  const int b = (int)(unit / a.ups);
  const int ul = (int)(unit - (int64_t)b * a.ups);
  const int h = ul / a.rgroups, rg = ul - h * a.rgroups;
  const int64_t pre = tile_prefix(a, a.plan, b);
  const int tiles_b = (int)(tile_prefix(a, a.plan, b + 1) - pre);
  const int qlen_b = q_rows_of(a, b);
  const int64_t first_tok = q_token_index(a, b, 0);
  const int R = rg * rows + r;
  const int gq = R / a.q_len, tq = R - gq * a.q_len;
  if (gq >= a.group || tq >= qlen_b) return;
  f32x4_t acc = {0.f, 0.f, 0.f, 0.f};
  if (tiles_b > 0) {
    const int64_t total = (int64_t)a.ups * tile_prefix(a, a.plan, a.batch);
    const int64_t nw = a.num_shares;
    const int64_t U0 = (int64_t)a.ups * pre + (int64_t)ul * tiles_b;
    const int64_t wa = share_of(U0, total, nw), wb = share_of(U0 + tiles_b - 1, total, nw);
    // Running LSE merge; the loads of different segments are independent.
    float M = -INFINITY, den = 0.f;
#pragma unroll 4
    for (int64_t w = wa; w <= wb; ++w) {
      const int64_t row = (unit + w) * rows + r;
      const float lw = a.part_lse[row];
      const f32x4_t ow = *reinterpret_cast<const f32x4_t *>(a.part_o + row * D + 4 * c);
      if (lw == -INFINITY) continue;
      const float Mn = fmaxf(M, lw);
      const float fo = __builtin_amdgcn_exp2f(M - Mn), fw = __builtin_amdgcn_exp2f(lw - Mn);
      acc = acc * fo + ow * fw;
      den = den * fo + fw;
      M = Mn;
    }
    acc *= den > 0.f ? 1.f / den : 0.f;
  }
  const int64_t head = (int64_t)h * a.group + gq;
  uint16_t *dst = a.o +
                  (a.cu_q ? (first_tok + tq) * a.o_st : (int64_t)b * a.o_sb + (int64_t)tq * a.o_st) +
                  head * a.o_sh + 4 * c;
  *reinterpret_cast<u32x2_t *>(dst) = u32x2_t{pack_bf16x2(acc[0], acc[1]), pack_bf16x2(acc[2], acc[3])};
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

typedef void (*AttnKernel)(const AttnArgs, const int32_t *, const int32_t *, const int32_t *);

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
  int num_wg;      // workgroups of the persistent grid
  int num_shares;  // num_wg * replicas
  size_t plan_off, q_off, lse_off, o_off, bytes;
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
  const int r = replicas(sz->rp.nrb);
  int64_t nw = (int64_t)info.cus * occupancy(k, 64 * sz->rp.nrb * r);
  const int cap = env_int("FLASHMAP_SPLITKV_WORKGROUPS", 0);
  if (cap > 0) nw = cap;
  const int64_t want = (tiles_bound + min_tiles - 1) / min_tiles;  // shares worth splitting
  if ((want + r - 1) / r < nw) nw = (want + r - 1) / r;
  if (nw < 1) nw = 1;
  sz->num_wg = (int)nw;
  sz->num_shares = (int)nw * r;
  const size_t rows = (size_t)sz->rp.nrb * 16;
  const size_t units = (size_t)batch * ups;
  const size_t slots = units + (size_t)sz->num_shares;  // partial slot unit + share
  size_t off = 0;
  sz->plan_off = off;
  if (need_plan) off = align256(off + sizeof(int32_t) * ((size_t)batch + 1));
  sz->q_off = off;
  off = align256(off + sizeof(uint16_t) * units * rows * d);
  sz->lse_off = off;
  off = align256(off + sizeof(float) * slots * rows);
  sz->o_off = off;
  off = align256(off + sizeof(float) * slots * rows * d);
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
  FM_REQUIRE(al16(c.q) && al16(c.out) && al16(a.u.k) && al16(a.u.v), "q/out/k/v must be 16-byte aligned");
  FM_REQUIRE(c.q_sb % 8 == 0 && c.q_st % 8 == 0 && c.q_sh % 8 == 0 && c.o_sb % 8 == 0 &&
                 c.o_st % 8 == 0 && c.o_sh % 8 == 0,
             "query/output strides must be multiples of 8 elements");
  FM_REQUIRE(a.u.k_s0 % 8 == 0 && a.u.k_s1 % 8 == 0 && a.k_s2 % 8 == 0 && a.u.v_s0 % 8 == 0 &&
                 a.u.v_s1 % 8 == 0 && a.v_s2 % 8 == 0,
             "key/value strides must be multiples of 8 elements");
  if (c.qn_w) FM_REQUIRE(c.rope_cos && c.rope_sin, "the query prologue needs the rotary table");
  // The kernels form per-tile addresses with 32-bit byte strides.
  if (a.k_s2 < 0 || a.v_s2 < 0 || a.k_s2 >= (1ll << 27) || a.v_s2 >= (1ll << 27))
    return fail(FM_ERR_UNSUPPORTED, "position strides must lie in [0, 2^27) elements");
  a.k_tok_b = (uint32_t)(2 * a.k_s2);
  a.v_tok_b = (uint32_t)(2 * a.v_s2);
  if (layout != CONTIG) {
    if (a.u.k_s0 < 0 || a.u.v_s0 < 0 || a.u.k_s0 >= (1ll << 31) || a.u.v_s0 >= (1ll << 31) ||
        (int64_t)a.page_size * (a.k_s2 > a.v_s2 ? a.k_s2 : a.v_s2) >= (1ll << 31))
      return fail(FM_ERR_UNSUPPORTED, "page strides must lie in [0, 2^31) elements");
    a.k_page_b = (uint32_t)(2 * a.u.k_s0);
    a.v_page_b = (uint32_t)(2 * a.u.v_s0);
    a.page_mask = (uint32_t)(a.page_size - 1);
    a.col_last = (uint32_t)(a.table_width - 1 < 0x7fffffffll ? a.table_width - 1 : 0x7fffffffll);
    a.page_last = (uint32_t)(a.num_pages - 1 < 0xffffffffll ? a.num_pages - 1 : 0xffffffffll);
  }
  const bool need_plan = a.seqlens != nullptr && c.plan == nullptr;
  Sizing sz;
  int rc = sizing(layout, c.batch, c.q_len, c.hq, c.hkv, c.d, c.max_k, need_plan, &sz);
  if (rc != FM_OK) return rc;
  if (c.ws == nullptr || c.ws_bytes < sz.bytes)
    return fail(FM_ERR_WORKSPACE, "workspace of %zu bytes, need %zu", c.ws_bytes, sz.bytes);
  FM_REQUIRE(al16(c.ws), "workspace must be 16-byte aligned");
  const int64_t units = (int64_t)c.batch * c.hkv * sz.rp.rgroups;
  FM_REQUIRE(units + sz.num_shares < (1ll << 31) && units * sz.rp.nrb < (1ll << 33), "too many units");

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
  a.ups = c.hkv * sz.rp.rgroups;
  a.nrb = sz.rp.nrb;
  a.scale_log2 = c.scale * 1.4426950408889634f;
  a.qn_w = c.qn_w;
  a.rope = Rope{c.rope_cos, c.rope_sin, c.rope_rs, c.rope_ps, c.rope_rows};
  a.q_pos = c.q_pos;
  a.eps = c.eps;
  a.num_shares = sz.num_shares;
  char *ws = (char *)c.ws;
  a.qp = (const uint16_t *)(ws + sz.q_off);
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
  const int64_t qblocks = (units * sz.rp.nrb + 3) / 4;
  if (c.d == 128)
    pack_queries_kernel<128><<<dim3((unsigned)qblocks), dim3(256), 0, c.stream>>>(a);
  else
    pack_queries_kernel<64><<<dim3((unsigned)qblocks), dim3(256), 0, c.stream>>>(a);
  FM_CHECK_HIP(hipGetLastError());
  AttnKernel k = select_kernel(layout, c.d, sz.rp.nrb);
  const int32_t *ktab = a.table, *kplan = a.plan, *kseq = a.seqlens;
  void *kargs[] = {&a, &ktab, &kplan, &kseq};
  profile_before(c.stream);
  const hipError_t lerr = hipLaunchKernel(reinterpret_cast<const void *>(k), dim3(sz.num_wg),
                                          dim3(64 * sz.rp.nrb * replicas(sz.rp.nrb)), kargs, 0, c.stream);
  profile_after(c.stream);
  if (lerr != hipSuccess) return fail(FM_ERR_HIP, "attention launch failed: %s", hipGetErrorString(lerr));
  // rows * D / 4 = 4 nrb D items per unit: a whole number of 256-thread workgroups.
  const int64_t cblocks = units * sz.rp.nrb * 4 * c.d / 256;
  FM_REQUIRE(cblocks < (1ll << 31), "too many units");
  if (c.d == 128)
    attn_combine_kernel<128><<<dim3((unsigned)cblocks), dim3(256), 0, c.stream>>>(a);
  else
    attn_combine_kernel<64><<<dim3((unsigned)cblocks), dim3(256), 0, c.stream>>>(a);
  FM_CHECK_HIP(hipGetLastError());
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
  a.u.k = (const uint16_t *)k;
  a.u.v = (const uint16_t *)v;
  a.u.k_s0 = k_stride_batch, a.u.k_s1 = k_stride_head, a.k_s2 = k_stride_pos;
  a.u.v_s0 = v_stride_batch, a.u.v_s1 = v_stride_head, a.v_s2 = v_stride_pos;
  // An empty cache: every sequence attends to nothing (zeros), whatever seqlens_k says.
  a.seqlens = kv_len > 0 ? seqlens_k : nullptr;
  a.uniform_len = kv_len;
  a.u.pos_cap = kv_len;
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
  a.u.k = (const uint16_t *)kv_cache;
  a.u.v = (const uint16_t *)kv_cache + v_offset;
  a.u.k_s0 = stride_block, a.u.k_s1 = stride_head, a.k_s2 = stride_token;
  a.u.v_s0 = stride_block, a.u.v_s1 = stride_head, a.v_s2 = stride_token;
  a.table = block_table;
  a.u.table_stride = block_table_stride;
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
  a.u.k = (const uint16_t *)key_buffer;
  a.u.v = (const uint16_t *)value_buffer;
  a.u.k_s0 = k_stride_slot, a.u.k_s1 = k_stride_head, a.k_s2 = 0;
  a.u.v_s0 = v_stride_slot, a.u.v_s1 = v_stride_head, a.v_s2 = 0;
  a.table = page_table;
  a.u.table_stride = page_table_stride;
  a.table_width = page_table_width;
  a.num_pages = pool_size;
  a.page_size = 1;
  a.page_shift = 0;
  a.seqlens = cache_seqlens;
  return run_attention(c, PAGED, a);
}
