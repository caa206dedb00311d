// a5/a6/a7: block attention of the K draft slots onto the context keys/values, for
// contiguous (FlashMapCache), block-paged (vLLM) and token-paged (SGLang) KV.
//
// Work decomposition (split-KV, "stream-K" style). A unit is (sequence b, KV head h,
// row group rg): the G query heads sharing KV head h times the q_len draft rows,
// packed into 16-row MFMA blocks (row r = query head h*G + r / q_len at token
// r % q_len, the GQA row convention of flashmap/sglang/verify_attention.py:77-79).
// Each unit's context is cut into tiles of 32 positions (64 for e4m3 K/V); all units'
// tiles form one line (sequence-major, then head, then row group) that is cut into
// num_shares shares of equal cost (every unit counting its tiles plus a fixed cost for
// its segment start, share_first_tiles), R per workgroup of the persistent grid (see
// replicas()). A share is walked unit by unit, one "segment" per unit it touches,
// leaving for every segment one partial (O normalized by its own softmax sum, in fp16
// with a row scale, and the log2-sum-exp) in slot unit + share, which is unique along
// the line. attn_combine_kernel merges each unit's partials (the LSE merge of
// flashmap/sglang/verify_attention.py:184-233) and writes the bf16 output.
//
// Three launches per call (two when the units are at most the shares: the streaming
// kernel then reads the caller's query rows and applies the prologue itself):
//   pack_queries_kernel  the query rows of every unit, in the order the MFMA blocks
//                        consume them, with the optional QK-RMSNorm + RoPE prologue
//                        applied (invalid rows are zero): the streaming kernel then
//                        addresses a unit's queries as one contiguous block and can
//                        prefetch them ahead of the unit
//   attn_fwd_kernel      the K/V stream and the online softmax
//   attn_combine_kernel  the merge and the scatter into the caller's output layout
// Small calls (the whole K/V within one pass of 8-tile workgroups over the CUs: batch 1
// at a few thousand positions) run attn_small_kernel in place of the first two (one
// workgroup per share of about one CU's worth of tiles, a loader wavefront issuing all of
// its loads at once, the caller's rows read directly) and attn_merge_wide_kernel in place
// of the combine (eight lanes per output row chunk, for the tens of segments per unit).
//
// Replica of the persistent kernel = one producer wavefront and one consumer wavefront
// per 16-row block of the unit (4 at GQA 4 x 16 rows). The producer streams the share's
// K/V tiles from HBM straight into an LDS ring of STAGES tiles with LDS-DMA
// (global_load_lds_dwordx4, no registers in flight) and stores the segments' partials;
// tile i is consumed after its hand-counted s_waitcnt vmcnt and a barrier while tiles
// i+1 .. i+STAGES-1 are in flight. K lands in LDS already in MFMA operand order. The
// consumers load the next unit's query rows while the current unit streams, so a unit
// change costs no pipeline drain.
// Per tile, wavefront w (its 16 rows r):
//   S^T[pos][r] = K Q^T       v_mfma_f32_16x16x32_bf16, A = K from LDS, B = Q in registers
//   online softmax on S^T:    each lane owns one row (lane % 16): the running max, sum
//                             and rescale are lane-local; the max crosses 4 lane groups
//   O^T[d][r] += V^T P^T      B = P^T is the S^T accumulator rounded to bf16 as is;
//                             A = V^T is read transposed out of LDS with
//                             ds_read_b64_tr_b16 (ds_read_b64_tr_b8 + an exact
//                             widening to bf16 for e4m3 V)
// so no wavefront exchanges data with another and each writes its own rows.
#include <math.h>
#include <stddef.h>

#include <atomic>
#include <climits>
#include <mutex>
#include <type_traits>

#include "fm_device.h"
#include "fm_host.h"

namespace fm {

constexpr int TILE = 32;    // context positions per tile (bf16 K/V)
constexpr int TILE_F8 = 64; // e4m3 K/V: the same bytes per tile as bf16
constexpr int NRB_MAX = 8;  // wavefronts (16-row blocks) per unit
constexpr int STAGES = 3;     // LDS ring depth (tiles), bf16 K/V
constexpr int STAGES_F8 = 3;  // e4m3 K/V (tiles of TILE_F8 positions)
constexpr int MAX_RUNS = 8;   // paged: runs of KV heads over several caches

// Replicas per workgroup: R independent groups of W consumer wavefronts and one producer
// wavefront, each streaming its own share through its own LDS ring, that meet at one
// barrier per tile. One workgroup per CU (at head_dim 128) then keeps every resident
// wavefront in lockstep: co-resident workgroups would instead be served oldest-first, and
// with equal static shares the youngest would finish last, leaving a tail with a
// fraction of the loads in flight. Two replicas while the workgroup stays within 12
// wavefronts (3 per SIMD, so up to 168 VGPRs each); for bf16 K/V in pages of 16 or more
// (or contiguous) up to 3 row blocks: from 4 (GQA 4 and 5) one replica streaming
// 64-position line tiles (below) measured faster. At GQA 5: C5 kernel 131.0 -> 128.8 us,
// combine 7.3 -> 6.7 us. At GQA 4, five alternating runs on one box: C3 175.96 -> 174.46
// us per call (half the shares, so about half the partials to merge); C4 171.45 -> 169.28
// us. On token pools the two-replica kernel's K staged by rows wins (verify, 68 rows: 193 us
// against 218 us with one replica).
enum Layout { CONTIG = 0, PAGED16 = 1, PAGED = 2 };
__host__ __device__ constexpr int replicas(int w, bool f8 = false, int layout = PAGED16) {
  return 2 * (w + 1) <= (f8 || layout == PAGED ? 12 : 8) ? 2 : 1;
}

// bf16 one-replica workgroups (W >= 5 row blocks) stream 64-position line tiles, each ring
// slot holding two 32-position stages: the barrier cycle costs about the same at every
// tile size (the producer's page ids and hand-off, the consumers' bookkeeping), so one
// replica moves twice the bytes per cycle (two replicas already move two tiles).
__host__ __device__ constexpr bool double_tiles(int w, bool f8, int layout) { return !f8 && replicas(w, f8, layout) == 1; }

// K/V geometry of the units.
struct UnitArgs {
  const char *k;  // bytes (the element size is the kernel's)
  const char *v;
  int64_t k_s0, k_s1;  // CONTIG: batch, head; paged: page (slot), head (elements)
  int64_t v_s0, v_s1;
  int64_t table_stride;
  int32_t pos_cap;  // CONTIG: positions the K/V tensors hold (reads are clamped below it)
  int32_t pad;
};

struct AttnArgs {
  UnitArgs u;
  // Per-tile address arithmetic in 32 bits (byte strides; the host checks they fit).
  uint32_t k_tok_b, v_tok_b;    // position / token stride
  uint32_t k_page_b, v_page_b;  // paged: page (slot) stride
  uint32_t page_mask;           // page_size - 1 (power-of-two pages)
  uint32_t col_last, page_last; // table_width - 1, num_pages - 1
  int32_t page_size, page_shift;
  // Token-paged (PAGED, page_size 1) only: csr != 0 reads sequence b's page ids at
  // table[indptr[b] ..] and its length as indptr[b + 1] - indptr[b] (indptr passed in
  // place of seqlens); ids are int32, or the low halves of int64 ids with id_shift 1.
  int32_t csr, id_shift;
  int64_t k_s2, v_s2;           // position strides (elements)
  // Paged layouts: the KV heads in runs over several caches of one geometry (vLLM's
  // virtual context-cache layout): heads h >= run_head[r] (r < nruns) read K/V from
  // run_k[r] / run_v[r] + h * head stride, the other heads from u.k / u.v (run 0). The
  // bases are offset by the run's first cache slot minus its first head.
  int32_t nruns;
  int32_t run_head[MAX_RUNS];
  const char *run_k[MAX_RUNS], *run_v[MAX_RUNS];
  int64_t table_width, num_pages;
  const int32_t *table;
  const int32_t *plan;     // tile prefix over sequences (NULL with seqlens == NULL)
  const int32_t *seqlens;  // NULL: every sequence has uniform_len positions
  int32_t uniform_len, uniform_tiles;
  int32_t batch, hkv, rgroups, ups;  // ups = hkv * rgroups units per sequence
  int32_t nrb;                       // 16-row blocks (wavefronts) per unit
  int32_t num_shares;  // workgroups x replicas
  int32_t share_c;     // a unit's extra cost in tiles when the line is cut into shares (share_first_tiles)
  int32_t *plan_out;   // set: the query pass's last workgroup writes the call's plan here
  float scale_log2;
  float v_scale;  // combine: scale of the context partials' values (1 but for verify calls)
  int32_t tail;   // verify calls: unit u's verify-token partial is slot units + num_shares + u
  // FP8 K/V: the packed queries are e4m3 with a score scale per row (q_rs: (units, 16 nrb)
  // floats); descales (q, k, v) per (sequence, KV head) at [b * sb + h * sh] (NULL: 1);
  // q_fp8: the caller's queries are e4m3 already (else bf16, quantized per (sequence,
  // query head) with scale amax / 448).
  int32_t f8, q_fp8;
  int32_t t64;  // the line's tiles are 64 positions (e4m3, and bf16 one-replica workgroups)
  float *q_rs;
  const float *qd, *kd, *vd;
  int64_t d_sb, d_sh;
  const uint16_t *qp;  // packed queries: (units, 16 nrb rows, D) bf16, invalid rows 0
  uint16_t *part_o;    // partials: (units + num_shares, 16 nrb, D) fp16, rows / their scale
  float *part_lse;     // (units + num_shares, 16 nrb, 2): log2-domain LSE, row scale
                       // (right after part_o)
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
//
// FP8 (e4m3 K/V, one byte per element): K block (pb, c) holds bytes 64 c .. 64 c + 63 of
// rows 16 pb + n at lane*16 (16 channels: the fp8 MFMA operands of two 32-channel
// k-steps); V block v holds rows RPB v .. RPB v + RPB - 1 by rows, the 16-byte chunk c of
// row r at chunk c ^ swz(r) (swz(r) = (r / rows per 256 bytes) mod LPR), so that the
// transposing ds_read_b64_tr_b8 of one 16-channel block spreads over the banks.
template <int D, bool F8 = false>
struct Geo {
  static constexpr int ES = F8 ? 1 : 2;        // bytes per element
  static constexpr int T = F8 ? TILE_F8 : TILE; // positions per tile
  static constexpr int NH = T / 16;             // 16-row blocks (page halves) per tile
  static constexpr int RB = D * ES;            // bytes per row
  static constexpr int KT = D / 32;            // bf16 k-steps over head_dim
  static constexpr int KC = RB / 64;           // 64-byte slices of a row (K blocks per 16 rows)
  static constexpr int DB = D / 16;            // 16-channel blocks of O^T
  static constexpr int KFRAGS = NH * KC;       // 1 KB K blocks per tile
  static constexpr int LPR = RB / 16;          // 16-byte chunks per row
  static constexpr int RPB = 64 / LPR;         // V rows per 1 KB block
  static constexpr int VBLKS = T / RPB;        // V blocks per tile
  static constexpr int VPITCH = F8 ? 1024 : 1024 + 32;  // bytes per V block (bf16: with pad)
  static constexpr int R256 = 256 / RB;        // FP8: rows per 256 bytes (the swizzle period)
  static constexpr int NI = KFRAGS + VBLKS;    // 16-byte LDS-DMA loads per lane per tile
  static constexpr int KBYTES = KFRAGS * 1024;
  static constexpr int VBYTES = VBLKS * VPITCH;
  static constexpr int TBYTES = 4 * T;         // page ids of the tile (generic paging)
  static constexpr int STAGE = KBYTES + VBYTES + TBYTES;
  static constexpr int NS = F8 ? STAGES_F8 : STAGES;  // ring depth
  static constexpr int SMEM = NS * STAGE;
};

__device__ __forceinline__ int64_t share_start(int64_t w, int64_t total, int64_t nw) {
  return w * total / nw;
}
__device__ __forceinline__ int64_t share_of(int64_t x, int64_t total, int64_t nw) {
  return ((x + 1) * nw - 1) / total;
}

typedef __attribute__((address_space(1))) float gfloat;  // global memory (global_* stores)
typedef __attribute__((address_space(1))) uint16_t gu16;

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
// p[0], p[1], q[0] and q[1] in one round trip.
__device__ __forceinline__ void sload2x2(const int32_t *p, const int32_t *q, int32_t &p0, int32_t &p1,
                                         int32_t &q0, int32_t &q1) {
  typedef __attribute__((ext_vector_type(2))) int32_t i32x2_t;
  i32x2_t v, w;
  asm volatile("s_load_dwordx2 %0, %2, 0x0\n\ts_load_dwordx2 %1, %3, 0x0\n\ts_waitcnt lgkmcnt(0)"
               : "=&s"(v), "=&s"(w)
               : "s"(uniform_ptr(p)), "s"(uniform_ptr(q)));
  p0 = v[0], p1 = v[1];
  q0 = w[0], q1 = w[1];
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
  int64_t row;  // paged layouts: offset of sequence b's page ids in the table (ids)
};

// Sequences whose (tile prefix, length) the streaming kernel stages in LDS at its start,
// so that no scalar load waits on the tile path (a scalar load's wait would also hold
// up the LDS reads around it, both counting on lgkmcnt); larger batches read them with
// scalar loads.
constexpr int SEQ_LDS = 1024;
typedef __attribute__((ext_vector_type(2))) int32_t i32x2_t;
typedef __attribute__((address_space(3))) const i32x2_t lds_i32x2_t;

// Plan and lengths of the streaming kernel; VAR: known to be per-sequence (the paged
// layouts always are), so the uniform-length fields are never read. tab: the staged
// (prefix, length) of sequences 0 .. batch when staged.
template <bool VAR>
struct SeqMeta {
  const int32_t *plan;
  const int32_t *seqlens;
  lds_i32x2_t *tab;
  bool staged;
  __device__ __forceinline__ bool var() const { return VAR || plan != nullptr; }
  __device__ __forceinline__ int64_t prefix(const AttnArgs &a, int b) const {
    if (!var()) return (int64_t)b * a.uniform_tiles;
    return staged ? (int64_t)tab[b][0] : (int64_t)sload(plan + b);
  }
  // The same with b differing between lanes (a vector load when not staged).
  __device__ __forceinline__ int64_t prefix_lane(const AttnArgs &a, int b) const {
    if (!var()) return (int64_t)b * a.uniform_tiles;
    return staged ? (int64_t)tab[b][0] : (int64_t)plan[b];
  }
  // tiles(b) = prefix(b + 1) - prefix(b), the length of sequence b and the offset of
  // its page ids. CSR: the second array is indptr, so the length is a difference.
  __device__ __forceinline__ void seq(const AttnArgs &a, int b, int &tiles, int &L, int64_t &row) const {
    if (!var()) {
      tiles = a.uniform_tiles;
      L = a.uniform_len;
      row = (int64_t)b * a.u.table_stride;
      return;
    }
    int32_t p0, p1, len;
    if (a.csr) {
      int32_t s0, s1;
      if (staged) {
        const i32x2_t e = tab[b], f = tab[b + 1];
        p0 = e[0], s0 = e[1], p1 = f[0], s1 = f[1];
      } else {
        sload2x2(plan + b, seqlens + b, p0, p1, s0, s1);
      }
      len = s1 - s0;
      row = s0;
    } else {
      if (staged) {
        const i32x2_t e = tab[b];
        p0 = e[0];
        len = e[1];
        p1 = tab[b + 1][0];
      } else {
        sload3(plan + b, seqlens + b, p0, p1, len);
      }
      row = (int64_t)b * a.u.table_stride;
    }
    tiles = p1 - p0;
    L = len > 0 ? len : 0;
  }
};

template <bool VAR>
__device__ __forceinline__ void cursor_load(const AttnArgs &a, const SeqMeta<VAR> &sm, Cursor &c) {
  sm.seq(a, c.b, c.tiles, c.L, c.row);
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

// Shares are cut by cost, not by tiles: every unit counts its tiles plus a.share_c, the
// measured overhead of a segment (taking the next unit's query rows, handing a partial
// over) in tiles, so that shares holding many short units get fewer tiles. The cost line
// follows the tile line: sequence b's units start at cost ups (prefix(b) + c b), each
// spans tiles_b + c, its tile t at c + t. share_c = 0 gives the tile line itself.
//
// F[k] = first tile (index on the tile line) of share s0 + k; a share at or past
// num_shares gives the line's end. Every lane takes one sequence per pass (one LDS read
// each when the metadata is staged), and a ballot per boundary counts the sequences whose
// cost start lies at or before it.
template <int NB, bool VAR>
__device__ __forceinline__ void share_first_tiles(const AttnArgs &a, const SeqMeta<VAR> &sm, int64_t s0,
                                                  int64_t (&F)[NB]) {
  const int64_t c = a.share_c;
  const int64_t end = (int64_t)a.ups * sm.prefix(a, a.batch);  // the tile line's end
  const int64_t total = end + (int64_t)a.ups * c * a.batch;     // the cost line's end
  int64_t P[NB];
#pragma unroll
  for (int k = 0; k < NB; ++k) P[k] = share_start(s0 + k, total, a.num_shares);
  if (c == 0) {
#pragma unroll
    for (int k = 0; k < NB; ++k) F[k] = P[k];
    return;
  }
  int cnt[NB];
#pragma unroll
  for (int k = 0; k < NB; ++k) cnt[k] = 0;
  const int lane = threadIdx.x & 63;
  for (int b0 = 0; b0 < a.batch; b0 += 64) {
    const int b = b0 + lane;
    const bool ok = b < a.batch;
    const int64_t cb = (int64_t)a.ups * ((ok ? sm.prefix_lane(a, b) : 0) + c * b);
#pragma unroll
    for (int k = 0; k < NB; ++k) cnt[k] += __popcll(__builtin_amdgcn_ballot_w64(ok && cb <= P[k]));
  }
#pragma unroll
  for (int k = 0; k < NB; ++k) {
    const int lo = cnt[k] - 1;  // the last sequence whose cost start is <= P (cost(0) = 0)
    const int64_t pre = sm.prefix(a, lo);
    const int64_t tb = sm.prefix(a, lo + 1) - pre;
    const int64_t off = P[k] - (int64_t)a.ups * (pre + c * lo);  // < ups (tb + c)
    const int64_t span = tb + c;
    int64_t ul;
    if ((off >> 31) == 0)  // the usual case: a 32-bit division
      ul = (int64_t)((uint32_t)off / (uint32_t)span);
    else
      ul = off / span;
    const int64_t pos = off - ul * span;
    const int64_t t = (int64_t)a.ups * pre + ul * tb + (pos >= c ? pos - c : 0);  // in the overhead: tile 0
    F[k] = s0 + k >= a.num_shares ? end : t;
  }
}

typedef __attribute__((address_space(3))) void *lds_ptr_t;

// K/V are read once per call: non-temporal (nt), so the stream does not displace data
// that is reused (queries, partials, page tables) from the caches.
__device__ __forceinline__ void dma16(const void *g, void *l) {
  __builtin_amdgcn_global_load_lds(g, (lds_ptr_t)l, 16, 0, /*nt*/ 2);
}

// s_waitcnt vmcnt(N): this wavefront's vector memory operations but the last N are
// complete (LDS-DMA writes included); LDS and scalar loads are left to the compiler.
template <int N>
__device__ __forceinline__ void wait_vm() {
  static_assert(N >= 0 && N < 64, "vmcnt holds 6 bits");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

// The same with a run-time count (page-id loads join the stream).
__device__ __forceinline__ void wait_vm(int n) {
#define FM_W(N) \
  case N:       \
    wait_vm<N>(); \
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
      wait_vm<0>();
  }
#undef FM_W
}

__device__ __forceinline__ void block_sync() {
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
}

// Paged layouts: DMA the page ids a tile's loads need into the stage's id slot, one
// dword per lane, issued in the load stream ahead of the tile's K/V loads (so their
// latency hides like that of K/V and no scalar load waits in the loop). Pages of 16
// positions or a multiple: the pages of the two 16-position halves; otherwise (e.g.
// SGLang's token pool): the page of each of the 32 positions. Positions are clamped
// to the sequence, columns to the table.
template <int LAYOUT, int D, bool F8 = false>
__device__ __forceinline__ void issue_ids(const AttnArgs &a, const int32_t *__restrict__ table,
                                          const Cursor &c, char *stage, int lane) {
  using G = Geo<D, F8>;
  const int32_t *row = table + (c.row << a.id_shift);
  const int last = c.L - 1 > 0 ? c.L - 1 : 0;
  if (LAYOUT == PAGED16) {
    if (lane < G::NH) {
      int p = c.lt * G::T + 16 * lane;
      p = p < last ? p : last;
      const uint32_t col = min((uint32_t)p >> a.page_shift, a.col_last);
      __builtin_amdgcn_global_load_lds(row + col, (lds_ptr_t)(stage + G::KBYTES + G::VBYTES), 4, 0, 0);
    }
  } else if (lane < G::T) {
    int p = c.lt * G::T + lane;
    p = p < last ? p : last;
    int64_t col = a.page_size == 1 ? p : p / a.page_size;
    col = col < a.table_width ? col : a.table_width - 1;
    __builtin_amdgcn_global_load_lds(row + (col << a.id_shift), (lds_ptr_t)(stage + G::KBYTES + G::VBYTES), 4,
                                     0, 0);
  }
}

// Scalar state of the K/V stream: the next tile to load and the K/V bases of its unit
// (CONTIG: sequence b, head h at position 0; paged: head h of page 0).
struct Loader {
  Cursor c;
  int lim;  // positions of the unit that may be read unclamped (CONTIG: below pos_cap too)
  int cap;  // CONTIG: positions the K/V tensors hold
  const char *kb, *vb;
};

template <int LAYOUT, int ES = 2>
__device__ __forceinline__ void loader_unit(const AttnArgs &a, Loader &ld) {
  const UnitArgs &ua = a.u;
  const int64_t h = ld.c.h;
  if (LAYOUT == CONTIG) {
    ld.cap = ua.pos_cap;
    ld.lim = ld.c.L < ua.pos_cap ? ld.c.L : ua.pos_cap;
    ld.kb = ua.k + ((int64_t)ld.c.b * ua.k_s0 + h * ua.k_s1) * ES;
    ld.vb = ua.v + ((int64_t)ld.c.b * ua.v_s0 + h * ua.v_s1) * ES;
  } else {
    ld.lim = ld.c.L;
    const char *kb = ua.k, *vb = ua.v;
#pragma unroll
    for (int r = 1; r < MAX_RUNS; ++r)
      if (r < a.nruns && h >= a.run_head[r]) kb = a.run_k[r], vb = a.run_v[r];
    ld.kb = kb + h * ua.k_s1 * ES;
    ld.vb = vb + h * ua.v_s1 * ES;
  }
}

template <int LAYOUT, int ES = 2>
__device__ __forceinline__ void loader_advance(const AttnArgs &a, const SeqMeta<LAYOUT != CONTIG> &sm,
                                               Loader &ld) {
  if (cursor_next(a, sm, ld.c)) loader_unit<LAYOUT, ES>(a, ld);
}

// K stages by rows (load_slot): the generic-paging layout (SGLang's token pools) at bf16
// and head_dim 128, where the MFMA-ordered stage would have each load instruction gather
// sixteen scattered pool rows (address translation then held the loads back), in the
// persistent kernel's two-replica workgroups (W consumers per replica). Measured, one
// box, kernel: verify 211 -> 191 us, the drafter's call on a token pool at batch 64
// (32/8 heads, 256-8192 positions) 198 -> 185 us, at batch 8 x 32768 positions 200 -> 189 us; one-replica workgroups (8 consumers, tree
// drafting) got 13 % slower with it, and vLLM's 16-position pages (whose sixteen rows lie
// 512 bytes apart in one page) 2 % slower: both keep the MFMA-ordered stage.
template <int LAYOUT, int D, bool F8, int W>
__host__ __device__ constexpr bool krow() { return LAYOUT == PAGED && D == 128 && replicas(W, F8, LAYOUT) == 2; }

// Row (within the tile) and byte offset within the row of this lane's k-th load of a
// tile, and whether it is a K load. Load i = wave + k*W of the NI loads (K blocks, then
// V blocks).
template <int D, bool F8 = false, bool KROW = false>
__device__ __forceinline__ void load_slot(int i, int lane, int &row, int &coff, bool &isk, int &dst) {
  using G = Geo<D, F8>;
  const int n = lane & 15, g = lane >> 4;
  isk = i < G::KFRAGS;
  if (isk) {
    if constexpr (KROW) {
      // K by rows (token paging, bf16, head_dim 128): instruction i loads four rows whole,
      // one per 16 lanes, so that it touches four pool rows, not sixteen: slot s = 4 i + g
      // of the stage's K (256 bytes each) holds tile row (i & 3) + 16 (i >> 2) + 4 g (the
      // rows this lane also loads for V, so one pool address per row), its 16-byte chunk p
      // being the row's chunk p ^ (s & 15). compute_tile reads the fragments from there.
      static_assert(D == 128, "row-major K stages are head_dim 128");
      if constexpr (F8) {
        // e4m3 rows of 128 bytes: instruction i loads rows 8 i .. 8 i + 7 (eight lanes a
        // row; the rows this lane also loads for V), slot chunk p holding the row's chunk
        // p ^ ((row >> 1) & 7).
        row = 8 * i + (lane >> 3);
        coff = 16 * ((lane & 7) ^ ((row >> 1) & 7));
      } else {
        const int slot = 4 * i + g;
        row = (i & 3) + 16 * (i >> 2) + 4 * g;
        coff = 16 * (n ^ (slot & 15));
      }
    } else {
      const int pb = i / G::KC, c = i - (i / G::KC) * G::KC;
      row = 16 * pb + n;
      coff = 64 * c + 16 * g;
    }
    dst = i * 1024;
  } else {
    const int vb = i - G::KFRAGS;
    if constexpr (F8) {
      row = vb * G::RPB + lane / G::LPR;
      coff = 16 * ((lane % G::LPR) ^ ((row / G::R256) % G::LPR));
    } else {
      row = 4 * G::RPB * (vb / 4) + 4 * (lane / G::LPR) + (vb % 4);
      coff = 16 * (lane % G::LPR);
    }
    dst = G::KBYTES + vb * G::VPITCH;
  }
}

template <int LAYOUT, int D, int W, bool F8 = false, bool KROW = false>
__device__ __forceinline__ void issue_kv(const AttnArgs &a, const Loader &ld, char *stage, int wave,
                                         int lane, const uint32_t (&loff)[(Geo<D, F8>::NI + W - 1) / W]) {
  using G = Geo<D, F8>;
  constexpr int KPW = (G::NI + W - 1) / W;
  const int pos0 = ld.c.lt * G::T;
  const int32_t *ids = reinterpret_cast<const int32_t *>(stage + G::KBYTES + G::VBYTES);
  uint32_t pg[G::NH];  // PAGED16: pages of the 16-position blocks (negative ids wrap high)
#pragma unroll
  for (int q = 0; q < G::NH; ++q)
    pg[q] = LAYOUT == PAGED16 ? min((uint32_t)__builtin_amdgcn_readfirstlane(ids[q]), a.page_last) : 0u;
  if (LAYOUT != PAGED && pos0 + G::T <= ld.lim) {
    const char *kh[G::NH], *vh[G::NH];  // first rows of the 16-position blocks
#pragma unroll
    for (int q = 0; q < G::NH; ++q) {
      if (LAYOUT == CONTIG) {
        kh[q] = ld.kb + (uint64_t)(uint32_t)(pos0 + 16 * q) * a.k_tok_b;
        vh[q] = ld.vb + (uint64_t)(uint32_t)(pos0 + 16 * q) * a.v_tok_b;
      } else {
        const uint32_t in = (uint32_t)(pos0 + 16 * q) & a.page_mask;
        kh[q] = ld.kb + (uint64_t)pg[q] * a.k_page_b + in * a.k_tok_b;
        vh[q] = ld.vb + (uint64_t)pg[q] * a.v_page_b + in * a.v_tok_b;
      }
    }
#pragma unroll
    for (int k = 0; k < KPW; ++k) {
      const int i = wave + k * W;
      if (i >= G::NI) break;
      int row, coff, dst;
      bool isk;
      load_slot<D, F8>(i, lane, row, coff, isk, dst);
      const int hp = row >> 4;  // uniform except for head_dim 64's bf16 V blocks
      const char *base = isk ? kh[0] : vh[0];
#pragma unroll
      for (int q = 1; q < G::NH; ++q)
        if (hp == q) base = isk ? kh[q] : vh[q];
      dma16(base + loff[k], stage + dst);
    }
    return;
  }
  int last = ld.c.L - 1 - pos0;  // last valid row of the tile
  last = last > 0 ? last : 0;     // (never negative, even for a plan that disagrees with L)
  // Generic paging: every load's page id read first, then the loads. An LDS read placed
  // between two LDS-DMA instructions is awaited before the next one issues (the DMA
  // writes LDS), which serialized a tile's 16 loads behind 16 LDS round trips.
  uint32_t pid[KPW];
  if (LAYOUT == PAGED) {
#pragma unroll
    for (int k = 0; k < KPW; ++k) {
      const int i = wave + k * W;
      if (i >= G::NI) break;
      int row, coff, dst;
      bool isk;
      load_slot<D, F8, KROW>(i, lane, row, coff, isk, dst);
      row = row < last ? row : last;
      pid[k] = min((uint32_t)ids[row], a.page_last);
    }
  }
  const bool unit_pages = a.page_size == 1;  // token paging: every position its own page
#pragma unroll
  for (int k = 0; k < KPW; ++k) {
    const int i = wave + k * W;
    if (i >= G::NI) break;
    int row, coff, dst;
    bool isk;
    load_slot<D, F8, KROW>(i, lane, row, coff, isk, dst);
    row = row < last ? row : last;
    const char *base = isk ? ld.kb : ld.vb;
    const uint32_t tok_b = isk ? a.k_tok_b : a.v_tok_b;
    const int p = pos0 + row;
    uint64_t off;
    if (LAYOUT == CONTIG) {
      const int pc = p < ld.cap ? p : ld.cap - 1;
      off = (uint64_t)(uint32_t)pc * tok_b;
    } else if (LAYOUT == PAGED16) {
      uint32_t page = pg[0];
#pragma unroll
      for (int q = 1; q < G::NH; ++q)
        if ((row >> 4) == q) page = pg[q];
      off = (uint64_t)page * (isk ? a.k_page_b : a.v_page_b) + ((uint32_t)p & a.page_mask) * tok_b;
    } else {
      const uint32_t in_page = unit_pages ? 0u : (uint32_t)(p - (p / a.page_size) * a.page_size);
      off = (uint64_t)pid[k] * (isk ? a.k_page_b : a.v_page_b) + in_page * tok_b;
    }
    dma16(base + off + coff, stage + dst);
  }
}

// O^T += V^T P^T for one tile, in two steps so that the V reads fly while the softmax
// runs: pv_issue starts the reads of the tile's V^T operands (vbase: the tile's V blocks
// in the stage layout), pv_finish awaits them and accumulates with pk, this lane's bf16
// P^T values (row n, positions 16 pb + 4 g + i). Between the two, the caller issues no
// LDS or scalar memory operation of its own.
template <int D>
struct VFrags {
  u32x2_t w[2][D / 16];
};

template <int D>
__device__ __forceinline__ void pv_issue(const char *vbase, VFrags<D> &v, int lane) {
  using G = Geo<D>;
  const int n = lane & 15, g = lane >> 4;
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
    vb[hh] = blk * G::VPITCH + slot * (2 * D) + 8 * c4;
  }
  // The reads are issued as inline asm with their own lgkmcnt wait: through the
  // builtin, the compiler cannot tell them apart from the LDS-DMA writes still in
  // flight for later tiles and drains those (vmcnt(0)) before every tile's P.V.
  typedef __attribute__((address_space(3))) const char lds_char_t;
  const uint32_t a0 = (uint32_t)(uintptr_t)(lds_char_t *)(vbase + vb[0]);
  const uint32_t a1 = (uint32_t)(uintptr_t)(lds_char_t *)(vbase + vb[1]);
#pragma unroll
  for (int db = 0; db < G::DB; ++db) {
    asm volatile("ds_read_b64_tr_b16 %0, %1 offset:%2" : "=v"(v.w[0][db]) : "v"(a0), "i"(32 * db));
    asm volatile("ds_read_b64_tr_b16 %0, %1 offset:%2" : "=v"(v.w[1][db]) : "v"(a1), "i"(32 * db));
  }
}

template <int D>
__device__ __forceinline__ void pv_finish(VFrags<D> &v, const u32x4_t &pk, f32x4_t (&acc)[D / 16]) {
  using G = Geo<D>;
  static_assert(G::DB == 8 || G::DB == 4, "head_dim 128 or 64");
  if constexpr (G::DB == 8) {
    asm volatile("s_waitcnt lgkmcnt(0)"
                 : "+v"(v.w[0][0]), "+v"(v.w[1][0]), "+v"(v.w[0][1]), "+v"(v.w[1][1]), "+v"(v.w[0][2]),
                   "+v"(v.w[1][2]), "+v"(v.w[0][3]), "+v"(v.w[1][3]), "+v"(v.w[0][4]), "+v"(v.w[1][4]),
                   "+v"(v.w[0][5]), "+v"(v.w[1][5]), "+v"(v.w[0][6]), "+v"(v.w[1][6]), "+v"(v.w[0][7]),
                   "+v"(v.w[1][7]));
  } else {
    asm volatile("s_waitcnt lgkmcnt(0)"
                 : "+v"(v.w[0][0]), "+v"(v.w[1][0]), "+v"(v.w[0][1]), "+v"(v.w[1][1]), "+v"(v.w[0][2]),
                   "+v"(v.w[1][2]), "+v"(v.w[0][3]), "+v"(v.w[1][3]));
  }
#pragma unroll
  for (int db = 0; db < G::DB; ++db) {
    const u32x4_t vf = {v.w[0][db][0], v.w[0][db][1], v.w[1][db][0], v.w[1][db][1]};
    acc[db] = mfma_16x16x32(vf, pk, acc[db]);
  }
}


// e4m3 V in the F8 stage layout: one ds_read_b64_tr_b8 per 16-channel block gives lane
// (n, g) V[pos(g, j)][16 db + n] for j < 8 (pos(g, j) = 4 g + j, then 16 + 4 g + j - 4:
// the positions of its P^T values). Within a 16-lane group the read hands lane s, in
// slot j, byte s % 8 of the 8 bytes lane 2 j + s / 8 addressed, so lane s addresses row
// pos(g, s / 2) at channels 16 db + 8 (s % 2). The e4m3 values are exact in bf16.
// pv_issue_f8 starts one 32-position half's reads (vbase: the half's rows), pv_finish_f8
// awaits both halves' reads (at its first half) and accumulates half h with pk.
template <int D>
struct VFragsF8 {
  u32x2_t w[2][D / 16];
};

template <int D>
__device__ __forceinline__ void pv_issue_f8(const char *vbase, u32x2_t (&w)[D / 16], int lane) {
  using G = Geo<D, true>;
  const int n = lane & 15, g = lane >> 4;
  const int j = n >> 1;
  const int r = j < 4 ? 4 * g + j : 12 + 4 * g + j;  // pos(g, j)
  const uint32_t sw16 = 16u * (uint32_t)((r / G::R256) % G::LPR);
  typedef __attribute__((address_space(3))) const char lds_char_t;
  const uint32_t base = (uint32_t)(uintptr_t)(lds_char_t *)(vbase + (r / G::RPB) * G::VPITCH + (r % G::RPB) * G::RB +
                                                             8 * (n & 1));
#pragma unroll
  for (int db = 0; db < G::DB; ++db)
    asm volatile("ds_read_b64_tr_b8 %0, %1" : "=v"(w[db]) : "v"(base + (sw16 ^ (16u * db))));
}

template <int D>
__device__ __forceinline__ void pv_finish_f8(VFragsF8<D> &v, int h, const u32x4_t &pk, f32x4_t (&acc)[D / 16]) {
  using G = Geo<D, true>;
  static_assert(G::DB == 8 || G::DB == 4, "head_dim 128 or 64");
  if (h == 0) {  // both halves' reads
    if constexpr (G::DB == 8) {
      asm volatile("s_waitcnt lgkmcnt(0)"
                   : "+v"(v.w[0][0]), "+v"(v.w[0][1]), "+v"(v.w[0][2]), "+v"(v.w[0][3]), "+v"(v.w[0][4]),
                     "+v"(v.w[0][5]), "+v"(v.w[0][6]), "+v"(v.w[0][7]), "+v"(v.w[1][0]), "+v"(v.w[1][1]),
                     "+v"(v.w[1][2]), "+v"(v.w[1][3]), "+v"(v.w[1][4]), "+v"(v.w[1][5]), "+v"(v.w[1][6]),
                     "+v"(v.w[1][7]));
    } else {
      asm volatile("s_waitcnt lgkmcnt(0)"
                   : "+v"(v.w[0][0]), "+v"(v.w[0][1]), "+v"(v.w[0][2]), "+v"(v.w[0][3]), "+v"(v.w[1][0]),
                     "+v"(v.w[1][1]), "+v"(v.w[1][2]), "+v"(v.w[1][3]));
    }
  }
#pragma unroll
  for (int db = 0; db < G::DB; ++db) {
    const u32x2_t w = v.w[h][db];
    const u32x4_t vf = {e4m3x2_to_bf16x2(w[0], false), e4m3x2_to_bf16x2(w[0], true),
                        e4m3x2_to_bf16x2(w[1], false), e4m3x2_to_bf16x2(w[1], true)};
    acc[db] = mfma_16x16x32(vf, pk, acc[db]);
  }
}

// max(a, b, c) in one v_max3_f32, for operands known not to be NaN.
__device__ __forceinline__ float max3f(float a, float b, float c) {
  float r;
  asm("v_max3_f32 %0, %1, %2, %3" : "=v"(r) : "v"(a), "v"(b), "v"(c));
  return r;
}

// One tile for this wavefront's 16 rows: S^T = K Q^T, online softmax, O^T += V^T P^T. sl:
// this lane's row's score scale in log2 units (softmax_scale log2(e), times the row's
// query and key descales with fp8 K/V). F8: K and Q are e4m3 (the fp8 MFMA, each 16-byte
// fragment the operands of two k-steps), V e4m3 widened to bf16 after the transposing
// read; P is bf16 either way.
template <int D, bool F8 = false, bool KROW = false>
__device__ __forceinline__ void compute_tile(const AttnArgs &a, const char *stage,
                                             const u32x4_t (&qf)[Geo<D, F8>::KC], float sl, f32x4_t (&acc)[D / 16],
                                             float &m, float &l, int pos0, int L, int lane) {
  using G = Geo<D, F8>;
  constexpr int NH = G::NH;  // 16-position blocks of the tile
  const int g = lane >> 4;
  f32x4_t s[NH];
  VFrags<D> vq;  // bf16: the tile's V^T operands, read while the softmax runs
  if constexpr (!F8) {
    // Every K fragment of the tile in flight at once, then the MFMAs (left to itself, the
    // compiler waits for each read before its MFMA: eight LDS round trips per tile).
    constexpr int NK = NH * G::KC;
    static_assert(NK == 8 || NK == 4, "head_dim 128 or 64");
    typedef __attribute__((address_space(3))) const char lds_char_t;
    u32x4_t kf[NK];
    if constexpr (KROW) {
      // K by rows (load_slot): fragment (pb, t) of lane (n, g) is row 16 pb + n, chunk
      // 4 t + g, which lies in slot s = 16 pb + 4 (n & 3) + (n >> 2) at chunk
      // (4 t + g) ^ (s & 15): 256 s + 64 (t ^ (n & 3)) + 16 (g ^ (n >> 2)). Each group of
      // eight (and of sixteen) lanes reads distinct 16-byte bank groups.
      static_assert(NK == 8, "row-major K stages are head_dim 128");
      const int n = lane & 15;
      const uint32_t k0 =
          (uint32_t)(uintptr_t)(lds_char_t *)(stage + 256 * (4 * (n & 3) + (n >> 2)) + 16 * (g ^ (n >> 2)));
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        const uint32_t kt = k0 + 64 * (t ^ (n & 3));
        asm volatile("ds_read_b128 %0, %1" : "=v"(kf[t]) : "v"(kt));
        asm volatile("ds_read_b128 %0, %1 offset:4096" : "=v"(kf[4 + t]) : "v"(kt));
      }
    } else {
      const uint32_t ka = (uint32_t)(uintptr_t)(lds_char_t *)(stage + lane * 16);
#pragma unroll
      for (int i = 0; i < NK; ++i) asm volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(kf[i]) : "v"(ka), "i"(1024 * i));
    }
    if constexpr (NK == 8) {
      asm volatile("s_waitcnt lgkmcnt(0)"
                   : "+v"(kf[0]), "+v"(kf[1]), "+v"(kf[2]), "+v"(kf[3]), "+v"(kf[4]), "+v"(kf[5]), "+v"(kf[6]),
                     "+v"(kf[7]));
    } else {
      asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(kf[0]), "+v"(kf[1]), "+v"(kf[2]), "+v"(kf[3]));
    }
#pragma unroll
    for (int pb = 0; pb < NH; ++pb) {
      f32x4_t c = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int t = 0; t < G::KC; ++t) c = mfma_16x16x32(kf[pb * G::KC + t], qf[t], c);
      s[pb] = c;  // S^T[pos 16 pb + 4 g + i][row n]
    }
    pv_issue<D>(stage + G::KBYTES, vq, lane);
  }
  VFragsF8<D> vq8;  // e4m3: the tile's V^T operands (both 32-position halves)
  if constexpr (F8) {
    // As for bf16: every K fragment in flight at once, then the MFMAs.
    constexpr int NK = NH * G::KC;
    static_assert(NK == 8 || NK == 4, "head_dim 128 or 64");
    typedef __attribute__((address_space(3))) const char lds_char_t;
    u32x4_t kf[NK];
    if constexpr (KROW) {
      // K by rows (load_slot): fragment (pb, c) of lane (n, g) is row 16 pb + n, bytes
      // 64 c + 16 g, at 128 (16 pb + n) + 64 (c ^ (m >> 2)) + 16 (g ^ (m & 3)) with
      // m = (n >> 1) & 7: eight (and sixteen) lanes read distinct 16-byte bank groups.
      static_assert(NK == 8, "row-major K stages are head_dim 128");
      const int n = lane & 15, m = (n >> 1) & 7;
      const uint32_t k0 = (uint32_t)(uintptr_t)(lds_char_t *)(stage + 128 * n + 16 * (g ^ (m & 3)));
#pragma unroll
      for (int c = 0; c < 2; ++c) {
        const uint32_t kc = k0 + 64 * (c ^ (m >> 2));
        asm volatile("ds_read_b128 %0, %1" : "=v"(kf[c]) : "v"(kc));
        asm volatile("ds_read_b128 %0, %1 offset:2048" : "=v"(kf[2 + c]) : "v"(kc));
        asm volatile("ds_read_b128 %0, %1 offset:4096" : "=v"(kf[4 + c]) : "v"(kc));
        asm volatile("ds_read_b128 %0, %1 offset:6144" : "=v"(kf[6 + c]) : "v"(kc));
      }
    } else {
      const uint32_t ka = (uint32_t)(uintptr_t)(lds_char_t *)(stage + lane * 16);
#pragma unroll
      for (int i = 0; i < NK; ++i) asm volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(kf[i]) : "v"(ka), "i"(1024 * i));
    }
    if constexpr (NK == 8) {
      asm volatile("s_waitcnt lgkmcnt(0)"
                   : "+v"(kf[0]), "+v"(kf[1]), "+v"(kf[2]), "+v"(kf[3]), "+v"(kf[4]), "+v"(kf[5]), "+v"(kf[6]),
                     "+v"(kf[7]));
    } else {
      asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(kf[0]), "+v"(kf[1]), "+v"(kf[2]), "+v"(kf[3]));
    }
#pragma unroll
    for (int pb = 0; pb < NH; ++pb) {
      f32x4_t c = {0.f, 0.f, 0.f, 0.f};
      if constexpr (G::KC == 2) {  // head_dim 128: one 128-channel fp8 MFMA
        const u32x4_t k0 = kf[2 * pb], k1 = kf[2 * pb + 1];
        const i32x8_t ka8 = {(int)k0[0], (int)k0[1], (int)k0[2], (int)k0[3],
                             (int)k1[0], (int)k1[1], (int)k1[2], (int)k1[3]};
        const i32x8_t qb = {(int)qf[0][0], (int)qf[0][1], (int)qf[0][2], (int)qf[0][3],
                            (int)qf[1][0], (int)qf[1][1], (int)qf[1][2], (int)qf[1][3]};
        c = mfma_16x16x128_f8(ka8, qb, c);
      } else {
#pragma unroll
        for (int t = 0; t < G::KC; ++t) {
          const u32x4_t k = kf[pb * G::KC + t];
          c = mfma_16x16x32_f8(u32x2_t{k[0], k[1]}, u32x2_t{qf[t][0], qf[t][1]}, c);
          c = mfma_16x16x32_f8(u32x2_t{k[2], k[3]}, u32x2_t{qf[t][2], qf[t][3]}, c);
        }
      }
      s[pb] = c;  // S^T[pos 16 pb + 4 g + i][row n]
    }
#pragma unroll
    for (int h = 0; h < NH / 2; ++h) pv_issue_f8<D>(stage + G::KBYTES + h * 32 * G::RB, vq8.w[h], lane);
  }
  if (pos0 + G::T > L) {
#pragma unroll
    for (int pb = 0; pb < NH; ++pb)
#pragma unroll
      for (int i = 0; i < 4; ++i)
        if (pos0 + 16 * pb + 4 * g + i >= L) s[pb][i] = -INFINITY;
  }
  // The lane's row max with three-input maxima: fmaxf makes the compiler quiet each MFMA
  // result first (an extra max per value); the scores are never NaN here (finite products,
  // -inf where masked).
  float mx = max3f(s[0][0], s[0][1], s[0][2]);
#pragma unroll
  for (int k = 3; k + 1 < 4 * NH; k += 2) mx = max3f(mx, s[k / 4][k % 4], s[(k + 1) / 4][(k + 1) % 4]);
  mx = max3f(mx, s[NH - 1][3], s[NH - 1][3]);  // 4 NH - 3 values after the first three: an odd count
  mx *= sl;  // this lane group's max (sl > 0, so scaling and max commute)
  // Lazy rescale: the reference max m moves only when a row's tile max exceeds it by
  // more than 8 (log2 units), so P <= 2^8 in between and O^T/l are rescaled rarely. This
  // is exact: O and l share the reference, and the output is O / l. A row's max exceeds
  // m + 8 exactly when one of its four lane groups' does (the row's lanes hold the same
  // m), so the row max across the groups is formed only when m moves.
  if (__builtin_amdgcn_ballot_w64(mx > m + 8.f) != 0) {
    const float mnew = fmaxf(m, max_over_groups(mx));
    const float alpha = __builtin_amdgcn_exp2f(m - mnew);  // 0 on the first tile (m = -inf)
    m = mnew;
    l *= alpha;
#pragma unroll
    for (int db = 0; db < G::DB; ++db) acc[db] *= alpha;
  }
  float p[NH][4];
  float ps = 0.f;
#pragma unroll
  for (int pb = 0; pb < NH; ++pb)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      p[pb][i] = __builtin_amdgcn_exp2f(fmaf(s[pb][i], sl, -m));
      ps += p[pb][i];
    }
  l += ps;
  // P.V in 32-position halves (the bf16 stage holds one; an e4m3 stage holds its rows
  // in order, 32 RB bytes per half).
#pragma unroll
  for (int h = 0; h < NH / 2; ++h) {
    const u32x4_t pk = {pack_bf16x2(p[2 * h][0], p[2 * h][1]), pack_bf16x2(p[2 * h][2], p[2 * h][3]),
                        pack_bf16x2(p[2 * h + 1][0], p[2 * h + 1][1]), pack_bf16x2(p[2 * h + 1][2], p[2 * h + 1][3])};
    if constexpr (F8)
      pv_finish_f8<D>(vq8, h, pk, acc);
    else
      pv_finish<D>(vq, pk, acc);
  }
}

template <int D>
__device__ __forceinline__ void pv_accumulate(const char *vbase, const u32x4_t &pk, f32x4_t (&acc)[D / 16],
                                              int lane) {
  VFrags<D> v;
  pv_issue<D>(vbase, v, lane);
  pv_finish<D>(v, pk, acc);
}

// The verify tokens' own keys and values and the mask among them (target verification:
// every request has q_len tokens that see its whole context and, among themselves,
// what the mask allows).
struct VerifyArgs {
  const uint16_t *k, *v;  // (batch * q_len, kv heads, D): token b * q_len + j
  int64_t k_st, k_sh, v_st, v_sh;
  const uint8_t *mask;         // mode 1 / 2; nonzero = visible
  const int64_t *mask_indptr;  // mode 1: start of request b's mask rows
  int32_t mode;                // 0 causal, 1 rows of context + q_len entries, 2 q_len x q_len blocks
  float scale_log2;            // softmax_scale * log2(e) of the tokens' scores
};

// The first TILE tokens' keys (K operands) and values (stage V layout) of a wavefront's
// verify tokens, loaded before its query rows so that their latency overlaps the rows'.
template <int D>
struct VerifyChunk {
  u32x4_t k[2][D / 32];
  u32x4_t v[Geo<D>::NI - Geo<D>::KFRAGS];
};

template <int D>
__device__ __forceinline__ void verify_tokens(const AttnArgs &a, const VerifyArgs &v, const u32x4_t (&qf)[D / 32], char *vs,
                              int64_t unit, int b, int h, int rg, int rb, int lane, const VerifyChunk<D> &c0);
template <int D>
__device__ __forceinline__ void verify_chunk_load(const AttnArgs &a, const VerifyArgs &v, int b, int h, int j0,
                                                  int lane, VerifyChunk<D> &c);

// The step plan: both tile prefixes (32- and 64-position tiles) of the sequences' lengths
// (CSR: indptr differences), plan[0 .. batch] and plan[batch + 1 ..], by the NT threads of
// one workgroup (an inclusive scan per chunk of NT sequences). attn_plan_kernel runs it
// alone; the query pass of a call without a plan runs it in one workgroup of its own.
template <int NT>
__device__ __forceinline__ void plan_prefixes(const int32_t *__restrict__ seqlens, int32_t batch,
                                              int32_t *__restrict__ plan, int32_t csr) {
  __shared__ int32_t buf[2][NT];
  int32_t carry[2] = {0, 0};
  int32_t *out[2] = {plan, plan + batch + 1};
  if (threadIdx.x == 0) out[0][0] = 0, out[1][0] = 0;
  for (int base = 0; base < batch; base += NT) {
    const int i = base + threadIdx.x;
    int32_t L = i < batch ? (csr ? seqlens[i + 1] - seqlens[i] : seqlens[i]) : 0;
    L = L > 0 ? L : 0;
    buf[0][threadIdx.x] = (L + TILE - 1) / TILE;
    buf[1][threadIdx.x] = (L + TILE_F8 - 1) / TILE_F8;
    __syncthreads();
    for (int off = 1; off < NT; off <<= 1) {
      const bool in = threadIdx.x >= (unsigned)off;
      const int32_t add0 = in ? buf[0][threadIdx.x - off] : 0, add1 = in ? buf[1][threadIdx.x - off] : 0;
      __syncthreads();
      buf[0][threadIdx.x] += add0;
      buf[1][threadIdx.x] += add1;
      __syncthreads();
    }
    if (i < batch) out[0][i + 1] = carry[0] + buf[0][threadIdx.x], out[1][i + 1] = carry[1] + buf[1][threadIdx.x];
    carry[0] += buf[0][NT - 1];
    carry[1] += buf[1][NT - 1];
    __syncthreads();
  }
}

// One query row per lane group (lane (n, g): channels 32 t + 8 g .. + 7 of its row) read
// from src, QK-RMSNormed and rotated when a.qn_w is set (at the rotary row of position
// a.q_pos[tok], or tok). A row with ok false reads nothing. The norm weights are issued
// first, so that they, the row and its position take one memory round trip and the
// rotary row (addressed by the position) a second. ALL: every row of the wavefront is
// valid and no load is conditional; a conditional load is joined with zeros after it, and
// the join had the compiler wait for each such load before issuing the next.
template <int D, bool ALL>
__device__ __forceinline__ void query_row(const AttnArgs &a, u32x4_t (&x)[D / 32], const uint16_t *src, bool ok,
                                          int64_t tok, int g) {
  constexpr int KT = D / 32;
  const bool in = ALL || ok;
  if (a.qn_w != nullptr) {
    PrologueOps<D> ops;
    load_norm_ops<D>(ops, a.qn_w, g);
#pragma unroll
    for (int t = 0; t < KT; ++t) x[t] = in ? load16(src + 32 * t) : u32x4_t{0, 0, 0, 0};
    const int64_t rr = clamp_row(a.rope, in ? (a.q_pos ? a.q_pos[tok] : tok) : 0);
    load_rope_ops<D>(ops, a.rope, rr, g);
    norm_rope_apply<D>(x, ops, a.eps);  // every lane: the norm crosses lane groups
  } else {
#pragma unroll
    for (int t = 0; t < KT; ++t) x[t] = in ? load16(src + 32 * t) : u32x4_t{0, 0, 0, 0};
  }
}

// query_row with ALL chosen at run time: true when no active lane's row is invalid.
template <int D>
__device__ __forceinline__ void query_row_any(const AttnArgs &a, u32x4_t (&x)[D / 32], const uint16_t *src, bool ok,
                                              int64_t tok, int g) {
  if (__builtin_amdgcn_ballot_w64(!ok) == 0)
    query_row<D, true>(a, x, src, ok, tok, g);
  else
    query_row<D, false>(a, x, src, ok, tok, g);
}

// The query rows of every unit in MFMA-block order: row r of unit (b, h, rg) is query
// head h*G + R / q_len at draft token R % q_len, R = rg * 16 nrb + r, rows beyond the
// group or the sequence's draft rows are zero. With the prologue requested, each row
// is QK-RMSNormed and rotated at its position (the code the standalone prologue runs,
// so the values are bit-identical to it). One wavefront per 16-row block. VERIFY: the
// wavefront then attends its rows to their request's verify tokens (verify_tokens).
template <int D, bool VERIFY>
__global__ __launch_bounds__(256) void pack_queries_kernel(const AttnArgs a, const VerifyArgs v) {
  constexpr int KT = D / 32;
  if (a.plan_out != nullptr && blockIdx.x == gridDim.x - 1) {  // the call's plan (one launch fewer)
    plan_prefixes<256>(a.seqlens, a.batch, a.plan_out, a.csr);
    return;
  }
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
  VerifyChunk<D> vc;
  if constexpr (VERIFY) verify_chunk_load<D>(a, v, b, h, 0, lane, vc);
  const int64_t tok = q_token_index(a, b, valid ? tq : 0);
  const int64_t head = (int64_t)h * a.group + (valid ? gq : 0);
  const uint16_t *src = a.q + (a.cu_q ? tok * a.q_st : (int64_t)b * a.q_sb + (int64_t)(valid ? tq : 0) * a.q_st) +
                        head * a.q_sh + 8 * g;
  u32x4_t qf[KT];
  query_row_any<D>(a, qf, src, valid, tok, g);
  uint16_t *dst = const_cast<uint16_t *>(a.qp) + (unit * 16 * a.nrb + r) * D + 8 * g;
#pragma unroll
  for (int t = 0; t < KT; ++t) store16_nt(dst + 32 * t, valid ? qf[t] : u32x4_t{0, 0, 0, 0});
  if constexpr (VERIFY) {
    using G = Geo<D>;
    __shared__ __attribute__((aligned(1024))) char vstage[4][G::VBLKS * G::VPITCH];
#pragma unroll
    for (int t = 0; t < KT; ++t)
      if (!valid) qf[t] = u32x4_t{0, 0, 0, 0};
    verify_tokens<D>(a, v, qf, vstage[wave_id()], unit, b, h, rg, rb, lane, vc);
  }
}

// The query pass of an fp8 call: the packed rows are e4m3 (row-major, D bytes each) with
// a score scale per row, the query descale times the key descale of the row's (sequence,
// KV head). q_fp8: the caller's rows are e4m3 with their descale; otherwise the bf16 rows
// (after the optional prologue) are quantized as flashmap/sglang/model.py:167-169 does:
// scale = max(amax, 1e-12) / 448 with amax over every token row of the row's query head
// in its sequence, q / scale rounded to nearest even (q_len is a multiple of 16, so a
// 16-row block holds one head; a head spanning several blocks has their rows re-read).
// One wavefront per 16-row block, lane (n, g) holding channels 32 t + 8 g .. + 7.
template <int D>
__global__ __launch_bounds__(256) void pack_queries_f8_kernel(const AttnArgs a) {
  if (a.plan_out != nullptr && blockIdx.x == gridDim.x - 1) {  // the call's plan (one launch fewer)
    plan_prefixes<256>(a.seqlens, a.batch, a.plan_out, a.csr);
    return;
  }
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
  const int qrows = q_rows_of(a, b);
  const bool valid = gq < a.group && tq < qrows;
  const int64_t head = (int64_t)h * a.group + (gq < a.group ? gq : 0);
  const int64_t dix = (int64_t)b * a.d_sb + (int64_t)h * a.d_sh;
  auto row_src = [&](int t_) {  // element offset of token t_ of this sequence, head `head`
    return (a.cu_q ? (int64_t)(a.cu_q[b] + t_) * a.q_st : (int64_t)b * a.q_sb + (int64_t)t_ * a.q_st) +
           head * a.q_sh;
  };
  u32x2_t q8[KT];
  float rs;
  if (a.q_fp8) {
    const uint8_t *src = reinterpret_cast<const uint8_t *>(a.q) + row_src(valid ? tq : 0) + 8 * g;
#pragma unroll
    for (int t = 0; t < KT; ++t) q8[t] = valid ? *reinterpret_cast<const u32x2_t *>(src + 32 * t) : u32x2_t{0, 0};
    rs = a.qd ? a.qd[dix] : 1.f;
  } else {
    auto load_row = [&](int t_, bool ok, u32x4_t (&x)[KT]) {  // every lane calls it (the norm crosses lanes)
      const uint16_t *src = a.q + row_src(ok ? t_ : 0) + 8 * g;
      query_row_any<D>(a, x, src, ok, q_token_index(a, b, ok ? t_ : 0), g);
#pragma unroll
      for (int t = 0; t < KT; ++t)
        if (!ok) x[t] = u32x4_t{0, 0, 0, 0};
    };
    auto amax_of = [&](const u32x4_t (&x)[KT]) {
      float mx = 0.f;
#pragma unroll
      for (int t = 0; t < KT; ++t)
#pragma unroll
        for (int q = 0; q < 4; ++q) mx = fmaxf(mx, fmaxf(fabsf(bf16_lo(x[t][q])), fabsf(bf16_hi(x[t][q]))));
      return mx;
    };
    u32x4_t qf[KT];
    load_row(tq, valid, qf);
    float mx = amax_of(qf);
    const int tq0 = tq - n;  // first token row of this block (all of head gq)
    for (int k = 0; k < a.q_len; k += 16) {  // the head's other blocks
      if (k == tq0) continue;
      u32x4_t x[KT];
      load_row(k + n, gq < a.group && k + n < qrows, x);
      mx = fmaxf(mx, amax_of(x));
    }
#pragma unroll
    for (int o = 1; o < 16; o <<= 1) mx = fmaxf(mx, __shfl_xor(mx, o));
    mx = max_over_groups(mx);
    const float scale = __fdiv_rn(fmaxf(mx, 1e-12f), 448.f);
#pragma unroll
    for (int t = 0; t < KT; ++t) {
      float v[8];
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        v[2 * q] = __fdiv_rn(bf16_lo(qf[t][q]), scale);
        v[2 * q + 1] = __fdiv_rn(bf16_hi(qf[t][q]), scale);
      }
      q8[t] = u32x2_t{pack_e4m3x4(v[0], v[1], v[2], v[3]), pack_e4m3x4(v[4], v[5], v[6], v[7])};
    }
    rs = scale;
  }
  rs *= a.kd ? a.kd[dix] : 1.f;
  uint8_t *dst = reinterpret_cast<uint8_t *>(const_cast<uint16_t *>(a.qp)) + (unit * 16 * a.nrb + r) * D + 8 * g;
#pragma unroll
  for (int t = 0; t < KT; ++t) *reinterpret_cast<u32x2_t *>(dst + 32 * t) = valid ? q8[t] : u32x2_t{0, 0};
  if (g == 0) a.q_rs[unit * 16 * a.nrb + r] = valid ? rs : 0.f;
}

// A segment's partial for this wavefront's 16 rows: O = acc * inv as fp16 of O / scale,
// scale = the row's largest |O| (so every value is within [-1, 1] and keeps 11
// significant bits wherever the row's magnitude lies). h[db] holds channels
// 16 db + 4 g .. + 3 of row n.
template <int D>
__device__ __forceinline__ float make_partial(const f32x4_t (&acc)[D / 16], float inv, u32x2_t (&h)[D / 16]) {
  float mx = 0.f;
#pragma unroll
  for (int db = 0; db < D / 16; ++db)
#pragma unroll
    for (int q = 0; q < 4; ++q) mx = fmaxf(mx, fabsf(acc[db][q]));
  mx = max_over_groups(mx) * inv;
  const float sc = mx > 0.f ? mx : 1.f;
  const float k = inv / sc;
#pragma unroll
  for (int db = 0; db < D / 16; ++db)
    h[db] = u32x2_t{pack_f16x2(acc[db][0] * k, acc[db][1] * k), pack_f16x2(acc[db][2] * k, acc[db][3] * k)};
  return sc;
}

typedef __attribute__((ext_vector_type(2))) float f32x2_t;

// Partial slot layout in the workspace: rows (slot * 16 W + r) of D fp16, and per row
// (lse, scale) as two floats.
template <int D>
__device__ __forceinline__ void store_partial_rows(const AttnArgs &a, const u32x2_t (&h)[D / 16], float lse,
                                                   float sc, int64_t row, int g) {
  gu16 *dst = (gu16 *)a.part_o + row * D + 4 * g;
#pragma unroll
  for (int db = 0; db < D / 16; ++db)
    *reinterpret_cast<__attribute__((address_space(1))) u32x2_t *>(dst + 16 * db) = h[db];
  if (g == 0)
    *reinterpret_cast<__attribute__((address_space(1))) f32x2_t *>((gfloat *)a.part_lse + 2 * row) = f32x2_t{lse, sc};
}

// The verify tokens' part of a verify call for one wavefront's 16 rows (lane (n, g):
// row n, query fragments qf in the streaming kernel's layout): the rows attend to their
// request's q_len tokens under the mask, TILE tokens at a time -- keys loaded straight
// into registers in the K-operand layout, values staged in this wavefront's LDS slice
// vs in the stage's V layout -- and the result is stored as the unit's tail partial
// (O / scale in fp16, log2-domain LSE; -inf for a row that sees no token). Tokens past
// q_len read the last token (finite) and get P = 0. No branch surrounds the MFMA or the
// transposing LDS reads, which need every lane.
template <int D>
__device__ __forceinline__ void verify_chunk_load(const AttnArgs &a, const VerifyArgs &v, int b, int h, int j0,
                                                  int lane, VerifyChunk<D> &c) {
  using G = Geo<D>;
  constexpr int KT = D / 32;
  const int n = lane & 15, g = lane >> 4;
  const int L = a.q_len;
  const int64_t tok0 = (int64_t)b * L;
  const int last = L - 1 - j0;  // last token of the chunk
  const uint16_t *kb = v.k + (int64_t)h * v.k_sh;
  const uint16_t *vb = v.v + (int64_t)h * v.v_sh;
#pragma unroll
  for (int i = G::KFRAGS; i < G::NI; ++i) {
    int row, coff, dst;
    bool isk;
    load_slot<D>(i, lane, row, coff, isk, dst);
    const int j = j0 + (row < last ? row : last);
    c.v[i - G::KFRAGS] = load16(reinterpret_cast<const char *>(vb + (tok0 + j) * v.v_st) + coff);
  }
#pragma unroll
  for (int pb = 0; pb < 2; ++pb) {
    const int jr = 16 * pb + n;
    const uint16_t *kr = kb + (tok0 + j0 + (jr < last ? jr : last)) * v.k_st + 8 * g;
#pragma unroll
    for (int t = 0; t < KT; ++t) c.k[pb][t] = load16(kr + 32 * t);
  }
}

template <int D>
__device__ __forceinline__ void verify_tokens(const AttnArgs &a, const VerifyArgs &v, const u32x4_t (&qf)[D / 32], char *vs,
                              int64_t unit, int b, int h, int rg, int rb, int lane, const VerifyChunk<D> &c0) {
  using G = Geo<D>;
  constexpr int KT = D / 32;
  const int n = lane & 15, g = lane >> 4;
  const int L = a.q_len;
  const int rows = a.nrb * 16;
  const int64_t tok0 = (int64_t)b * L;
  const int R = rg * rows + rb * 16 + n;
  const int tq = R - (R / L) * L;  // row n's verify token
  int64_t mrow = 0;                // mask entry of (token tq, token 0)
  if (v.mode == 1) {
    const int ctx = a.seqlens[b + 1] - a.seqlens[b];  // CSR: indptr
    mrow = v.mask_indptr[b] + (int64_t)tq * (ctx + L) + ctx;
  } else if (v.mode == 2) {
    mrow = (tok0 + tq) * L;
  }
  f32x4_t acc[G::DB];
#pragma unroll
  for (int db = 0; db < G::DB; ++db) acc[db] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  float m = -INFINITY, l = 0.f;
  VerifyChunk<D> c = c0;  // the first chunk's loads were issued ahead
  for (int j0 = 0; j0 < L; j0 += TILE) {
    if (j0 > 0) verify_chunk_load<D>(a, v, b, h, j0, lane, c);
#pragma unroll
    for (int i = G::KFRAGS; i < G::NI; ++i) {  // values, as the stage's V blocks
      int row, coff, dst;
      bool isk;
      load_slot<D>(i, lane, row, coff, isk, dst);
      *reinterpret_cast<u32x4_t *>(vs + (dst - G::KBYTES) + lane * 16) = c.v[i - G::KFRAGS];
    }
    f32x4_t s[2];
#pragma unroll
    for (int pb = 0; pb < 2; ++pb) {  // S^T[token 16 pb + 4 g + i][row n]
      f32x4_t sc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int t = 0; t < KT; ++t) sc = mfma_16x16x32(c.k[pb][t], qf[t], sc);
      s[pb] = sc;
    }
    float mx = -INFINITY;
#pragma unroll
    for (int pb = 0; pb < 2; ++pb)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int j = j0 + 16 * pb + 4 * g + i;
        const bool seen = j < L && (v.mode == 0 ? j <= tq : v.mask[mrow + j] != 0);
        s[pb][i] = seen ? s[pb][i] * v.scale_log2 : -INFINITY;
        mx = fmaxf(mx, s[pb][i]);
      }
    const float mn = fmaxf(m, max_over_groups(mx));
    const float alpha = mn > -INFINITY ? __builtin_amdgcn_exp2f(m - mn) : 1.f;  // 0 at the first seen token
    l *= alpha;
#pragma unroll
    for (int db = 0; db < G::DB; ++db) acc[db] *= alpha;
    float p[2][4];
#pragma unroll
    for (int pb = 0; pb < 2; ++pb)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        p[pb][i] = s[pb][i] > -INFINITY ? __builtin_amdgcn_exp2f(s[pb][i] - mn) : 0.f;
        l += p[pb][i];
      }
    m = mn;
    const u32x4_t pk = {pack_bf16x2(p[0][0], p[0][1]), pack_bf16x2(p[0][2], p[0][3]),
                        pack_bf16x2(p[1][0], p[1][1]), pack_bf16x2(p[1][2], p[1][3])};
    asm volatile("" ::: "memory");  // the value stores above precede the transposing reads
    pv_accumulate<D>(vs, pk, acc, lane);
  }
  const float lt = sum_over_groups(l);
  const float inv = lt > 0.f ? 1.f / lt : 0.f;
  const float lse = lt > 0.f ? m + log2f(lt) : -INFINITY;
  u32x2_t hp[G::DB];
  const float sc = make_partial<D>(acc, inv, hp);
  store_partial_rows<D>(a, hp, lse, sc, ((int64_t)a.batch * a.ups + a.num_shares + unit) * rows + rb * 16 + n, g);
}

// The hand-off of partials from the consumers to the producer: an LDS slot of the
// 16 W rows (D fp16 each, 16-byte chunk c of row r stored at chunk c ^ (r mod D/8), so
// that both the consumers' 8-byte writes and the producer's 16-byte reads spread over
// the banks), then (lse, scale) per row. The producer issues the global stores: a
// consumer's stores would queue behind the producer's loads in the CU's memory pipeline
// and hold every wavefront of the workgroup at the next barrier.
template <int D, int W>
struct OutSlot {
  static constexpr int ROWS = 16 * W;
  static constexpr int CH = D / 8;         // 16-byte chunks per row
  static constexpr int OBYTES = ROWS * D * 2;
  static constexpr int BYTES = OBYTES + ROWS * 8;
};

template <int D, int W>
__device__ __forceinline__ void out_write(char *slot, const u32x2_t (&h)[D / 16], float lse, float sc, int wave,
                                          int n, int g) {
  using O = OutSlot<D, W>;
  typedef __attribute__((address_space(3))) u32x2_t lds_u32x2_t;
  typedef __attribute__((address_space(3))) f32x2_t lds_f32x2_t;
  int r = wave * 16 + n;
  // Opaque to the optimizer: the addresses below are formed here, once per partial,
  // instead of being hoisted out of the tile loop and held in registers throughout it.
  asm volatile("" : "+v"(r));
#pragma unroll
  for (int db = 0; db < D / 16; ++db) {
    const int c = 2 * db + (g >> 1);
    *(lds_u32x2_t *)(slot + r * (2 * D) + ((c ^ (r & (O::CH - 1))) << 4) + 8 * (g & 1)) = h[db];
  }
  if (g == 0) *(lds_f32x2_t *)(slot + O::OBYTES + 8 * r) = f32x2_t{lse, sc};
}

template <int D, int W>
__device__ __forceinline__ void out_store(const AttnArgs &a, const char *slot, int64_t slot_idx, int lane) {
  using O = OutSlot<D, W>;
  typedef __attribute__((address_space(3))) const u32x4_t lds_u32x4_t;
  typedef __attribute__((address_space(3))) const f32x2_t lds_f32x2_t;
  typedef __attribute__((address_space(1))) char gchar;
  gchar *const base = (gchar *)a.part_o + slot_idx * O::OBYTES;
  constexpr int NK = O::ROWS * O::CH / 64, BATCH = NK % 4 == 0 ? 4 : (NK % 2 == 0 ? 2 : 1);
#pragma unroll 1
  for (int k0 = 0; k0 < NK; k0 += BATCH) {  // a few reads in flight, few registers
    u32x4_t v[BATCH];
#pragma unroll
    for (int j = 0; j < BATCH; ++j) v[j] = *(lds_u32x4_t *)(slot + 16 * ((k0 + j) * 64 + lane));
#pragma unroll
    for (int j = 0; j < BATCH; ++j) {
      const int q = (k0 + j) * 64 + lane, r = q / O::CH, p = q % O::CH;
      *(__attribute__((address_space(1))) u32x4_t *)(base + r * (2 * D) + ((p ^ (r & (O::CH - 1))) << 4)) = v[j];
    }
  }
  for (int r = lane; r < O::ROWS; r += 64)
    *reinterpret_cast<__attribute__((address_space(1))) f32x2_t *>((gfloat *)a.part_lse + 2 * (slot_idx * O::ROWS + r)) =
        *(lds_f32x2_t *)(slot + O::OBYTES + 8 * r);
}

// A partial held in the producer's registers (its share's first completed segment),
// stored after the producer's last load: partial stores interleaved with the load
// stream cost about 1 us per MB at the batch-64 workload, stores after it almost
// nothing. Only where it fits the producer's spare registers (W D <= 512).
template <int D, int W>
struct HeldPartial {
  using O = OutSlot<D, W>;
  static constexpr bool OK = W * D <= 512;
  static constexpr int NK = O::ROWS * O::CH / 64, NL = (O::ROWS + 63) / 64;
  u32x4_t v[OK ? NK : 1];
  f32x2_t ls[OK ? NL : 1];
};

template <int D, int W>
__device__ __forceinline__ void held_read(HeldPartial<D, W> &hp, const char *slot, int lane) {
  using O = OutSlot<D, W>;
  typedef __attribute__((address_space(3))) const u32x4_t lds_u32x4_t;
  typedef __attribute__((address_space(3))) const f32x2_t lds_f32x2_t;
#pragma unroll
  for (int k = 0; k < HeldPartial<D, W>::NK; ++k) hp.v[k] = *(lds_u32x4_t *)(slot + 16 * (k * 64 + lane));
#pragma unroll
  for (int j = 0; j < HeldPartial<D, W>::NL; ++j) {
    const int r = j * 64 + lane;
    hp.ls[j] = r < O::ROWS ? *(lds_f32x2_t *)(slot + O::OBYTES + 8 * r) : f32x2_t{0.f, 0.f};
  }
}

template <int D, int W>
__device__ __forceinline__ void held_store(const AttnArgs &a, const HeldPartial<D, W> &hp, int64_t slot_idx, int lane) {
  using O = OutSlot<D, W>;
  typedef __attribute__((address_space(1))) char gchar;
  gchar *const base = (gchar *)a.part_o + slot_idx * O::OBYTES;
#pragma unroll
  for (int k = 0; k < HeldPartial<D, W>::NK; ++k) {
    const int q = k * 64 + lane, r = q / O::CH, p = q % O::CH;
    *(__attribute__((address_space(1))) u32x4_t *)(base + r * (2 * D) + ((p ^ (r & (O::CH - 1))) << 4)) = hp.v[k];
  }
#pragma unroll
  for (int j = 0; j < HeldPartial<D, W>::NL; ++j) {
    const int r = j * 64 + lane;
    if (r < O::ROWS)
      *reinterpret_cast<__attribute__((address_space(1))) f32x2_t *>((gfloat *)a.part_lse + 2 * (slot_idx * O::ROWS + r)) =
          hp.ls[j];
  }
}

// LDS writes of this wavefront complete (before a barrier that publishes them).
__device__ __forceinline__ void lds_publish() { asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory"); }

// ---------------------------------------------------------------------------------
// Direct query rows (bf16 calls without verify tokens, q_len <= QTOK): the consumers read
// their rows straight from the caller's layout and apply the QK-RMSNorm + RoPE prologue
// themselves at each segment's start, with norm_rope_apply, the code the standalone
// prologue runs (the values are bit-identical to it). What the prologue reads is staged
// in LDS, so that no global load waits on the tile path:
//   - at kernel start, per sequence: its first query token row and draft rows, and the
//     rotary table row of each of its first QTOK draft tokens (positions resolved and
//     clamped), plus the norm weights;
//   - per unit, the rotary records (D floats: the table row's cos / sin of every pair) of
//     the QTOK tokens, brought into the replica's rope buffer by LDS-DMA that the consumer
//     wavefronts issue at the second tile of the previous unit's segment and await (their
//     own vmcnt) at its last tile, before the barrier that opens the unit;
//   - the next unit's raw rows, loaded into registers a unit ahead (as the packed rows
//     of the other calls are).
// A unit whose records are not in the buffer (the share's first, one after a segment of a
// single tile, or after sequences without context) reads its operands with global loads.
// The prologue runs inside the workgroup's barrier cycle (about 1.5 us per segment start
// at 64 rows x D 128, against a 1.25 us tile), so direct rows pay per segment what the
// query pass pays once per call: the host takes them for small calls only (one unit per
// two shares or fewer), where every share starts about one segment and a launch is saved.
constexpr int QTOK = 16;

template <int LAYOUT, int D, int W, bool F8, bool DQ>
__host__ __device__ constexpr int kernel_seq_cap() {
  using G = Geo<D, F8>;
  constexpr int R = replicas(W, F8, LAYOUT);
  constexpr int ring = G::SMEM * (double_tiles(W, F8, LAYOUT) ? 2 : 1);
  constexpr int fixed = R * (ring + OutSlot<D, W>::BYTES) + (DQ ? R * QTOK * D * 4 + D * 4 : 0);
  constexpr int per = 8 + (DQ ? 8 + 4 * QTOK : 0);  // (prefix, length); (first token, rows) and rope rows
  constexpr int cap = (163840 - fixed - 1024) / per - 1;
  return cap < SEQ_LDS ? cap : SEQ_LDS;
}

// Row of this lane in unit u for a direct call: draft row or not, its token within the
// sequence, and the element offset of its channel 8 g in the caller's query.
struct QRowD {
  bool ok;
  int tq;
  int64_t off;
};
__device__ __forceinline__ QRowD direct_row(const AttnArgs &a, lds_i32x2_t *qmeta, int u, int r, int g) {
  asm volatile("" : "+v"(r), "+v"(g));  // formed per call, not held across the tile loop
  const int b = u / a.ups, ul = u - b * a.ups;
  const int h = ul / a.rgroups, rg = ul - h * a.rgroups;
  const i32x2_t e = qmeta[b];  // (first token, rows)
  const int R = rg * 16 * a.nrb + r;
  const int gq = R / a.q_len, tq = R - gq * a.q_len;
  QRowD x;
  x.ok = gq < a.group && tq < e[1];
  x.tq = x.ok ? tq : 0;
  const int64_t tok = (int64_t)e[0] + x.tq;
  const int64_t head = (int64_t)h * a.group + (x.ok ? gq : 0);
  x.off = (a.cu_q ? tok * a.q_st : (int64_t)b * a.q_sb + (int64_t)x.tq * a.q_st) + head * a.q_sh + 8 * g;
  return x;
}

// The token (record index, < q_len) of this lane's row r in unit u. A row past its
// sequence's draft rows names some token too; its values are zeroed after the prologue.
__device__ __forceinline__ int direct_tq(const AttnArgs &a, int u, int r) {
  const int ul = u - (u / a.ups) * a.ups;
  const int R = (ul - (ul / a.rgroups) * a.rgroups) * 16 * a.nrb + r;
  return R - (R / a.q_len) * a.q_len;
}

__device__ __forceinline__ void direct_load_rows(const AttnArgs &a, const QRowD &x, u32x4_t (&q)[4]) {
  typedef __attribute__((address_space(1))) const u32x4_t g_u32x4_t;
  const uint16_t *src = a.q + x.off;
  if (x.ok) {
#pragma unroll
    for (int t = 0; t < 4; ++t) q[t] = *(g_u32x4_t *)(src + 32 * t);
  }
}
__device__ __forceinline__ void direct_load_rows(const AttnArgs &a, const QRowD &x, u32x4_t (&q)[2]) {
  typedef __attribute__((address_space(1))) const u32x4_t g_u32x4_t;
  const uint16_t *src = a.q + x.off;
  if (x.ok) {
#pragma unroll
    for (int t = 0; t < 2; ++t) q[t] = *(g_u32x4_t *)(src + 32 * t);
  }
}

// The rope buffer's record of token t (D floats): the table row as it lies (interleaved
// (cos, sin) pairs), or cos of the D/2 pairs then their sin (split tables). LDS-DMA of the
// QTOK records of sequence b: 16-byte chunk k of the records (k = 64 m + lane) is issued
// by wavefront m % W, so every consumer wavefront issues ceil(NCH / W) of them.
typedef __attribute__((address_space(3))) const int32_t lds_i32_t;

template <int D, int W>
__device__ __forceinline__ void rope_records_dma(const AttnArgs &a, lds_i32_t *rrow_b, char *rbuf, int wave,
                                                 int lane) {
  constexpr int CPT = D * 4 / 16;               // chunks per record
  constexpr int NI = QTOK * CPT / 64;           // 1 KB DMA instructions per unit
  constexpr int PER = (NI + W - 1) / W;         // per consumer wavefront
  const bool il = a.rope.pair_stride == 2;
  asm volatile("" : "+v"(lane));  // per-lane offsets formed here, not held across the tile loop
  // Every table row first: an LDS read after an LDS-DMA would wait for the DMA's writes.
  const float *src[PER];
#pragma unroll
  for (int p = 0; p < PER; ++p) {
    const int m = wave + p * W;
    const int k = 64 * (m < NI ? m : 0) + lane, t = k / CPT, j = k - (k / CPT) * CPT;
    const int64_t rr = rrow_b[t];
    src[p] = il || j < CPT / 2 ? a.rope.cos + rr * a.rope.row_stride + 4 * j
                               : a.rope.sin + rr * a.rope.row_stride + 4 * (j - CPT / 2);
  }
  // Issued as inline asm, outside the compiler's LDS-DMA tracking: through the builtin, the
  // compiler would make every later LDS access of this wavefront (the tile's K reads, the
  // partial's hand-off) wait for these loads, which queue behind the producer's stream.
  // The callers await them explicitly (wait_vm<0> before the barrier that publishes them).
  typedef __attribute__((address_space(3))) char lds_char_t;
#pragma unroll
  for (int p = 0; p < PER; ++p) {
    const int m = wave + p * W;
    if (m < NI) {
      const uint32_t dst = (uint32_t)(uintptr_t)(lds_char_t *)(rbuf + 1024 * m);
      asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, off"
                   :
                   : "s"(dst), "v"(src[p])
                   : "memory", "m0");
    }
  }
}

// The prologue of this lane's rows x from operands in registers: the norm weights of its
// channels (wl, wh) and its rotary values as the record layout lays them out (IL:
// interleaved (cos, sin) pairs; else cos, then sin). Each layout has its own copy of the
// arithmetic, so the loaded registers are used as they lie, with no copies.
template <int D, bool IL>
__device__ __forceinline__ void prologue_apply(u32x4_t (&x)[D / 32], const f32x4_t (&wl)[D / 32],
                                                   const f32x4_t (&wh)[D / 32], const f32x4_t (&v0)[D / 32],
                                                   const f32x4_t (&v1)[D / 32], float eps) {
  constexpr int KT = D / 32;
  PrologueOps<D> ops;
#pragma unroll
  for (int t = 0; t < KT; ++t) {
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      ops.w[t][q] = wl[t][q], ops.w[t][4 + q] = wh[t][q];
      ops.c[t][q] = IL ? (q < 2 ? v0[t][2 * q] : v1[t][2 * q - 4]) : v0[t][q];
      ops.s[t][q] = IL ? (q < 2 ? v0[t][2 * q + 1] : v1[t][2 * q - 3]) : v1[t][q];
    }
  }
  norm_rope_apply<D>(x, ops, eps);
}
// The prologue with its operands from LDS: norm weights, rotary values from record tq of
// the rope buffer.
template <int D>
__device__ __forceinline__ void prologue_lds(u32x4_t (&x)[D / 32], const float *w_lds, const char *rbuf, int tq, int g,
                                             bool il, float eps) {
  constexpr int KT = D / 32;
  typedef __attribute__((address_space(3))) const f32x4_t lds_f32x4_t;
  const float *rec = reinterpret_cast<const float *>(rbuf) + tq * D;
  PrologueOps<D> ops;
#pragma unroll
  for (int t = 0; t < KT; ++t) {
    const f32x4_t lo = *(lds_f32x4_t *)(w_lds + 32 * t + 8 * g);
    const f32x4_t hi = *(lds_f32x4_t *)(w_lds + 32 * t + 8 * g + 4);
#pragma unroll
    for (int q = 0; q < 4; ++q) ops.w[t][q] = lo[q], ops.w[t][4 + q] = hi[q];
    if (il) {  // interleaved records: the lane's pairs lie together
      const f32x4_t v0 = *(lds_f32x4_t *)(rec + 32 * t + 8 * g);
      const f32x4_t v1 = *(lds_f32x4_t *)(rec + 32 * t + 8 * g + 4);
      ops.c[t][0] = v0[0], ops.s[t][0] = v0[1], ops.c[t][1] = v0[2], ops.s[t][1] = v0[3];
      ops.c[t][2] = v1[0], ops.s[t][2] = v1[1], ops.c[t][3] = v1[2], ops.s[t][3] = v1[3];
    } else {  // split records: cos, then sin at D / 2
      const f32x4_t cv = *(lds_f32x4_t *)(rec + 16 * t + 4 * g);
      const f32x4_t sv = *(lds_f32x4_t *)(rec + D / 2 + 16 * t + 4 * g);
#pragma unroll
      for (int q = 0; q < 4; ++q) ops.c[t][q] = cv[q], ops.s[t][q] = sv[q];
    }
  }
  norm_rope_apply<D>(x, ops, eps);
}

// The same prologue with the rotary values read from the table in global memory (the
// units whose records are not in the rope buffer). Only the two table layouts the direct
// calls admit (split or interleaved (cos, sin) rows): 16-byte loads of the lane's pairs,
// issued together with the weights' LDS reads.
template <int D>
__device__ __forceinline__ void prologue_global(u32x4_t (&x)[D / 32], const AttnArgs &a, const float *w_lds,
                                                int64_t rr, int g, bool il) {
  constexpr int KT = D / 32;
  typedef __attribute__((address_space(3))) const f32x4_t lds_f32x4_t;
  asm volatile("" : "+v"(g), "+v"(rr));  // per-lane addresses formed here, not held across the tile loop
  const float *row_c = a.rope.cos + rr * a.rope.row_stride, *row_s = a.rope.sin + rr * a.rope.row_stride;
  f32x4_t wl[KT], wh[KT], v0[KT], v1[KT];
#pragma unroll
  for (int t = 0; t < KT; ++t) {
    const f32x4u_t c0 = *(g_f32x4u_t *)(il ? row_c + 32 * t + 8 * g : row_c + 16 * t + 4 * g);
    const f32x4u_t c1 = *(g_f32x4u_t *)(il ? row_c + 32 * t + 8 * g + 4 : row_s + 16 * t + 4 * g);
    v0[t] = f32x4_t{c0[0], c0[1], c0[2], c0[3]};
    v1[t] = f32x4_t{c1[0], c1[1], c1[2], c1[3]};
    wl[t] = *(lds_f32x4_t *)(w_lds + 32 * t + 8 * g);
    wh[t] = *(lds_f32x4_t *)(w_lds + 32 * t + 8 * g + 4);
  }
  if (il) {
    prologue_apply<D, true>(x, wl, wh, v0, v1, a.eps);
  } else {
    prologue_apply<D, false>(x, wl, wh, v0, v1, a.eps);
  }
}

// e4m3 query rows from the prologue's bf16 rows, as the query pass makes them (lane (n, g)
// holds channels 32 t + 8 g .. + 7 of row n, the wavefront's 16 rows being one query head's
// draft tokens): the head's scale max(amax, 1e-12) / 448 over the 16 rows, every value
// divided by it (correctly rounded) and rounded to e4m3 (torch's (q / scale).to(e4m3)),
// then moved across the row's four lanes into the fp8 MFMA operand layout: fragment f of
// lane (n, g) holds channels 64 f + 16 g .. + 15. Word s of that fragment is chunk
// c = 8 f + 2 g + s / 2 (8 channels), which the row-quad layout keeps in lane (n, c % 4),
// register c / 4 = 2 f + g / 2, word s % 2. Returns the scale.
template <int D>
__device__ __forceinline__ float quantize_query_rows(const u32x4_t (&x)[D / 32], u32x4_t (&qf)[D / 64], int n,
                                                     int g) {
  constexpr int KT = D / 32;
  float mx = 0.f;
#pragma unroll
  for (int t = 0; t < KT; ++t)
#pragma unroll
    for (int q = 0; q < 4; ++q) mx = fmaxf(mx, fmaxf(fabsf(bf16_lo(x[t][q])), fabsf(bf16_hi(x[t][q]))));
#pragma unroll
  for (int o = 1; o < 16; o <<= 1) mx = fmaxf(mx, __shfl_xor(mx, o));
  mx = max_over_groups(mx);
  const float scale = __fdiv_rn(fmaxf(mx, 1e-12f), 448.f);
  u32x2_t q8[KT];
#pragma unroll
  for (int t = 0; t < KT; ++t) {
    float v[8];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      v[2 * q] = __fdiv_rn(bf16_lo(x[t][q]), scale);
      v[2 * q + 1] = __fdiv_rn(bf16_hi(x[t][q]), scale);
    }
    q8[t] = u32x2_t{pack_e4m3x4(v[0], v[1], v[2], v[3]), pack_e4m3x4(v[4], v[5], v[6], v[7])};
  }
  const bool upper = (g >> 1) != 0;  // lanes of groups 2, 3 take register 2 f + 1
#pragma unroll
  for (int f = 0; f < D / 64; ++f) {
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      const int src = n + 16 * ((2 * g + (w >> 1)) & 3);
      const int lo = __shfl((int)q8[2 * f][w & 1], src);
      const int hi = __shfl((int)q8[2 * f + 1][w & 1], src);
      qf[f][w] = (uint32_t)(upper ? hi : lo);
    }
  }
  return scale;
}

// One workgroup = R replicas x (W consumer wavefronts + 1 producer wavefront).
//
// The producer issues every load of its replica's K/V stream (LDS-DMA into the ring, plus
// the page ids with paged layouts), alone waits on vmcnt, with counts fixed by
// construction, and stores the partials the consumers hand over through LDS. The
// consumers read LDS, compute and load their query rows a unit ahead. One barrier per
// tile hands stage i from the producer (its loads complete) to the consumers and stage
// i-1 back (their reads of it done), and a partial written in iteration t to the
// producer, who stores it in iteration t + 1.
template <int LAYOUT, int W, int D, bool F8 = false, bool DQ = false>
__global__ __launch_bounds__(64 * (W + 1) * replicas(W, F8, LAYOUT)) void attn_fwd_kernel(
    const AttnArgs a, const int32_t *__restrict__ table, const int32_t *__restrict__ plan,
    const int32_t *__restrict__ seqlens) {
  using G = Geo<D, F8>;
  using O = OutSlot<D, W>;
  constexpr int QF = G::KC;                // 16-byte query fragments per lane
  constexpr int UNIT_Q = 16 * W * G::RB;   // bytes of a unit's packed query rows
  constexpr bool IDS = LAYOUT != CONTIG;  // page ids join the load stream
  constexpr int R = replicas(W, F8, LAYOUT);
  constexpr int S = G::NS;
  constexpr bool DBL = double_tiles(W, F8, LAYOUT);  // two 32-position stages per line tile
  constexpr int SUB = DBL ? 2 : 1;
  constexpr int TL = SUB * G::T;                 // positions per line tile
  constexpr int SLOT = SUB * G::STAGE;           // bytes per ring slot
  constexpr int GN = SUB * G::NI, GI = SUB;      // loads and page-id loads per line tile
  constexpr int RBYTES = S * SLOT + O::BYTES;    // per replica: the ring, then the out slot
  constexpr int SEQ = kernel_seq_cap<LAYOUT, D, W, F8, DQ>();  // sequences whose metadata is staged in LDS
  constexpr int RBUF = QTOK * D * 4;                  // DQ: a replica's rope buffer
  static_assert(S >= 3, "the wait schedule keeps one group between tiles");
  static_assert((S - 2) * GN + (S - 2) * GI < 64, "vmcnt holds 6 bits");
  static_assert(SEQ >= 1, "LDS budget");
  __shared__ __attribute__((aligned(1024))) char smem_all[R * RBYTES];
  __shared__ i32x2_t seq_tab[SEQ + 1];
  // DQ: the replicas' rope buffers, the norm weights, (first token, rows) and the rotary
  // table rows of the first QTOK draft tokens of each sequence.
  __shared__ __attribute__((aligned(16))) char dq_lds[DQ ? R * RBUF + D * 4 + SEQ * (8 + 4 * QTOK) : 16];
  char *const rope_bufs = dq_lds;
  float *const w_tab = reinterpret_cast<float *>(dq_lds + R * RBUF);
  i32x2_t *const qmeta = reinterpret_cast<i32x2_t *>(dq_lds + R * RBUF + D * 4);
  int32_t *const rrow = reinterpret_cast<int32_t *>(dq_lds + R * RBUF + D * 4 + SEQ * 8);
  SeqMeta<LAYOUT != CONTIG> sm{plan, seqlens, (lds_i32x2_t *)seq_tab, false};
  const bool stage_seq = sm.var() && a.batch <= SEQ;
  if (stage_seq || DQ) {  // uniform: every wavefront takes the barrier (DQ calls have batch <= SEQ)
    // Every load of a thread's entries issued before any is used, two entries per pass
    // (a DQ call's batch x QTOK rotary rows take two passes of the workgroup at batch 64):
    // the staging costs one round trip to memory per pass, two with explicit query
    // positions (token row, then position).
    const bool pro = DQ && a.qn_w != nullptr;
    auto wanted = [&](int j) { return j <= a.batch || (pro && (j < a.batch * QTOK || j < D)); };
    constexpr int NJ = 2;
    for (int j0 = threadIdx.x; wanted(j0); j0 += NJ * blockDim.x) {
      int32_t p0[NJ], len[NJ], c0[NJ], c1[NJ], b0[NJ], b1[NJ];
      float wj[NJ];
#pragma unroll
      for (int k = 0; k < NJ; ++k) {
        const int j = j0 + k * (int)blockDim.x;
        const int bb = j / QTOK;
        p0[k] = 0, len[k] = 0, c0[k] = j * a.q_len, c1[k] = (j + 1) * a.q_len, b0[k] = 0, b1[k] = 0, wj[k] = 0.f;
        if (stage_seq && j <= a.batch) p0[k] = plan[j], len[k] = j < a.batch || a.csr ? seqlens[j] : 0;  // CSR: indptr[j]
        if (DQ && j < a.batch && a.cu_q) c0[k] = a.cu_q[j], c1[k] = a.cu_q[j + 1];
        if (pro && j < D) wj[k] = a.qn_w[j];
        if (pro && j < a.batch * QTOK) {
          b0[k] = a.cu_q ? a.cu_q[bb] : bb * a.q_len;
          b1[k] = a.cu_q ? a.cu_q[bb + 1] : (bb + 1) * a.q_len;
        }
      }
      int64_t pos[NJ];
#pragma unroll
      for (int k = 0; k < NJ; ++k) {
        const int j = j0 + k * (int)blockDim.x;
        const int tt = j - (j / QTOK) * QTOK;
        const int64_t tok = (int64_t)b0[k] + tt;
        pos[k] = 0;
        if (pro && j < a.batch * QTOK && tt < b1[k] - b0[k]) pos[k] = a.q_pos ? a.q_pos[tok] : tok;
      }
#pragma unroll
      for (int k = 0; k < NJ; ++k) {
        const int j = j0 + k * (int)blockDim.x;
        if (stage_seq && j <= a.batch) seq_tab[j] = i32x2_t{p0[k], len[k]};
        if constexpr (DQ) {
          if (j < a.batch) {
            int32_t rows = c1[k] - c0[k];
            rows = rows < 0 ? 0 : (rows > a.q_len ? a.q_len : rows);
            qmeta[j] = i32x2_t{c0[k], rows};
          }
          if (pro && j < D) w_tab[j] = wj[k];
          if (pro && j < a.batch * QTOK) rrow[j] = (int32_t)clamp_row(a.rope, pos[k]);
        }
      }
    }
    lds_publish();
    block_sync();
    sm.staged = stage_seq;
  }
  const int lane = threadIdx.x & 63, wv = wave_id();
  const int rep = wv / (W + 1), wave = wv - rep * (W + 1);  // replica; W = the producer
  __builtin_assume(wave >= 0 && wave <= W && rep >= 0 && rep < R);
  const int n = lane & 15, g = lane >> 4;
  char *const smem = smem_all + rep * RBYTES;
  char *const out = smem + S * SLOT;
  const int share = (int)blockIdx.x * R + rep;
  int64_t F[R + 1];  // first tiles of the workgroup's shares and the next one
  share_first_tiles(a, sm, (int64_t)blockIdx.x * R, F);
  int64_t T0 = F[0];
  int ntiles = 0;
  // Iterations of the workgroup: the largest share among its replicas (every wavefront
  // takes part in every barrier; a replica past its share only waits at them).
  int nloop = 0;
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int nr = (int)(F[r + 1] - F[r]);
    nloop = nr > nloop ? nr : nloop;
    if (r == rep) T0 = F[r], ntiles = nr;
  }
  Cursor cc = Cursor{0, 0, 0, 0, 0, 0, 0, 0};  // tile being computed (i)
  if (ntiles > 0) cc = cursor_at(a, sm, T0);
  auto stage = [&](int t) { return smem + (t % S) * SLOT; };
  // A segment ends at tile t when t is its unit's last or the share's last tile. Its
  // partial goes through the out slot unless tile t - 1 ended one too (the slot may
  // still be read then); the consumers then store it themselves.

  if (wave == W) {
    // ------------------------------------------------------------------ producer
    // Issue order: K/V of tile t (NI loads) at iteration t - (S - 1) and, with paged
    // layouts, the page ids of tile t + S - 1 right before them, so that the wait for
    // tile i's group also completes the ids that the loads of tile i + S - 1 read.
    // Partial stores only ever make a wait more conservative (stores complete out of
    // order with loads; loads among themselves in order).
    uint32_t loff[G::NI];  // byte offsets inside a half tile of this lane's loads
#pragma unroll
    for (int i = 0; i < G::NI; ++i) {
      int row, coff, dst;
      bool isk;
      load_slot<D, F8>(i, lane, row, coff, isk, dst);
      loff[i] = (uint32_t)(row & 15) * (isk ? a.k_tok_b : a.v_tok_b) + (uint32_t)coff;
    }
    Loader ld;  // next tile to load (i + S - 1)
    ld.c = cc;
    if (ntiles > 0) loader_unit<LAYOUT, G::ES>(a, ld);
    Cursor ct = cc;  // paged layouts: next tile whose page ids are loaded
    Cursor pc = cc;  // the tile whose partial (if any) is stored next
    bool pc_prev_end = false;
    HeldPartial<D, W> held;
    int64_t held_slot = -1;  // >= 0: a partial is held for the end
    // A line tile's page ids and K/V loads: with double tiles, its two 32-position stages
    // (the cursor's tile index counted in 32-position tiles for them).
    auto ids_of = [&](const Cursor &c, char *st) {
      if constexpr (DBL) {
        Cursor c2 = c;
        c2.lt = 2 * c.lt;
        issue_ids<LAYOUT, D, F8>(a, table, c2, st, lane);
        c2.lt += 1;
        issue_ids<LAYOUT, D, F8>(a, table, c2, st + G::STAGE, lane);
      } else {
        issue_ids<LAYOUT, D, F8>(a, table, c, st, lane);
      }
    };
    auto kv_of = [&](char *st) {
      if constexpr (DBL) {
        Loader l2 = ld;
        l2.c.lt = 2 * ld.c.lt;
        issue_kv<LAYOUT, D, 1, F8, krow<LAYOUT, D, F8, W>()>(a, l2, st, 0, lane, loff);
        l2.c.lt += 1;
        issue_kv<LAYOUT, D, 1, F8, krow<LAYOUT, D, F8, W>()>(a, l2, st + G::STAGE, 0, lane, loff);
      } else {
        issue_kv<LAYOUT, D, 1, F8, krow<LAYOUT, D, F8, W>()>(a, ld, st, 0, lane, loff);
      }
    };
    auto handoff = [&](int t) {  // after the barrier that follows tile t
      const bool end = pc.lt == pc.tiles - 1 || t == ntiles - 1;
      if (end && !pc_prev_end) {
        if (HeldPartial<D, W>::OK && held_slot < 0 && t < ntiles - 1) {
          held_read<D, W>(held, out, lane);
          held_slot = (int64_t)pc.u + share;
        } else {
          out_store<D, W>(a, out, (int64_t)pc.u + share, lane);
        }
      }
      pc_prev_end = end;
      if (t + 1 < ntiles) cursor_next(a, sm, pc);
    };
    if (IDS) {
      for (int j = 0; j < S && j < ntiles; ++j) {
        ids_of(ct, stage(j));
        if (j + 1 < ntiles) cursor_next(a, sm, ct);
      }
      wait_vm<0>();
    }
    for (int j = 0; j < S - 1 && j < ntiles; ++j) {
      kv_of(stage(j));
      if (j + 1 < ntiles) loader_advance<LAYOUT, G::ES>(a, sm, ld);
      if (IDS && j + S <= 2 * S - 3 && j + S < ntiles) {
        ids_of(ct, stage(j + S));
        cursor_next(a, sm, ct);
      }
    }
    for (int i = 0; i < nloop; ++i) {
      // Tile i's group is complete once only what was issued after it may be
      // outstanding: the groups of tiles i+1 .. i+S-2 and (paged layouts) the page ids
      // of tiles i+S .. i+2S-3.
      if (i < ntiles) {
        const int later = ntiles - 1 - i;
        if (IDS && later >= 2 * S - 3) {
          wait_vm<(GN + GI) * (S - 2)>();
        } else if (IDS) {
          int nwait = GN * (later < S - 2 ? later : S - 2);
          const int ids = later - (S - 1);  // tiles at or after i + S
          nwait += GI * (ids <= 0 ? 0 : (ids < S - 2 ? ids : S - 2));
          wait_vm(nwait);
        } else if (later >= S - 2) {
          wait_vm<GN *(S - 2)>();
        } else if (S > 3 && later == 1) {
          wait_vm<GN>();
        } else {
          wait_vm<0>();
        }
      }
      block_sync();
      if (i >= 1 && i - 1 < ntiles) handoff(i - 1);
      if (i >= ntiles) continue;
      if (i + S - 1 < ntiles) {
        if (IDS && i + 2 * S - 2 < ntiles) {
          ids_of(ct, stage(i + 2 * S - 2));
          cursor_next(a, sm, ct);
        }
        kv_of(stage(i + S - 1));
        if (i + S < ntiles) loader_advance<LAYOUT, G::ES>(a, sm, ld);
      }
    }
    block_sync();
    if (ntiles > 0 && ntiles == nloop) handoff(ntiles - 1);
    if (HeldPartial<D, W>::OK && held_slot >= 0) held_store<D, W>(a, held, held_slot, lane);
    return;
  }

  // ------------------------------------------------------------------- consumers
  typedef __attribute__((address_space(1))) const u32x4_t g_u32x4_t;
  const char *qbase = reinterpret_cast<const char *>(a.qp) + (wave * 16 + n) * G::RB + 16 * g;
  auto qsrc = [&](int u) { return qbase + (uint64_t)(uint32_t)u * UNIT_Q; };
  // F8: the rows' score scales (query descale x key descale), loaded with the rows.
  typedef __attribute__((address_space(1))) const float g_float_t;
  auto qscale = [&](int u) { return *(g_float_t *)(a.q_rs + (int64_t)u * (16 * W) + wave * 16 + n); };
  // Query rows of the next unit are loaded into qn as soon as the current unit's are
  // taken (the first unit's before the producer's first loads are queued ahead of
  // them), so their latency hides behind a whole unit. The next unit on the line is
  // u + 1 unless sequences without context lie between; then the rows are loaded when
  // the unit starts.
  const int units = a.batch * a.ups;
  int qn_unit = -1;
  constexpr int QB = DQ ? D / 32 : QF;  // a lane's 16-byte registers of its query row as loaded
  u32x4_t qn[QB], qf[QF];
  float rsn = 1.f, sl = a.scale_log2;
  // F8 direct rows: the key descale of a unit's (sequence, KV head), loaded with its rows
  auto kdesc = [&](int u) {
    if (!F8 || a.kd == nullptr) return 1.f;
    const int b = u / a.ups, h = (u - b * a.ups) / a.rgroups;
    return *(g_float_t *)(a.kd + (int64_t)b * a.d_sb + (int64_t)h * a.d_sh);
  };
  if (!DQ && ntiles > 0) {
#pragma unroll
    for (int t = 0; t < QF; ++t) qn[t] = *(g_u32x4_t *)(qsrc(cc.u) + 64 * t);
    if (F8) rsn = qscale(cc.u);
    qn_unit = cc.u;
  }
  // DQ: this replica's rope buffer; rb_unit: the unit whose records it holds (complete),
  // dma_unit: the unit whose records this segment brings in (its DMA issued at the
  // segment's second tile, awaited at its last).
  char *const rbuf = rope_bufs + rep * RBUF;
  const bool il = a.rope.pair_stride == 2;
  int rb_unit = -1, dma_unit = -1;
  bool dma_issued = false;
  bool qn_ok = false;
  if constexpr (DQ) {
    if (ntiles > 0) {  // the first unit: its rows, and its records before the first barrier
      if (a.qn_w != nullptr) {
        rope_records_dma<D, W>(a, (lds_i32_t *)rrow + (cc.u / a.ups) * QTOK, rbuf, wave, lane);
        rb_unit = cc.u;
      }
      const QRowD x = direct_row(a, (lds_i32x2_t *)qmeta, cc.u, wave * 16 + n, g);
      direct_load_rows(a, x, qn);
      if (F8) rsn = kdesc(cc.u);
      qn_ok = x.ok;
      qn_unit = cc.u;
      wait_vm<0>();
    }
  }
  f32x4_t acc[G::DB];
  float m = -INFINITY, l = 0.f;
  bool prev_end = false;
  for (int i = 0; i < nloop; ++i) {
    block_sync();
    if (i >= ntiles) continue;
    if constexpr (DQ) {
    if (i == 0 || cc.lt == 0) {  // a segment starts: its query rows, prologue applied
      bool ok = qn_ok;
      int tq = 0;
      u32x4_t xr[QB];  // the rows as loaded (bf16)
      float kd = rsn;
      if (qn_unit == cc.u) {
#pragma unroll
        for (int t = 0; t < QB; ++t) xr[t] = qn[t];
        tq = direct_tq(a, cc.u, wave * 16 + n);
      } else {
        const QRowD x = direct_row(a, (lds_i32x2_t *)qmeta, cc.u, wave * 16 + n, g);
        direct_load_rows(a, x, xr);
        if (F8) kd = kdesc(cc.u);
        ok = x.ok;
        tq = x.tq;
      }
#pragma unroll
      for (int t = 0; t < QB; ++t) {
        asm volatile("" : "+v"(xr[t]));
        qn[t] = u32x4_t{0, 0, 0, 0};  // consumed: no registers held for it through the prologue
      }
      if (a.qn_w != nullptr) {
        if (rb_unit == cc.u) {
          prologue_lds<D>(xr, w_tab, rbuf, tq, g, il, a.eps);
        } else {
          const int b = cc.u / a.ups;
          prologue_global<D>(xr, a, w_tab, ((lds_i32_t *)rrow)[b * QTOK + tq], g, il);
        }
      }
#pragma unroll
      for (int t = 0; t < QB; ++t)
        if (!ok) xr[t] = u32x4_t{0, 0, 0, 0};
      if constexpr (F8) {  // e4m3 rows per (sequence, query head), as the query pass makes them
        sl = a.scale_log2 * (quantize_query_rows<D>(xr, qf, n, g) * kd);
      } else {
#pragma unroll
        for (int t = 0; t < QF; ++t) qf[t] = xr[t];
      }
      rb_unit = -1;
      qn_unit = -1;
      dma_unit = -1;
      dma_issued = false;
      if (cc.u + 1 < units && cc.lt + ntiles - i > cc.tiles) {  // the share reaches unit u + 1
        const QRowD x = direct_row(a, (lds_i32x2_t *)qmeta, cc.u + 1, wave * 16 + n, g);
        direct_load_rows(a, x, qn);
        if (F8) rsn = kdesc(cc.u + 1);
        qn_ok = x.ok;
        qn_unit = cc.u + 1;
        if (a.qn_w != nullptr) dma_unit = cc.u + 1;
      }
#pragma unroll
      for (int db = 0; db < G::DB; ++db) acc[db] = f32x4_t{0.f, 0.f, 0.f, 0.f};
      m = -INFINITY;
      l = 0.f;
    } else if (dma_unit >= 0 && !dma_issued) {
      // Second tile of the segment: every wavefront is past the buffer's reads of the
      // segment's start (the barrier above), so the next unit's records may come in.
      rope_records_dma<D, W>(a, (lds_i32_t *)rrow + (dma_unit / a.ups) * QTOK, rbuf, wave, lane);
      dma_issued = true;
    }
    } else {
    if (i == 0 || cc.lt == 0) {  // a segment starts: its query rows
      if (qn_unit == cc.u) {
#pragma unroll
        for (int t = 0; t < QF; ++t) qf[t] = qn[t];
        if (F8) sl = a.scale_log2 * rsn;
      } else {
#pragma unroll
        for (int t = 0; t < QF; ++t) qf[t] = *(g_u32x4_t *)(qsrc(cc.u) + 64 * t);
        if (F8) sl = a.scale_log2 * qscale(cc.u);
      }
#pragma unroll
      for (int t = 0; t < QF; ++t) asm volatile("" : "+v"(qf[t]));
      qn_unit = -1;
      if (cc.u + 1 < units && cc.lt + ntiles - i > cc.tiles) {  // the share reaches unit u + 1
#pragma unroll
        for (int t = 0; t < QF; ++t) qn[t] = *(g_u32x4_t *)(qsrc(cc.u + 1) + 64 * t);
        if (F8) rsn = qscale(cc.u + 1);
        qn_unit = cc.u + 1;
      }
#pragma unroll
      for (int db = 0; db < G::DB; ++db) acc[db] = f32x4_t{0.f, 0.f, 0.f, 0.f};
      m = -INFINITY;
      l = 0.f;
    }
    }
    compute_tile<D, F8, krow<LAYOUT, D, F8, W>()>(a, stage(i), qf, sl, acc, m, l, cc.lt * TL, cc.L, lane);
    if constexpr (DBL) {  // the line tile's second 32 positions, where the sequence reaches them
      if (cc.lt * TL + G::T < cc.L)
        compute_tile<D, F8, krow<LAYOUT, D, F8, W>()>(a, stage(i) + G::STAGE, qf, sl, acc, m, l,
                                                      cc.lt * TL + G::T, cc.L, lane);
    }
    const bool end = cc.lt == cc.tiles - 1 || i == ntiles - 1;
    if (DQ && end && dma_issued) {
      // The next unit's records in place before the barrier that opens it (this
      // wavefront's own loads: the rows prefetched, then the records' DMA).
      wait_vm<0>();
      rb_unit = dma_unit;
    }
    if (end) {  // the segment ends: its partial
      const float lt_sum = sum_over_groups(l);
      const float inv = lt_sum > 0.f ? 1.f / lt_sum : 0.f;
      const float lse = m + log2f(lt_sum);
      u32x2_t h[G::DB];
      const float sc = make_partial<D>(acc, inv, h);
      if (!prev_end) {
        out_write<D, W>(out, h, lse, sc, wave, n, g);
        lds_publish();
      } else {
        store_partial_rows<D>(a, h, lse, sc, ((int64_t)cc.u + share) * (16 * W) + wave * 16 + n, g);
      }
    }
    prev_end = end;
    if (i + 1 < ntiles) cursor_next(a, sm, cc);
  }
  block_sync();
}

// Small calls: a few units split over many shares (one sequence at batch 1, a handful at
// most), whose whole K/V fits one pass of workgroups over the CUs. One workgroup per share
// of at most SMALL_TILES tiles (the host sizes shares to about one per CU), W consumer
// wavefronts (one per 16-row block of the unit) and one loader wavefront, no ring: the
// loader issues the share's page ids, then every K/V load of the share at once into
// stages of their own (the persistent kernel's stage layout), and publishes each tile
// with a barrier as its loads complete. The consumers meanwhile load the first segment's
// query rows and apply the prologue (their own memory queue, so its dependent loads --
// positions, then rotary rows -- are not ordered behind the K/V stream), then compute the
// tiles in order. A share of several units loads each further unit's query rows at its
// segment start. The same line of tiles, shares and partial slots as attn_fwd_kernel;
// attn_merge_wide_kernel merges the partials.
constexpr int SMALL_TILES = 8;  // stages per workgroup: 8 x 17.2 KB of LDS at head_dim 128

template <int D>
__device__ __forceinline__ void small_query_rows(const AttnArgs &a, int64_t unit, int r, int g,
                                                 u32x4_t (&qf)[D / 32]) {
  constexpr int KT = D / 32;
  const int b = (int)(unit / a.ups);
  const int ul = (int)(unit - (int64_t)b * a.ups);
  const int h = ul / a.rgroups, rg = ul - h * a.rgroups;
  const int R = rg * 16 * a.nrb + r;
  const int gq = R / a.q_len, tq = R - gq * a.q_len;
  const bool valid = gq < a.group && tq < q_rows_of(a, b);
  const int64_t tok = q_token_index(a, b, valid ? tq : 0);
  const int64_t head = (int64_t)h * a.group + (valid ? gq : 0);
  const uint16_t *src = a.q + (a.cu_q ? tok * a.q_st : (int64_t)b * a.q_sb + (int64_t)(valid ? tq : 0) * a.q_st) +
                        head * a.q_sh + 8 * g;
  query_row_any<D>(a, qf, src, valid, tok, g);
#pragma unroll
  for (int t = 0; t < KT; ++t)
    if (!valid) qf[t] = u32x4_t{0, 0, 0, 0};
}

template <int LAYOUT, int W, int D>
__global__ __launch_bounds__(64 * (W + 1)) void attn_small_kernel(const AttnArgs a,
                                                                  const int32_t *__restrict__ table,
                                                                  const int32_t *__restrict__ plan,
                                                                  const int32_t *__restrict__ seqlens) {
  using G = Geo<D>;
  constexpr bool IDS = LAYOUT != CONTIG;
  __shared__ __attribute__((aligned(1024))) char stages[SMALL_TILES * G::STAGE];
  const int lane = threadIdx.x & 63, wave = wave_id();
  const int n = lane & 15, g = lane >> 4;
  SeqMeta<LAYOUT != CONTIG> sm{plan, seqlens, nullptr, false};
  const int share = (int)blockIdx.x;
  int64_t F[2];
  share_first_tiles(a, sm, (int64_t)share, F);
  const int64_t T0 = F[0];
  const int ntiles = (int)(F[1] - F[0]);
  if (ntiles <= 0) return;  // uniform over the workgroup
  auto stage = [&](int t) { return stages + (t % SMALL_TILES) * G::STAGE; };
  Cursor cc = cursor_at(a, sm, T0);
  // Both roles take the same barriers: per chunk of SMALL_TILES tiles (a share longer than
  // that only with lengths past max_seqlen_k), one before its stages are reloaded (not
  // for the first) and one per tile as it lands.
  if (wave == W) {  // ---------------------------------------------------------- loader
    uint32_t loff[G::NI];  // byte offsets inside a 16-position block of this lane's loads
#pragma unroll
    for (int i = 0; i < G::NI; ++i) {
      int row, coff, dst;
      bool isk;
      load_slot<D>(i, lane, row, coff, isk, dst);
      loff[i] = (uint32_t)(row & 15) * (isk ? a.k_tok_b : a.v_tok_b) + (uint32_t)coff;
    }
    Cursor ct = cc;  // paged layouts: the next tile whose page ids are loaded
    Loader ld;       // the next tile whose K/V are loaded
    ld.c = cc;
    loader_unit<LAYOUT>(a, ld);
    for (int c0 = 0; c0 < ntiles; c0 += SMALL_TILES) {
      const int c1 = ntiles - c0 < SMALL_TILES ? ntiles : c0 + SMALL_TILES;
      if (c0 > 0) block_sync();  // the consumers are done with the stages being reloaded
      if (IDS) {  // the chunk's page ids, which the K/V loads below read from LDS
        for (int j = c0; j < c1; ++j) {
          issue_ids<LAYOUT, D>(a, table, ct, stage(j), lane);
          if (j + 1 < ntiles) cursor_next(a, sm, ct);
        }
        wait_vm<0>();
        asm volatile("" ::: "memory");  // the id reads stay after the wait
      }
      for (int j = c0; j < c1; ++j) {
        issue_kv<LAYOUT, D, 1>(a, ld, stage(j), 0, lane, loff);
        if (j + 1 < ntiles) loader_advance<LAYOUT>(a, sm, ld);
      }
      for (int j = c0; j < c1; ++j) {  // tile j lands: its loads and all before are complete
        wait_vm((c1 - 1 - j) * G::NI);
        block_sync();
      }
    }
    return;
  }
  // ---------------------------------------------------------------------- consumers
  const int r = wave * 16 + n;
  u32x4_t qf[G::KT];
  small_query_rows<D>(a, cc.u, r, g, qf);  // while the loader's tiles fly
  f32x4_t acc[G::DB];
  float m = -INFINITY, l = 0.f;
  for (int c0 = 0; c0 < ntiles; c0 += SMALL_TILES) {
    const int c1 = ntiles - c0 < SMALL_TILES ? ntiles : c0 + SMALL_TILES;
    if (c0 > 0) block_sync();
    for (int i = c0; i < c1; ++i) {
      block_sync();  // tile i has landed
      if (i == 0 || cc.lt == 0) {  // a segment starts: a fresh accumulator (rows of a further unit)
        if (i > 0) small_query_rows<D>(a, cc.u, r, g, qf);
#pragma unroll
        for (int db = 0; db < G::DB; ++db) acc[db] = f32x4_t{0.f, 0.f, 0.f, 0.f};
        m = -INFINITY;
        l = 0.f;
      }
      compute_tile<D, false>(a, stage(i), qf, a.scale_log2, acc, m, l, cc.lt * G::T, cc.L, lane);
      if (cc.lt == cc.tiles - 1 || i == ntiles - 1) {  // the segment ends: its partial
        const float lt_sum = sum_over_groups(l);
        const float inv = lt_sum > 0.f ? 1.f / lt_sum : 0.f;
        const float lse = m + log2f(lt_sum);
        u32x2_t h[G::DB];
        const float sc = make_partial<D>(acc, inv, h);
        store_partial_rows<D>(a, h, lse, sc, ((int64_t)cc.u + share) * (16 * W) + r, g);
      }
      if (i + 1 < ntiles) cursor_next(a, sm, cc);
    }
  }
}

// Running log2-domain LSE merge of one thread's 8 channels of an output row: acc and den
// are the segments' values and softmax masses, both relative to exp2(M).
struct RowMerge {
  f32x4_t acc[2] = {{0.f, 0.f, 0.f, 0.f}, {0.f, 0.f, 0.f, 0.f}};
  float M = -INFINITY, den = 0.f;
  // A segment whose values xs * x and mass d are relative to exp2(mseg) (finite).
  __device__ __forceinline__ void add(float mseg, float xs, float d, const f32x4_t (&x)[2]) {
    const float Mn = fmaxf(M, mseg);
    const float fo = __builtin_amdgcn_exp2f(M - Mn), fn = __builtin_amdgcn_exp2f(mseg - Mn);
    const float fx = fn * xs;
#pragma unroll
    for (int j = 0; j < 2; ++j) acc[j] = acc[j] * fo + x[j] * fx;
    den = den * fo + d * fn;
    M = Mn;
  }
  __device__ __forceinline__ void finish() {
    const float inv = den > 0.f ? 1.f / den : 0.f;
    acc[0] *= inv;
    acc[1] *= inv;
  }
};

// Adds the partials of row r of unit (b, ul) -- one per share its tiles fell to, in
// slots unit + w -- each a normalized output with its LSE, values scaled by vs. The
// segments go in batches of MB whose loads are all issued before any is used (one
// memory round trip per batch: the loop's trip count is not known at compile time, so
// the loads are gathered into registers explicitly), each batch merged relative to its
// own largest LSE and then into the running merge. MB = 8 takes about three times the
// registers of MB = 2 (121 against 42 VGPRs at D 128), which halves the combine's
// occupancy: the host picks the smallest MB of 2, 4 and 8 that holds a unit's average
// segment count.
template <int D, int MB>
__device__ __forceinline__ void merge_partials(const AttnArgs &a, int64_t unit, int b, int ul, int r, int c,
                                               float vs, RowMerge &mg) {
  typedef __attribute__((ext_vector_type(2))) float f32x2_t;
  const int rows = a.nrb * 16;
  const int64_t pre = tile_prefix(a, a.plan, b);
  const int tiles_b = (int)(tile_prefix(a, a.plan, b + 1) - pre);
  if (tiles_b <= 0) return;
  const int64_t uc = a.share_c;  // a unit's extra cost on the line (share_first_tiles)
  const int64_t total = (int64_t)a.ups * (tile_prefix(a, a.plan, a.batch) + uc * a.batch);  // the cost line
  const int64_t nw = a.num_shares;
  const int64_t U0 = (int64_t)a.ups * (pre + uc * b) + (int64_t)ul * (tiles_b + uc) + uc;  // cost of tile 0
  const int64_t wa = share_of(U0, total, nw);
  const int nseg = (int)(share_of(U0 + tiles_b - 1, total, nw) - wa) + 1;
  const int64_t row0 = (unit + wa) * rows + r;
  // More shares than tiles (lengths far below max_seqlen_k, or the small-call kernel's
  // shares of a few tiles): some shares are empty and write nothing, so their slots hold
  // another call's (or another unit's) data and are skipped. With total >= nw every share
  // holds a tile.
  const bool sparse = nw > total;
  for (int s0 = 0; s0 < nseg; s0 += MB) {
    f32x2_t ls[MB];
    u32x4_t ow[MB];
#pragma unroll
    for (int j = 0; j < MB; ++j) {
      const int64_t row = row0 + (int64_t)(s0 + j) * rows;
      const int64_t w = wa + s0 + j;
      const bool in = s0 + j < nseg && (!sparse || share_start(w + 1, total, nw) > share_start(w, total, nw));
      ls[j] = in ? *reinterpret_cast<const f32x2_t *>(a.part_lse + 2 * row) : f32x2_t{-INFINITY, 1.f};
      ow[j] = in ? load16(a.part_o + row * D + 8 * c) : u32x4_t{0, 0, 0, 0};
    }
    float Mb = -INFINITY;
#pragma unroll
    for (int j = 0; j < MB; ++j) Mb = fmaxf(Mb, ls[j][0]);
    if (Mb == -INFINITY) continue;  // no segment of the batch saw a position
    f32x4_t acc[2] = {{0.f, 0.f, 0.f, 0.f}, {0.f, 0.f, 0.f, 0.f}};
    float den = 0.f;
#pragma unroll
    for (int j = 0; j < MB; ++j) {
      const bool seen = ls[j][0] != -INFINITY;  // an empty segment adds nothing, whatever its values
      const float f = seen ? __builtin_amdgcn_exp2f(ls[j][0] - Mb) : 0.f;
      const float fx = f * (ls[j][1] * vs);
      den += f;
#pragma unroll
      for (int k = 0; k < 2; ++k) {
        const f32x4_t x = {f16_lo(ow[j][2 * k]), f16_hi(ow[j][2 * k]), f16_lo(ow[j][2 * k + 1]),
                           f16_hi(ow[j][2 * k + 1])};
        if (seen) acc[k] += x * fx;
      }
    }
    mg.add(Mb, 1.f, den, acc);
  }
}

__device__ __forceinline__ void store_row8(uint16_t *dst, const f32x4_t (&acc)[2]) {
  store16_nt(dst, u32x4_t{pack_bf16x2(acc[0][0], acc[0][1]), pack_bf16x2(acc[0][2], acc[0][3]),
                       pack_bf16x2(acc[1][0], acc[1][1]), pack_bf16x2(acc[1][2], acc[1][3])});
}

// Merge each unit's partials and write the bf16 output; units of empty sequences get
// zeros. One workgroup per 16-row block, one thread per (row, 8 channels), so the unit
// and its sequence metadata are uniform per workgroup.
template <int D, int MB>
__global__ __launch_bounds__(2 * D) void attn_combine_kernel(const AttnArgs a) {
  constexpr int C = D / 8;  // 8-channel chunks per row
  const int rows = a.nrb * 16;
  const int64_t unit = blockIdx.x / a.nrb;
  const int r = (int)(blockIdx.x - unit * a.nrb) * 16 + (int)threadIdx.x / C;
  const int c = (int)threadIdx.x % C;
  const int b = (int)(unit / a.ups);
  const int ul = (int)(unit - (int64_t)b * a.ups);
  const int h = ul / a.rgroups, rg = ul - h * a.rgroups;
  const int qlen_b = q_rows_of(a, b);
  const int64_t first_tok = q_token_index(a, b, 0);
  const int R = rg * rows + r;
  const int gq = R / a.q_len, tq = R - gq * a.q_len;
  if (gq >= a.group || tq >= qlen_b) return;
  RowMerge mg;
  merge_partials<D, MB>(a, unit, b, ul, r, c, a.vd ? a.v_scale * a.vd[(int64_t)b * a.d_sb + (int64_t)h * a.d_sh] : a.v_scale,
                    mg);
  if (a.tail) {  // the verify tokens' partial
    typedef __attribute__((ext_vector_type(2))) float f32x2_t;
    const int64_t row = ((int64_t)a.batch * a.ups + a.num_shares + unit) * rows + r;
    const f32x2_t ls = *reinterpret_cast<const f32x2_t *>(a.part_lse + 2 * row);
    const u32x4_t ow = load16(a.part_o + row * D + 8 * c);
    if (ls[0] != -INFINITY) {
      f32x4_t x[2];
#pragma unroll
      for (int j = 0; j < 2; ++j)
        x[j] = f32x4_t{f16_lo(ow[2 * j]), f16_hi(ow[2 * j]), f16_lo(ow[2 * j + 1]), f16_hi(ow[2 * j + 1])};
      mg.add(ls[0], ls[1], 1.f, x);
    }
  }
  mg.finish();
  const int64_t head = (int64_t)h * a.group + gq;
  store_row8(a.o + (a.cu_q ? (first_tok + tq) * a.o_st : (int64_t)b * a.o_sb + (int64_t)tq * a.o_st) +
                 head * a.o_sh + 8 * c,
             mg.acc);
}

// Merge for calls whose units are split over many shares (the small-call kernel: tens of
// segments per unit). Eight lanes per (unit, row, 8-channel chunk): lane j takes segments
// j, j + 8, ..., WIDE_MB of them per batch with all of the batch's loads issued before
// any is used, so up to 8 WIDE_MB segments cost one memory round trip; the eight running
// merges then combine over a butterfly. attn_combine_kernel's one thread per chunk
// walks the segments itself, which at 16-32 segments is several round trips and 16-32
// partial rows read by each of a few workgroups per unit.
constexpr int WIDE_LANES = 8;
constexpr int WIDE_MB = 4;

template <int D>
__global__ __launch_bounds__(256) void attn_merge_wide_kernel(const AttnArgs a) {
  typedef __attribute__((ext_vector_type(2))) float f32x2_t;
  constexpr int C = D / 8;  // 8-channel chunks per row
  const int rows = a.nrb * 16;
  const int64_t item = ((int64_t)blockIdx.x * 256 + threadIdx.x) / WIDE_LANES;
  const int j = (int)threadIdx.x % WIDE_LANES;
  const int64_t units = (int64_t)a.batch * a.ups;
  if (item >= units * rows * C) return;  // whole groups of eight lanes
  const int64_t unit = item / (rows * C);
  const int rc = (int)(item - unit * rows * C);
  const int r = rc / C, c = rc - r * C;
  const int b = (int)(unit / a.ups);
  const int ul = (int)(unit - (int64_t)b * a.ups);
  const int h = ul / a.rgroups, rg = ul - h * a.rgroups;
  const int R = rg * rows + r;
  const int gq = R / a.q_len, tq = R - gq * a.q_len;
  if (gq >= a.group || tq >= q_rows_of(a, b)) return;  // the group's row is not a draft row
  const float vs = a.vd ? a.v_scale * a.vd[(int64_t)b * a.d_sb + (int64_t)h * a.d_sh] : a.v_scale;
  RowMerge mg;
  const int64_t pre = tile_prefix(a, a.plan, b);
  const int tiles_b = (int)(tile_prefix(a, a.plan, b + 1) - pre);
  if (tiles_b > 0) {
    const int64_t uc = a.share_c;  // a unit's extra cost on the line (share_first_tiles)
    const int64_t total = (int64_t)a.ups * (tile_prefix(a, a.plan, a.batch) + uc * a.batch);  // the cost line
    const int64_t nw = a.num_shares;
    const int64_t U0 = (int64_t)a.ups * (pre + uc * b) + (int64_t)ul * (tiles_b + uc) + uc;  // cost of tile 0
    const int64_t wa = share_of(U0, total, nw);
    const int nseg = (int)(share_of(U0 + tiles_b - 1, total, nw) - wa) + 1;
    const bool sparse = nw > total;  // empty shares write nothing: their slots are skipped
    for (int s0 = j; s0 < nseg; s0 += WIDE_LANES * WIDE_MB) {
      f32x2_t ls[WIDE_MB];
      u32x4_t ow[WIDE_MB];
#pragma unroll
      for (int k = 0; k < WIDE_MB; ++k) {
        const int s = s0 + k * WIDE_LANES;
        const int64_t w = wa + s;
        const bool in = s < nseg && (!sparse || share_start(w + 1, total, nw) > share_start(w, total, nw));
        const int64_t row = (unit + w) * rows + r;
        ls[k] = in ? *reinterpret_cast<const f32x2_t *>(a.part_lse + 2 * row) : f32x2_t{-INFINITY, 1.f};
        ow[k] = in ? load16(a.part_o + row * D + 8 * c) : u32x4_t{0, 0, 0, 0};
      }
      float Mb = -INFINITY;
#pragma unroll
      for (int k = 0; k < WIDE_MB; ++k) Mb = fmaxf(Mb, ls[k][0]);
      if (Mb == -INFINITY) continue;  // no segment of the batch saw a position
      f32x4_t acc[2] = {{0.f, 0.f, 0.f, 0.f}, {0.f, 0.f, 0.f, 0.f}};
      float den = 0.f;
#pragma unroll
      for (int k = 0; k < WIDE_MB; ++k) {
        const bool seen = ls[k][0] != -INFINITY;
        const float f = seen ? __builtin_amdgcn_exp2f(ls[k][0] - Mb) : 0.f;
        const float fx = f * (ls[k][1] * vs);
        den += f;
#pragma unroll
        for (int e = 0; e < 2; ++e) {
          const f32x4_t x = {f16_lo(ow[k][2 * e]), f16_hi(ow[k][2 * e]), f16_lo(ow[k][2 * e + 1]),
                             f16_hi(ow[k][2 * e + 1])};
          if (seen) acc[e] += x * fx;
        }
      }
      mg.add(Mb, 1.f, den, acc);
    }
  }
  // Butterfly over the group's eight lanes (every lane of the group reaches it).
#pragma unroll
  for (int off = 1; off < WIDE_LANES; off <<= 1) {
    const float Mo = __shfl_xor(mg.M, off, WIDE_LANES);
    const float dn = __shfl_xor(mg.den, off, WIDE_LANES);
    f32x4_t xo[2];
#pragma unroll
    for (int e = 0; e < 2; ++e)
#pragma unroll
      for (int q = 0; q < 4; ++q) xo[e][q] = __shfl_xor(mg.acc[e][q], off, WIDE_LANES);
    if (Mo != -INFINITY) mg.add(Mo, 1.f, dn, xo);
  }
  if (j != 0) return;
  mg.finish();
  const int64_t head = (int64_t)h * a.group + gq;
  store_row8(a.o + (a.cu_q ? (q_token_index(a, b, 0) + tq) * a.o_st : (int64_t)b * a.o_sb + (int64_t)tq * a.o_st) +
                 head * a.o_sh + 8 * c,
             mg.acc);
}

// plan[0] = 0, plan[b + 1] = plan[b] + ceil(max(L_b, 0) / tile), L_b = seqlens[b], or
// seqlens[b + 1] - seqlens[b] when seqlens is a CSR indptr (csr != 0).
// The plan holds two tile prefixes, for bf16 K/V (TILE positions) at plan[0 .. batch] and
// for e4m3 K/V (TILE_F8) at plan[batch + 1 .. 2 batch + 1], so one step plan serves calls
// of either kind.
__global__ __launch_bounds__(1024) void attn_plan_kernel(const int32_t *__restrict__ seqlens,
                                                         int32_t batch, int32_t *__restrict__ plan,
                                                         int32_t csr) {
  plan_prefixes<1024>(seqlens, batch, plan, csr);
}

// ---------------------------------------------------------------------------------
// Host side: grid sizing, workspace layout, dispatch.

typedef void (*AttnKernel)(const AttnArgs, const int32_t *, const int32_t *, const int32_t *);

template <int LAYOUT, int D, bool F8, bool DQ>
static AttnKernel pick_kernel(int w) {
  switch (w) {
    case 1: return attn_fwd_kernel<LAYOUT, 1, D, F8, DQ>;
    case 2: return attn_fwd_kernel<LAYOUT, 2, D, F8, DQ>;
    case 3: return attn_fwd_kernel<LAYOUT, 3, D, F8, DQ>;
    case 4: return attn_fwd_kernel<LAYOUT, 4, D, F8, DQ>;
    case 5: return attn_fwd_kernel<LAYOUT, 5, D, F8, DQ>;
    case 6: return attn_fwd_kernel<LAYOUT, 6, D, F8, DQ>;
    case 7: return attn_fwd_kernel<LAYOUT, 7, D, F8, DQ>;
    default: return attn_fwd_kernel<LAYOUT, 8, D, F8, DQ>;
  }
}

// How a call's consumers get their query rows: straight from the caller's layout with the
// prologue applied in the kernel (bf16, no verify tokens, q_len <= QTOK, the batch's
// metadata fits the kernel's LDS, and a small call: at most one unit per two shares), else
// packed by a query pass (pack_queries_kernel, or pack_queries_f8_kernel for e4m3 K/V).
// Q_F8_DIRECT: e4m3 K/V with bf16 queries read from the caller's rows, the prologue and
// the per-(sequence, head) quantization applied in the attention kernel (q_len 16).
enum QMode { Q_DIRECT = 0, Q_PACKED = 1, Q_F8 = 2, Q_F8_DIRECT = 3 };

static bool is_f8(int qmode) { return qmode == Q_F8 || qmode == Q_F8_DIRECT; }
static bool has_pass(int qmode) { return qmode == Q_PACKED || qmode == Q_F8; }

template <int LAYOUT, int D, bool F8>
static int dq_seq_cap(int w) {
  switch (w) {
    case 1: return kernel_seq_cap<LAYOUT, D, 1, F8, true>();
    case 2: return kernel_seq_cap<LAYOUT, D, 2, F8, true>();
    case 3: return kernel_seq_cap<LAYOUT, D, 3, F8, true>();
    case 4: return kernel_seq_cap<LAYOUT, D, 4, F8, true>();
    case 5: return kernel_seq_cap<LAYOUT, D, 5, F8, true>();
    case 6: return kernel_seq_cap<LAYOUT, D, 6, F8, true>();
    case 7: return kernel_seq_cap<LAYOUT, D, 7, F8, true>();
    default: return kernel_seq_cap<LAYOUT, D, 8, F8, true>();
  }
}

// Sequences a direct-rows kernel stages in LDS, for a call's layout and head_dim.
template <bool F8>
static int dq_cap(int layout, int d, int w) {
  if (layout == PAGED) return d == 128 ? dq_seq_cap<PAGED, 128, F8>(w) : dq_seq_cap<PAGED, 64, F8>(w);
  return d == 128 ? dq_seq_cap<PAGED16, 128, F8>(w) : dq_seq_cap<PAGED16, 64, F8>(w);
}

template <int LAYOUT, int D>
static AttnKernel pick_small(int w) {
  switch (w) {
    case 2: return attn_small_kernel<LAYOUT, 2, D>;
    case 4: return attn_small_kernel<LAYOUT, 4, D>;
    case 5: return attn_small_kernel<LAYOUT, 5, D>;
    case 8: return attn_small_kernel<LAYOUT, 8, D>;
    default: return nullptr;
  }
}

// The small-call kernel for (layout, head_dim, row blocks per unit), or NULL where it has
// no instance (row blocks other than 2, 4, 5, 8).
static AttnKernel select_small(int layout, int d, int w) {
  if (d == 128) {
    if (layout == CONTIG) return pick_small<CONTIG, 128>(w);
    if (layout == PAGED16) return pick_small<PAGED16, 128>(w);
    return pick_small<PAGED, 128>(w);
  }
  if (layout == CONTIG) return pick_small<CONTIG, 64>(w);
  if (layout == PAGED16) return pick_small<PAGED16, 64>(w);
  return pick_small<PAGED, 64>(w);
}

static AttnKernel select_kernel(int layout, int d, int w, int qmode) {
  if (qmode == Q_F8) {
    if (d == 128) return layout == PAGED16 ? pick_kernel<PAGED16, 128, true, false>(w) : pick_kernel<PAGED, 128, true, false>(w);
    return layout == PAGED16 ? pick_kernel<PAGED16, 64, true, false>(w) : pick_kernel<PAGED, 64, true, false>(w);
  }
  if (qmode == Q_F8_DIRECT) {
    if (d == 128) return layout == PAGED16 ? pick_kernel<PAGED16, 128, true, true>(w) : pick_kernel<PAGED, 128, true, true>(w);
    return layout == PAGED16 ? pick_kernel<PAGED16, 64, true, true>(w) : pick_kernel<PAGED, 64, true, true>(w);
  }
  const bool dq = qmode == Q_DIRECT;
  if (d == 128) {
    if (layout == CONTIG) return dq ? pick_kernel<CONTIG, 128, false, true>(w) : pick_kernel<CONTIG, 128, false, false>(w);
    if (layout == PAGED16) return dq ? pick_kernel<PAGED16, 128, false, true>(w) : pick_kernel<PAGED16, 128, false, false>(w);
    return dq ? pick_kernel<PAGED, 128, false, true>(w) : pick_kernel<PAGED, 128, false, false>(w);
  }
  if (layout == CONTIG) return dq ? pick_kernel<CONTIG, 64, false, true>(w) : pick_kernel<CONTIG, 64, false, false>(w);
  if (layout == PAGED16) return dq ? pick_kernel<PAGED16, 64, false, true>(w) : pick_kernel<PAGED16, 64, false, false>(w);
  return dq ? pick_kernel<PAGED, 64, false, true>(w) : pick_kernel<PAGED, 64, false, false>(w);
}

struct RowPlan {
  int nrb;      // 16-row blocks per unit
  int rgroups;  // units per KV head
};

// Row blocks per unit (= consumer wavefronts per replica) and row groups per KV head. A
// unit of one 16-row block (MHA with K = 16) gets a second, all-zero block: two consumer
// wavefronts per replica stream the same K/V 20 % faster than one on MI355X (R8B, 16 KV
// heads: 388 -> 323 us), whose idle half of the math is free on this HBM-bound path. The
// zero rows are packed as zeros and never stored.
static RowPlan row_plan(int group, int q_len) {
  const int total = (group * q_len + 15) / 16;
  RowPlan p;
  p.rgroups = (total + NRB_MAX - 1) / NRB_MAX;
  p.nrb = (total + p.rgroups - 1) / p.rgroups;
  if (p.nrb == 1) p.nrb = 2;
  return p;
}

// Tuning overrides from the environment (FLASHMAP_*), read once, at the first call, and
// again only on fm_tuning_reload(): the launch path reads no environment. INT_MIN: unset.
struct Tuning {
  std::atomic<int> min_tiles{INT_MIN}, workgroups{INT_MIN}, small_tiles{INT_MIN}, query_pass{INT_MIN},
      share_cost{INT_MIN}, combine_mb{INT_MIN};
};
static Tuning g_tuning;
static std::once_flag g_tuning_once;

static int env_value(const char *name) {
  const char *v = getenv(name);
  return (v == nullptr || *v == 0) ? INT_MIN : atoi(v);
}

static void read_tuning() {
  g_tuning.min_tiles = env_value("FLASHMAP_SPLITKV_MIN_TILES");
  g_tuning.workgroups = env_value("FLASHMAP_SPLITKV_WORKGROUPS");
  g_tuning.small_tiles = env_value("FLASHMAP_SMALL_TILES");
  g_tuning.query_pass = env_value("FLASHMAP_QUERY_PASS");
  g_tuning.share_cost = env_value("FLASHMAP_SHARE_COST");
  g_tuning.combine_mb = env_value("FLASHMAP_COMBINE_MB");
}

static const Tuning &tuning() {
  std::call_once(g_tuning_once, read_tuning);
  return g_tuning;
}

static int tuned(const std::atomic<int> &v, int dflt) {
  const int x = v.load(std::memory_order_relaxed);
  return x == INT_MIN ? dflt : x;
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
  size_t plan_off, q_off, rs_off, lse_off, o_off, bytes;
};

static size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

// tail: a verify call (one more partial slot per unit, for its verify tokens). qmode: how
// the queries reach the consumers (Q_DIRECT needs no packed rows in the workspace).
static int sizing(int layout, int batch, int q_len, int hq, int hkv, int d, int max_k,
                  bool need_plan, Sizing *sz, bool tail = false, int qmode = Q_PACKED, int small_tiles = 0) {
  DeviceInfo info;
  int rc = device_info(&info);
  if (rc != FM_OK) return rc;
  sz->rp = row_plan(hq / hkv, q_len);
  AttnKernel k = select_kernel(layout, d, sz->rp.nrb, qmode);
  const int64_t ups = (int64_t)hkv * sz->rp.rgroups;
  const bool t64 = is_f8(qmode) || (small_tiles == 0 && double_tiles(sz->rp.nrb, false, layout));
  const int tile = t64 ? TILE_F8 : TILE;
  const int64_t tiles_bound = ups * batch * (((int64_t)max_k + tile - 1) / tile);
  const Tuning &tu = tuning();
  const int min_tiles = tuned(tu.min_tiles, 8) > 0 ? tuned(tu.min_tiles, 8) : 1;
  const int r = replicas(sz->rp.nrb, is_f8(qmode), layout);
  int64_t nw = (int64_t)info.cus * occupancy(k, 64 * (sz->rp.nrb + 1) * r);
  const int cap = tuned(tu.workgroups, 0);
  if (cap > 0) nw = cap;
  const int64_t want = (tiles_bound + min_tiles - 1) / min_tiles;  // shares worth splitting
  if ((want + r - 1) / r < nw) nw = (want + r - 1) / r;
  if (nw < 1) nw = 1;
  sz->num_wg = (int)nw;
  sz->num_shares = (int)nw * r;
  if (small_tiles > 0) {  // the small-call kernel: one workgroup per share of <= small_tiles tiles
    const int64_t shares = (tiles_bound + small_tiles - 1) / small_tiles;
    sz->num_wg = sz->num_shares = (int)(shares > 0 ? shares : 1);
  }
  const size_t rows = (size_t)sz->rp.nrb * 16;
  const size_t units = (size_t)batch * ups;
  const size_t slots = units + (size_t)sz->num_shares + (tail ? units : 0);  // unit + share; tails
  size_t off = 0;
  sz->plan_off = off;
  if (need_plan) off = align256(off + 2 * sizeof(int32_t) * ((size_t)batch + 1));
  sz->q_off = off;  // packed query rows (none for direct rows); fp8: a score scale per row
  if (has_pass(qmode)) off = align256(off + sizeof(uint16_t) * units * rows * d);
  sz->rs_off = off;
  if (qmode == Q_F8) off = align256(off + sizeof(float) * units * rows);
  sz->lse_off = off;
  off = align256(off + 2 * sizeof(float) * slots * rows);
  sz->o_off = off;
  off = align256(off + sizeof(uint16_t) * slots * rows * d);
  sz->bytes = off;
  return FM_OK;
}

// Tiles per share of attn_small_kernel for a bf16 call without verify tokens, or 0 where
// the persistent kernel runs: the small kernel takes calls whose K/V fits one pass of
// SMALL_TILES-tile workgroups over the CUs and whose row blocks per unit it has an
// instance for. Shares are sized to about one per CU (each CU's loads in flight bound
// the stream; partials grow with the shares). FLASHMAP_SMALL_TILES sets the tiles per
// share (1 .. SMALL_TILES) instead; 0 turns the kernel off.
static int small_tiles_for(int layout, int batch, int q_len, int hq, int hkv, int d, int max_k) {
  DeviceInfo info;
  if (device_info(&info) != FM_OK) return 0;
  const RowPlan rp = row_plan(hq / hkv, q_len);
  const int64_t tiles_bound = (int64_t)hkv * rp.rgroups * batch * (((int64_t)max_k + TILE - 1) / TILE);
  if (tiles_bound > (int64_t)info.cus * SMALL_TILES || select_small(layout, d, rp.nrb) == nullptr) return 0;
  int tps = (int)((tiles_bound + info.cus - 1) / info.cus);
  tps = tuned(tuning().small_tiles, tps);
  tps = tps > SMALL_TILES ? SMALL_TILES : tps;
  return tps > 0 ? tps : 0;
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
  bool static_ws = false;  // ws is the library's static scratch (fm_block_attn_paged_static)
};

// vf: a verify call (its combine also attends to the verify tokens).
static int run_attention(const CommonIn &c, int layout, AttnArgs a, const VerifyArgs *vf = nullptr) {
  FM_REQUIRE(c.batch >= 0 && c.q_len >= 0 && c.hq > 0 && c.hkv > 0, "bad sizes");
  if (c.batch == 0 || c.q_len == 0) return FM_OK;
  if (c.d != 64 && c.d != 128) return fail(FM_ERR_UNSUPPORTED, "head_dim %d not supported (64 or 128)", c.d);
  FM_REQUIRE(c.hq % c.hkv == 0, "num_q_heads %d is not a multiple of num_kv_heads %d", c.hq, c.hkv);
  FM_REQUIRE(c.q && c.out, "NULL query/output");
  FM_REQUIRE(al16(c.q) && al16(c.out) && al16(a.u.k) && al16(a.u.v), "q/out/k/v must be 16-byte aligned");
  FM_REQUIRE(c.q_sb % 8 == 0 && c.q_st % 8 == 0 && c.q_sh % 8 == 0 && c.o_sb % 8 == 0 &&
                 c.o_st % 8 == 0 && c.o_sh % 8 == 0,
             "query/output strides must be multiples of 8 elements");
  const int es = a.f8 ? 1 : 2;  // bytes per K/V element
  const int64_t kv_mult = 16 / es;  // the loads are 16-byte aligned
  FM_REQUIRE(a.u.k_s0 % kv_mult == 0 && a.u.k_s1 % kv_mult == 0 && a.k_s2 % kv_mult == 0 &&
                 a.u.v_s0 % kv_mult == 0 && a.u.v_s1 % kv_mult == 0 && a.v_s2 % kv_mult == 0,
             "key/value strides must be multiples of %d elements", (int)kv_mult);
  if (a.f8) {
    if (layout == CONTIG) return fail(FM_ERR_UNSUPPORTED, "fp8 K/V needs a paged layout");
    if (!a.q_fp8 && c.q_len % 16 != 0)
      return fail(FM_ERR_UNSUPPORTED, "per-head query quantization needs max_seqlen_q %% 16 == 0 (got %d)", c.q_len);
  }
  if (c.qn_w) FM_REQUIRE(c.rope_cos && c.rope_sin, "the query prologue needs the rotary table");
  // The kernels form per-tile addresses with 32-bit byte strides.
  if (a.k_s2 < 0 || a.v_s2 < 0 || a.k_s2 >= (1ll << 27) || a.v_s2 >= (1ll << 27))
    return fail(FM_ERR_UNSUPPORTED, "position strides must lie in [0, 2^27) elements");
  a.k_tok_b = (uint32_t)(es * a.k_s2);
  a.v_tok_b = (uint32_t)(es * a.v_s2);
  if (layout != CONTIG) {
    if (a.u.k_s0 < 0 || a.u.v_s0 < 0 || a.u.k_s0 >= (1ll << 31) || a.u.v_s0 >= (1ll << 31) ||
        (int64_t)a.page_size * (a.k_s2 > a.v_s2 ? a.k_s2 : a.v_s2) >= (1ll << 31))
      return fail(FM_ERR_UNSUPPORTED, "page strides must lie in [0, 2^31) elements");
    a.k_page_b = (uint32_t)(es * a.u.k_s0);
    a.v_page_b = (uint32_t)(es * a.u.v_s0);
    a.page_mask = (uint32_t)(a.page_size - 1);
    a.col_last = (uint32_t)(a.table_width - 1 < 0x7fffffffll ? a.table_width - 1 : 0x7fffffffll);
    a.page_last = (uint32_t)(a.num_pages - 1 < 0xffffffffll ? a.num_pages - 1 : 0xffffffffll);
  }
  // A plan made here (none given) holds both tile prefixes (bf16 and e4m3 tiles).
  const bool need_plan = a.seqlens != nullptr && c.plan == nullptr;
  int qmode = a.f8 ? Q_F8 : Q_PACKED;
  Sizing sz;
  int rc = sizing(layout, c.batch, c.q_len, c.hq, c.hkv, c.d, c.max_k, need_plan, &sz, vf != nullptr, qmode);
  if (rc != FM_OK) return rc;
  if (!a.f8 && vf == nullptr && c.q_len <= QTOK) {
    const RowPlan rp = row_plan(c.hq / c.hkv, c.q_len);
    // Rotary rows read in 16-byte chunks: split cos / sin rows (both 16-byte aligned) or
    // interleaved (cos, sin) rows (sin = cos + 1, the row 16-byte aligned).
    const bool split = c.rope_ps == 1 && ((uintptr_t)c.rope_sin & 15) == 0;
    const bool inter = c.rope_ps == 2 && c.rope_sin == c.rope_cos + 1;
    const bool fast_rope = c.qn_w == nullptr || ((split || inter) && ((uintptr_t)c.rope_cos & 15) == 0 &&
                                                 c.rope_rs % 4 == 0 && ((uintptr_t)c.qn_w & 3) == 0);
    const int cap = dq_cap<false>(layout, c.d, rp.nrb);
    // Direct rows cost a prologue at every segment start, inside the workgroup's barrier
    // cycle (about 5000 shader cycles at 64 rows x D 128), which the cost cut of the line
    // absorbs (6 tiles per unit); the query pass costs a launch and one read + write of the
    // rows. Measured: direct rows win up to one unit per share of 32-position tiles (batch
    // 64 x 8 KV heads, 512 units over 512 shares: 176 us per call against 179 us with the
    // pass), or two per share of 64-position line tiles (one replica: the same 512 units over
    // 256 shares); calls of more units keep the pass. FLASHMAP_QUERY_PASS=1 forces the pass,
    // =0 the direct rows where they apply; at one share cost both give the same bits.
    const int force = tuned(tuning().query_pass, -1);
    const int64_t units = (int64_t)c.batch * c.hkv * rp.rgroups;
    const bool small = units <= (int64_t)sz.num_shares * (double_tiles(rp.nrb, false, layout) ? 2 : 1);
    if (fast_rope && c.batch <= cap && (force == 0 || (force < 0 && small))) qmode = Q_DIRECT;
  }
  // e4m3 K/V with bf16 queries of one 16-row block per query head: with
  // FLASHMAP_QUERY_PASS=0 the attention kernel applies the prologue and quantizes each
  // (sequence, head) itself, bit for bit as the pass does. Not the default: measured at
  // batch 64 x 32/8 heads (C3's draw on an e4m3 cache), one box, the call takes 122.8 us
  // at its best share cost (10 tiles; 141 us at 4) against 113.8 us with the pass: the
  // quantization's 32 correctly rounded divisions per lane at every segment start sit in
  // the workgroup's barrier cycle, and the kernel needs 168 VGPRs with a small spill.
  if (a.f8 && !a.q_fp8 && vf == nullptr && c.q_len == QTOK) {
    const RowPlan rp = row_plan(c.hq / c.hkv, c.q_len);
    const bool split = c.rope_ps == 1 && ((uintptr_t)c.rope_sin & 15) == 0;
    const bool inter = c.rope_ps == 2 && c.rope_sin == c.rope_cos + 1;
    const bool fast_rope = c.qn_w == nullptr || ((split || inter) && ((uintptr_t)c.rope_cos & 15) == 0 &&
                                                 c.rope_rs % 4 == 0 && ((uintptr_t)c.qn_w & 3) == 0);
    const int cap = dq_cap<true>(layout, c.d, rp.nrb);
    const int force = tuned(tuning().query_pass, -1);
    if (fast_rope && c.batch <= cap && force == 0) qmode = Q_F8_DIRECT;
  }
  // Small calls: attn_small_kernel with the caller's rows read directly (two launches),
  // unless the workspace was sized for the persistent kernel only (a static scratch).
  int small_tiles = (!a.f8 && vf == nullptr) ? small_tiles_for(layout, c.batch, c.q_len, c.hq, c.hkv, c.d, c.max_k)
                                             : 0;
  if (small_tiles > 0) {
    Sizing ss;
    rc = sizing(layout, c.batch, c.q_len, c.hq, c.hkv, c.d, c.max_k, need_plan, &ss, false, Q_DIRECT, small_tiles);
    if (rc != FM_OK) return rc;
    if (ss.bytes <= c.ws_bytes) {
      sz = ss;
      qmode = Q_DIRECT;
    } else {
      small_tiles = 0;
    }
  }
  if (small_tiles == 0 && (qmode == Q_DIRECT || qmode == Q_F8_DIRECT)) {
    rc = sizing(layout, c.batch, c.q_len, c.hq, c.hkv, c.d, c.max_k, need_plan, &sz, vf != nullptr, qmode);
    if (rc != FM_OK) return rc;
  }
  if (c.static_ws && sz.bytes > c.ws_bytes)
    return fail(FM_ERR_WORKSPACE,
                "this call needs %zu bytes of scratch; the library's static scratch holds %zu bytes "
                "(use fm_block_attn_paged with a workspace of fm_attn_workspace_bytes)",
                sz.bytes, c.ws_bytes);
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
  // A unit's extra cost when cutting the line into shares (share_first_tiles), in tiles:
  // what a segment start and a partial hand-off cost the persistent kernel, measured best
  // at 2 tiles for bf16 (32 positions) and 4 for e4m3 (64 positions). Where the units span
  // four or more shares each on average, every share holds one or two segments whatever
  // the cut, and an extra cost only unbalances shares of equal units (batch 8 of
  // 32768-position sequences over 256 shares: 1.5-2 us slower; the 128-row tree units of 8192
  // positions: no change): the line is cut by tiles, as it is for the small-call kernel.
  // FLASHMAP_SHARE_COST overrides.
  a.t64 = a.f8 || (small_tiles == 0 && double_tiles(sz.rp.nrb, false, layout));
  const int share_c = small_tiles == 0 && units * 4 > sz.num_shares
                          ? (qmode == Q_F8_DIRECT ? 10 : a.f8 ? 4 : a.t64 ? (qmode == Q_DIRECT ? 3 : 1)
                                                                          : qmode == Q_DIRECT ? 6 : 2)
                          : 0;
  a.share_c = small_tiles > 0 ? 0 : tuned(tuning().share_cost, share_c);
  if (a.share_c < 0) a.share_c = 0;
  a.tail = vf != nullptr;
  if (!a.tail) a.v_scale = 1.f;
  char *ws = (char *)c.ws;
  a.qp = (const uint16_t *)(ws + sz.q_off);
  a.q_rs = (float *)(ws + sz.rs_off);
  a.part_lse = (float *)(ws + sz.lse_off);
  a.part_o = (uint16_t *)(ws + sz.o_off);
  // A call without a plan makes its own: in the query pass's last workgroup when there is a
  // query pass (one launch fewer), else with attn_plan_kernel.
  const bool pass = has_pass(qmode);
  if (a.seqlens != nullptr) {
    const int32_t *plan = c.plan;
    if (need_plan) {
      int32_t *own = (int32_t *)(ws + sz.plan_off);
      if (pass) {
        a.plan_out = own;
      } else {
        attn_plan_kernel<<<1, 1024, 0, c.stream>>>(a.seqlens, c.batch, own, a.csr);
        FM_CHECK_HIP(hipGetLastError());
      }
      plan = own;
    }
    a.plan = plan + (a.t64 ? c.batch + 1 : 0);  // the prefix of this call's tile size
  } else {
    a.plan = nullptr;
    a.uniform_tiles = (a.uniform_len + (a.t64 ? TILE_F8 : TILE) - 1) / (a.t64 ? TILE_F8 : TILE);
  }
  const int64_t qblocks = (units * sz.rp.nrb + 3) / 4 + (a.plan_out != nullptr ? 1 : 0);
  const VerifyArgs nov{};
  if (!pass) {
    // no query pass: the attention kernel reads the rows and applies the prologue
  } else if (a.f8 && c.d == 128) {
    pack_queries_f8_kernel<128><<<dim3((unsigned)qblocks), dim3(256), 0, c.stream>>>(a);
  } else if (a.f8) {
    pack_queries_f8_kernel<64><<<dim3((unsigned)qblocks), dim3(256), 0, c.stream>>>(a);
  } else if (vf != nullptr && c.d == 128) {
    pack_queries_kernel<128, true><<<dim3((unsigned)qblocks), dim3(256), 0, c.stream>>>(a, *vf);
  } else if (vf != nullptr) {
    pack_queries_kernel<64, true><<<dim3((unsigned)qblocks), dim3(256), 0, c.stream>>>(a, *vf);
  } else if (c.d == 128) {
    pack_queries_kernel<128, false><<<dim3((unsigned)qblocks), dim3(256), 0, c.stream>>>(a, nov);
  } else {
    pack_queries_kernel<64, false><<<dim3((unsigned)qblocks), dim3(256), 0, c.stream>>>(a, nov);
  }
  if (pass) FM_CHECK_HIP(hipGetLastError());
  AttnKernel k = small_tiles > 0 ? select_small(layout, c.d, sz.rp.nrb) : select_kernel(layout, c.d, sz.rp.nrb, qmode);
  const dim3 kblock(small_tiles > 0 ? 64 * (sz.rp.nrb + 1) : 64 * (sz.rp.nrb + 1) * replicas(sz.rp.nrb, a.f8 != 0, layout));
  const int32_t *ktab = a.table, *kplan = a.plan, *kseq = a.seqlens;
  void *kargs[] = {&a, &ktab, &kplan, &kseq};
  profile_before(c.stream);
  const hipError_t lerr = hipLaunchKernel(reinterpret_cast<const void *>(k), dim3(sz.num_wg), kblock, kargs, 0,
                                          c.stream);
  profile_after(c.stream);
  if (lerr != hipSuccess) return fail(FM_ERR_HIP, "attention launch failed: %s", hipGetErrorString(lerr));
  if (small_tiles > 0) {  // the wide merge: eight lanes per (unit, row, 8-channel chunk)
    const int64_t lanes = units * sz.rp.nrb * 16 * (c.d / 8) * WIDE_LANES;
    const int64_t mblocks = (lanes + 255) / 256;
    FM_REQUIRE(mblocks < (1ll << 31), "too many units");
    if (c.d == 128)
      attn_merge_wide_kernel<128><<<dim3((unsigned)mblocks), dim3(256), 0, c.stream>>>(a);
    else
      attn_merge_wide_kernel<64><<<dim3((unsigned)mblocks), dim3(256), 0, c.stream>>>(a);
    FM_CHECK_HIP(hipGetLastError());
    return FM_OK;
  }
  // One workgroup of 2 D threads per 16-row block, merging a unit's partials MB at a time:
  // MB about the segments a unit has (a segment per share it touches: shares / units + 1
  // on average), so that most units take one memory round trip at the fewest registers.
  const int64_t cblocks = units * sz.rp.nrb;
  FM_REQUIRE(cblocks < (1ll << 31), "too many units");
  const int64_t segs = (sz.num_shares + units - 1) / units + 1;
  int mb = tuned(tuning().combine_mb, segs <= 2 ? 2 : segs <= 4 ? 4 : 8);
  mb = mb <= 2 ? 2 : mb <= 4 ? 4 : 8;
  const dim3 cg((unsigned)cblocks);
  if (c.d == 128) {
    if (mb == 2) attn_combine_kernel<128, 2><<<cg, dim3(256), 0, c.stream>>>(a);
    else if (mb == 4) attn_combine_kernel<128, 4><<<cg, dim3(256), 0, c.stream>>>(a);
    else attn_combine_kernel<128, 8><<<cg, dim3(256), 0, c.stream>>>(a);
  } else {
    if (mb == 2) attn_combine_kernel<64, 2><<<cg, dim3(128), 0, c.stream>>>(a);
    else if (mb == 4) attn_combine_kernel<64, 4><<<cg, dim3(128), 0, c.stream>>>(a);
    else attn_combine_kernel<64, 8><<<cg, dim3(128), 0, c.stream>>>(a);
  }
  FM_CHECK_HIP(hipGetLastError());
  return FM_OK;
}

}  // namespace fm

using namespace fm;

extern "C" size_t fm_attn_plan_bytes(int32_t batch) {
  return 2 * sizeof(int32_t) * ((size_t)(batch < 0 ? 0 : batch) + 1);
}

extern "C" int fm_attn_plan(const int32_t *seqlens, int32_t batch, int32_t *plan, void *stream) {
  FM_REQUIRE(batch >= 0, "bad batch");
  FM_REQUIRE(plan != nullptr && (batch == 0 || seqlens != nullptr), "NULL pointer");
  attn_plan_kernel<<<1, 1024, 0, (hipStream_t)stream>>>(seqlens, batch, plan, 0);
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
  // with room for an in-call plan; calls the small-call kernel takes at the largest share
  // count any FLASHMAP_SMALL_TILES gives (one tile per share: at most CUs x SMALL_TILES
  // shares).
  size_t bytes = 0;
  int rc = FM_OK;
  for (int v = 0; v < 5 && rc == FM_OK; ++v) {  // the three layouts, then the two fp8 ones
    const int layout = v < 3 ? v : v - 2;
    Sizing sz;
    rc = sizing(layout, batch, max_seqlen_q, num_q_heads, num_kv_heads, head_dim, max_seqlen_k,
                true, &sz, false, v >= 3 ? Q_F8 : Q_PACKED);
    if (rc == FM_OK && sz.bytes > bytes) bytes = sz.bytes;
    if (rc == FM_OK && v >= 3) {  // e4m3 calls with direct rows (their kernel's grid may differ)
      rc = sizing(layout, batch, max_seqlen_q, num_q_heads, num_kv_heads, head_dim, max_seqlen_k, true, &sz,
                  false, Q_F8_DIRECT);
      if (rc == FM_OK && sz.bytes > bytes) bytes = sz.bytes;
    }
    const int st = v < 3 ? small_tiles_for(layout, batch, max_seqlen_q, num_q_heads, num_kv_heads, head_dim,
                                           max_seqlen_k)
                         : 0;
    if (rc == FM_OK && st > 0) {  // the small-call kernel at one tile per share: the most shares
      rc = sizing(layout, batch, max_seqlen_q, num_q_heads, num_kv_heads, head_dim, max_seqlen_k, true, &sz,
                  false, Q_DIRECT, 1);
      if (rc == FM_OK && sz.bytes > bytes) bytes = sz.bytes;
    }
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
  a.u.k = (const char *)k;
  a.u.v = (const char *)v;
  a.u.k_s0 = k_stride_batch, a.u.k_s1 = k_stride_head, a.k_s2 = k_stride_pos;
  a.u.v_s0 = v_stride_batch, a.u.v_s1 = v_stride_head, a.v_s2 = v_stride_pos;
  // An empty cache: every sequence attends to nothing (zeros), whatever seqlens_k says.
  a.seqlens = kv_len > 0 ? seqlens_k : nullptr;
  a.uniform_len = kv_len;
  a.u.pos_cap = kv_len;
  return run_attention(c, CONTIG, a);
}

// The vLLM cache view (layout PAGED16 for power-of-two pages of >= 16 positions).
static int setup_paged(AttnArgs &a, int &layout, const void *kv_cache, int64_t num_blocks, int64_t stride_block,
                       int64_t stride_head, int64_t stride_token, int64_t v_offset, int32_t page_size,
                       const int32_t *block_table, int64_t block_table_stride, int64_t block_table_width,
                       const int32_t *seqused_k, int es) {
  FM_REQUIRE(kv_cache && block_table && seqused_k, "NULL cache/block table/seqused_k");
  FM_REQUIRE(page_size > 0 && num_blocks > 0 && block_table_width > 0, "bad page geometry");
  FM_REQUIRE(v_offset % (16 / es) == 0, "v_offset must be a multiple of %d elements", 16 / es);
  const bool pow2 = (page_size & (page_size - 1)) == 0;
  layout = (pow2 && page_size % 16 == 0) ? PAGED16 : PAGED;
  a.u.k = (const char *)kv_cache;
  a.u.v = (const char *)kv_cache + es * v_offset;
  a.u.k_s0 = stride_block, a.u.k_s1 = stride_head, a.k_s2 = stride_token;
  a.u.v_s0 = stride_block, a.u.v_s1 = stride_head, a.v_s2 = stride_token;
  a.table = block_table;
  a.u.table_stride = block_table_stride;
  a.table_width = block_table_width;
  a.num_pages = num_blocks;
  a.page_size = page_size;
  a.page_shift = pow2 ? __builtin_ctz((unsigned)page_size) : 0;
  a.seqlens = seqused_k;
  return FM_OK;
}

// The fp8 fields of a call: queries e4m3 (q_fp8) or bf16 to quantize, descales
// (3, batch, kv heads) at [kind * s_kind + b * s_batch + h * s_head] or NULL (all 1).
static int setup_fp8(AttnArgs &a, const CommonIn &c, int32_t q_fp8, const float *descales, int64_t s_kind,
                     int64_t s_batch, int64_t s_head) {
  FM_REQUIRE(!(q_fp8 && c.qn_w), "the query prologue needs bf16 queries");
  a.f8 = 1;
  a.q_fp8 = q_fp8 ? 1 : 0;
  if (descales != nullptr) {
    a.qd = q_fp8 ? descales : nullptr;
    a.kd = descales + s_kind;
    a.vd = descales + 2 * s_kind;
    a.d_sb = s_batch;
    a.d_sh = s_head;
  }
  return FM_OK;
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
  CommonIn c{q, q_stride_batch, q_stride_token, q_stride_head, out, out_stride_batch,
             out_stride_token, out_stride_head, cu_seqlens_q, batch, max_seqlen_q, max_seqlen_k,
             num_q_heads, num_kv_heads, head_dim, softmax_scale, q_norm_weight, rope_cos,
             rope_sin, rope_row_stride, rope_pair_stride, rope_rows, q_positions, eps, plan,
             workspace, workspace_bytes, (hipStream_t)stream};
  AttnArgs a{};
  int layout = 0;
  const int rc = setup_paged(a, layout, kv_cache, num_blocks, stride_block, stride_head, stride_token, v_offset,
                             page_size, block_table, block_table_stride, block_table_width, seqused_k, 2);
  return rc != FM_OK ? rc : run_attention(c, layout, a);
}

// The workspace of fm_block_attn_paged_static: device memory the library holds itself
// (one copy per GPU the library runs on, kept until the process ends) for callers that
// cannot allocate. Host code never passes `scratch` itself to a kernel (in host code the
// name is a host-side stand-in): it takes the array's device address per device with
// hipGetSymbolAddress once, with that device current, and uses that address.
constexpr size_t STATIC_SCRATCH_BYTES = (size_t)32 << 20;
static __device__ __align__(256) char scratch[STATIC_SCRATCH_BYTES];

static std::mutex g_scratch_mu;
static std::vector<void *> g_scratch_ptr;  // per device: the address of its `scratch`

static int static_scratch(void **ptr) {
  int dev = 0;
  FM_CHECK_HIP(hipGetDevice(&dev));
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if ((int)g_scratch_ptr.size() <= dev) g_scratch_ptr.resize(dev + 1, nullptr);
  if (g_scratch_ptr[dev] == nullptr) {
    void *p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || p == nullptr)
      return fail(FM_ERR_HIP, "hipGetSymbolAddress(scratch) on device %d failed: %s", dev, hipGetErrorString(e));
    g_scratch_ptr[dev] = p;
  }
  *ptr = g_scratch_ptr[dev];
  return FM_OK;
}

extern "C" size_t fm_static_scratch_bytes(void) { return STATIC_SCRATCH_BYTES; }

// Set-up of fm_block_attn_paged_static on the current device, outside any graph capture:
// the scratch array's address, the device's properties, the tuning overrides and the
// occupancy of every attention kernel a bf16 paged call can pick, so that a first call
// made under capture does no host query of its own.
extern "C" int fm_static_scratch_init(void) {
  void *p = nullptr;
  int rc = static_scratch(&p);
  if (rc != FM_OK) return rc;
  DeviceInfo info;
  rc = device_info(&info);
  if (rc != FM_OK) return rc;
  tuning();
  for (int d : {64, 128})
    for (int layout : {(int)PAGED16, (int)PAGED})
      for (int w = 1; w <= NRB_MAX; ++w)
        for (int qmode : {(int)Q_DIRECT, (int)Q_PACKED})
          occupancy(select_kernel(layout, d, w, qmode), 64 * (w + 1) * replicas(w, false, layout));
  return FM_OK;
}

extern "C" int fm_tuning_reload(void) {
  std::call_once(g_tuning_once, read_tuning);
  read_tuning();
  return FM_OK;
}

extern "C" int fm_block_attn_paged_static(
    const void *q, int64_t q_stride_batch, int64_t q_stride_token, int64_t q_stride_head, void *out,
    int64_t out_stride_batch, int64_t out_stride_token, int64_t out_stride_head,
    const int32_t *cu_seqlens_q, const void *kv_cache, int64_t num_blocks, int64_t stride_block,
    int64_t stride_head, int64_t stride_token, int64_t v_offset, int32_t page_size,
    const int32_t *block_table, int64_t block_table_stride, int64_t block_table_width,
    const int32_t *seqused_k, int32_t batch, int32_t max_seqlen_q, int32_t max_seqlen_k,
    int32_t num_q_heads, int32_t num_kv_heads, int32_t head_dim, float softmax_scale,
    const float *q_norm_weight, const float *rope_cos, const float *rope_sin,
    int64_t rope_row_stride, int64_t rope_pair_stride, int64_t rope_rows,
    const int64_t *q_positions, float eps, const int32_t *plan, void *stream) {
  void *ws = nullptr;
  int rc = static_scratch(&ws);
  if (rc != FM_OK) return rc;
  CommonIn c{q, q_stride_batch, q_stride_token, q_stride_head, out, out_stride_batch,
             out_stride_token, out_stride_head, cu_seqlens_q, batch, max_seqlen_q, max_seqlen_k,
             num_q_heads, num_kv_heads, head_dim, softmax_scale, q_norm_weight, rope_cos,
             rope_sin, rope_row_stride, rope_pair_stride, rope_rows, q_positions, eps, plan,
             ws, STATIC_SCRATCH_BYTES, (hipStream_t)stream, true};
  AttnArgs a{};
  int layout = 0;
  rc = setup_paged(a, layout, kv_cache, num_blocks, stride_block, stride_head, stride_token, v_offset,
                   page_size, block_table, block_table_stride, block_table_width, seqused_k, 2);
  return rc != FM_OK ? rc : run_attention(c, layout, a);
}

extern "C" int fm_block_attn_paged_runs(
    const void *q, int64_t q_stride_batch, int64_t q_stride_token, int64_t q_stride_head, void *out,
    int64_t out_stride_batch, int64_t out_stride_token, int64_t out_stride_head,
    const int32_t *cu_seqlens_q, const void *const *run_caches, const int32_t *run_first_slot,
    const int32_t *run_count, int32_t num_runs, int32_t heads_per_cache, int64_t num_blocks,
    int64_t stride_block, int64_t stride_head, int64_t stride_token, int64_t v_offset, int32_t page_size,
    const int32_t *block_table, int64_t block_table_stride, int64_t block_table_width,
    const int32_t *seqused_k, int32_t batch, int32_t max_seqlen_q, int32_t max_seqlen_k,
    int32_t num_q_heads, int32_t num_kv_heads, int32_t head_dim, float softmax_scale,
    const float *q_norm_weight, const float *rope_cos, const float *rope_sin,
    int64_t rope_row_stride, int64_t rope_pair_stride, int64_t rope_rows,
    const int64_t *q_positions, float eps, const int32_t *plan, void *workspace,
    size_t workspace_bytes, void *stream) {
  FM_REQUIRE(run_caches && run_first_slot && run_count, "NULL run arrays");
  FM_REQUIRE(num_runs >= 1 && num_runs <= MAX_RUNS, "num_runs %d outside [1, %d]", num_runs, MAX_RUNS);
  FM_REQUIRE(heads_per_cache > 0, "heads_per_cache must be positive");
  int heads = 0;
  for (int r = 0; r < num_runs; ++r) {
    FM_REQUIRE(run_caches[r] != nullptr && al16(run_caches[r]), "run %d: NULL or misaligned cache", r);
    FM_REQUIRE(run_count[r] > 0 && run_first_slot[r] >= 0 && run_first_slot[r] + run_count[r] <= heads_per_cache,
               "run %d: slots [%d, %d) outside a cache of %d heads", r, run_first_slot[r],
               run_first_slot[r] + run_count[r], heads_per_cache);
    heads += run_count[r];
  }
  FM_REQUIRE(heads == num_kv_heads, "the runs hold %d heads, expected num_kv_heads %d", heads, num_kv_heads);
  CommonIn c{q, q_stride_batch, q_stride_token, q_stride_head, out, out_stride_batch,
             out_stride_token, out_stride_head, cu_seqlens_q, batch, max_seqlen_q, max_seqlen_k,
             num_q_heads, num_kv_heads, head_dim, softmax_scale, q_norm_weight, rope_cos,
             rope_sin, rope_row_stride, rope_pair_stride, rope_rows, q_positions, eps, plan,
             workspace, workspace_bytes, (hipStream_t)stream};
  AttnArgs a{};
  int layout = 0;
  const int rc = setup_paged(a, layout, run_caches[0], num_blocks, stride_block, stride_head, stride_token,
                             v_offset, page_size, block_table, block_table_stride, block_table_width, seqused_k, 2);
  if (rc != FM_OK) return rc;
  // Run r serves heads [first, first + count) from slots [slot, slot + count): its base is
  // the cache moved by (slot - first) heads, so that head h sits at base + h * stride_head.
  a.nruns = num_runs;
  int first = 0;
  for (int r = 0; r < num_runs; ++r) {
    const uintptr_t base = (uintptr_t)run_caches[r] + (uintptr_t)(((int64_t)run_first_slot[r] - first) * stride_head * 2);
    a.run_head[r] = first;
    a.run_k[r] = (const char *)base;
    a.run_v[r] = (const char *)(base + (uintptr_t)(2 * v_offset));
    first += run_count[r];
  }
  a.u.k = a.run_k[0];
  a.u.v = a.run_v[0];
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
  a.u.k = (const char *)key_buffer;
  a.u.v = (const char *)value_buffer;
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

// Context length a verify call plans its grid for: the hint, else the pool size (a
// request cannot hold more distinct pool rows).
static int32_t verify_max_context(int32_t max_context, int64_t pool_size) {
  if (max_context > 0) return max_context;
  return (int32_t)(pool_size < 0x7fffffffll ? pool_size : 0x7fffffffll);
}

extern "C" size_t fm_verify_workspace_bytes(int32_t batch, int32_t verify_len, int32_t num_q_heads,
                                            int32_t num_kv_heads, int32_t head_dim, int32_t max_context,
                                            int64_t pool_size, int device) {
  if (batch <= 0 || verify_len <= 0 || num_kv_heads <= 0 || num_q_heads % num_kv_heads != 0 ||
      (head_dim != 64 && head_dim != 128))
    return 256;
  int prev = 0;
  if (hipGetDevice(&prev) != hipSuccess) return 0;
  if (device != prev && hipSetDevice(device) != hipSuccess) return 0;
  Sizing sz;
  const int rc = sizing(PAGED, batch, verify_len, num_q_heads, num_kv_heads, head_dim,
                        verify_max_context(max_context, pool_size), true, &sz, true, Q_PACKED);
  if (device != prev) hipSetDevice(prev);
  return rc == FM_OK ? sz.bytes : 0;
}

extern "C" int fm_verify_attention(
    const void *q, int64_t q_stride_token, int64_t q_stride_head, const void *k_ext,
    int64_t k_ext_stride_token, int64_t k_ext_stride_head, const void *v_ext, int64_t v_ext_stride_token,
    int64_t v_ext_stride_head, void *out, int64_t out_stride_token, int64_t out_stride_head,
    const void *key_buffer, const void *value_buffer, int64_t pool_size, int64_t k_stride_slot,
    int64_t k_stride_head, int64_t v_stride_slot, int64_t v_stride_head, const int32_t *kv_indptr,
    const void *kv_indices, int32_t kv_index_bytes, const uint8_t *custom_mask, const int64_t *mask_indptr,
    int32_t mask_mode, int32_t batch, int32_t verify_len, int32_t num_q_heads, int32_t num_kv_heads,
    int32_t head_dim, float sm_scale, float k_scale, float v_scale, int32_t max_context,
    void *workspace, size_t workspace_bytes, void *stream) {
  FM_REQUIRE(batch >= 0 && verify_len >= 0, "bad sizes");
  if (batch == 0 || verify_len == 0) return FM_OK;
  FM_REQUIRE(key_buffer && value_buffer && kv_indptr && kv_indices, "NULL pool/indptr/indices");
  FM_REQUIRE(k_ext && v_ext, "NULL verify keys/values");
  FM_REQUIRE(pool_size > 0, "bad pool size");
  FM_REQUIRE(kv_index_bytes == 4 || kv_index_bytes == 8, "kv_indices must be int32 or int64");
  FM_REQUIRE(mask_mode >= 0 && mask_mode <= 2, "mask_mode %d (0 causal, 1 full rows, 2 verify blocks)",
             mask_mode);
  FM_REQUIRE(mask_mode == 0 || custom_mask != nullptr, "the mask mode needs custom_mask");
  FM_REQUIRE(mask_mode != 1 || mask_indptr != nullptr, "full-row masks need mask_indptr");
  FM_REQUIRE(al16(k_ext) && al16(v_ext), "verify keys/values must be 16-byte aligned");
  FM_REQUIRE(k_ext_stride_token % 8 == 0 && k_ext_stride_head % 8 == 0 && v_ext_stride_token % 8 == 0 &&
                 v_ext_stride_head % 8 == 0,
             "verify key/value strides must be multiples of 8 elements");
  const int64_t q_sb = (int64_t)verify_len * q_stride_token, o_sb = (int64_t)verify_len * out_stride_token;
  CommonIn c{q, q_sb, q_stride_token, q_stride_head, out, o_sb, out_stride_token, out_stride_head,
             nullptr, batch, verify_len, verify_max_context(max_context, pool_size), num_q_heads,
             num_kv_heads, head_dim, sm_scale * k_scale, nullptr, nullptr, nullptr, 0, 0, 0, nullptr,
             0.f, nullptr, workspace, workspace_bytes, (hipStream_t)stream};
  AttnArgs a{};
  a.u.k = (const char *)key_buffer;
  a.u.v = (const char *)value_buffer;
  a.u.k_s0 = k_stride_slot, a.u.k_s1 = k_stride_head, a.k_s2 = 0;
  a.u.v_s0 = v_stride_slot, a.u.v_s1 = v_stride_head, a.v_s2 = 0;
  a.table = (const int32_t *)kv_indices;
  a.u.table_stride = 0;
  a.table_width = 1ll << 40;  // CSR rows are bounded by indptr, not by a table width
  a.num_pages = pool_size;
  a.page_size = 1;
  a.page_shift = 0;
  a.csr = 1;
  a.id_shift = kv_index_bytes == 8 ? 1 : 0;
  a.seqlens = kv_indptr;
  a.v_scale = v_scale;
  VerifyArgs vf{(const uint16_t *)k_ext, (const uint16_t *)v_ext, k_ext_stride_token, k_ext_stride_head,
                v_ext_stride_token, v_ext_stride_head, custom_mask, mask_indptr, mask_mode,
                sm_scale * 1.4426950408889634f};
  return run_attention(c, PAGED, a, &vf);
}

extern "C" int fm_block_attn_paged_fp8(
    const void *q, int32_t q_fp8, int64_t q_stride_batch, int64_t q_stride_token, int64_t q_stride_head,
    void *out, int64_t out_stride_batch, int64_t out_stride_token, int64_t out_stride_head,
    const int32_t *cu_seqlens_q, const void *kv_cache, int64_t num_blocks, int64_t stride_block,
    int64_t stride_head, int64_t stride_token, int64_t v_offset, int32_t page_size,
    const int32_t *block_table, int64_t block_table_stride, int64_t block_table_width,
    const int32_t *seqused_k, int32_t batch, int32_t max_seqlen_q, int32_t max_seqlen_k,
    int32_t num_q_heads, int32_t num_kv_heads, int32_t head_dim, float softmax_scale,
    const float *descales, int64_t descale_stride_kind, int64_t descale_stride_batch,
    int64_t descale_stride_head, const float *q_norm_weight, const float *rope_cos, const float *rope_sin,
    int64_t rope_row_stride, int64_t rope_pair_stride, int64_t rope_rows, const int64_t *q_positions,
    float eps, const int32_t *plan, void *workspace, size_t workspace_bytes, void *stream) {
  CommonIn c{q, q_stride_batch, q_stride_token, q_stride_head, out, out_stride_batch,
             out_stride_token, out_stride_head, cu_seqlens_q, batch, max_seqlen_q, max_seqlen_k,
             num_q_heads, num_kv_heads, head_dim, softmax_scale, q_norm_weight, rope_cos,
             rope_sin, rope_row_stride, rope_pair_stride, rope_rows, q_positions, eps, plan,
             workspace, workspace_bytes, (hipStream_t)stream};
  AttnArgs a{};
  int layout = 0;
  int rc = setup_paged(a, layout, kv_cache, num_blocks, stride_block, stride_head, stride_token, v_offset,
                       page_size, block_table, block_table_stride, block_table_width, seqused_k, 1);
  if (rc == FM_OK)
    rc = setup_fp8(a, c, q_fp8, descales, descale_stride_kind, descale_stride_batch, descale_stride_head);
  return rc != FM_OK ? rc : run_attention(c, layout, a);
}

extern "C" int fm_block_attn_token_paged_fp8(
    const void *q, int32_t q_fp8, int64_t q_stride_batch, int64_t q_stride_token, int64_t q_stride_head,
    void *out, int64_t out_stride_batch, int64_t out_stride_token, int64_t out_stride_head,
    const int32_t *cu_seqlens_q, const void *key_buffer, const void *value_buffer, int64_t pool_size,
    int64_t k_stride_slot, int64_t k_stride_head, int64_t v_stride_slot, int64_t v_stride_head,
    const int32_t *page_table, int64_t page_table_stride, int64_t page_table_width,
    const int32_t *cache_seqlens, int32_t batch, int32_t max_seqlen_q, int32_t max_seqlen_k,
    int32_t num_q_heads, int32_t num_kv_heads, int32_t head_dim, float softmax_scale,
    const float *descales, int64_t descale_stride_kind, int64_t descale_stride_batch,
    int64_t descale_stride_head, const float *q_norm_weight, const float *rope_cos, const float *rope_sin,
    int64_t rope_row_stride, int64_t rope_pair_stride, int64_t rope_rows, const int64_t *q_positions,
    float eps, const int32_t *plan, void *workspace, size_t workspace_bytes, void *stream) {
  FM_REQUIRE(key_buffer && value_buffer && page_table && cache_seqlens, "NULL pool/page table/seqlens");
  FM_REQUIRE(pool_size > 0 && page_table_width > 0, "bad pool geometry");
  CommonIn c{q, q_stride_batch, q_stride_token, q_stride_head, out, out_stride_batch,
             out_stride_token, out_stride_head, cu_seqlens_q, batch, max_seqlen_q, max_seqlen_k,
             num_q_heads, num_kv_heads, head_dim, softmax_scale, q_norm_weight, rope_cos,
             rope_sin, rope_row_stride, rope_pair_stride, rope_rows, q_positions, eps, plan,
             workspace, workspace_bytes, (hipStream_t)stream};
  AttnArgs a{};
  a.u.k = (const char *)key_buffer;
  a.u.v = (const char *)value_buffer;
  a.u.k_s0 = k_stride_slot, a.u.k_s1 = k_stride_head, a.k_s2 = 0;
  a.u.v_s0 = v_stride_slot, a.u.v_s1 = v_stride_head, a.v_s2 = 0;
  a.table = page_table;
  a.u.table_stride = page_table_stride;
  a.table_width = page_table_width;
  a.num_pages = pool_size;
  a.page_size = 1;
  a.page_shift = 0;
  a.seqlens = cache_seqlens;
  const int rc = setup_fp8(a, c, q_fp8, descales, descale_stride_kind, descale_stride_batch, descale_stride_head);
  return rc != FM_OK ? rc : run_attention(c, PAGED, a);
}
