// (a) draft and (b) verify attention of the self-spec round: W window query rows of each sequence attend to the
// committed prefix (paged K/V, 16-token pages) plus the window's own K/V (staging), with the draft
// (n_causal leading causal rows, the rest bidirectional) or verify (causal) window mask.
//
// gfx950 design
//   * GQA packing: the G = Hq/Hkv query heads of one KV head and the W window rows form R = G*W query rows that
//     share every K/V byte read (row n = w*G + g); rows are MFMA N-tiles of 16. One workgroup takes a unit
//     (sequence, kv head, key split) for all its rows (up to 10 N-tiles; wider windows use several row groups), so
//     each K/V byte of the split enters the CU's LDS once.
//   * Wide kernel (batches): up to 4 row waves, each owning NGW <= 3 N-tiles (Q fragments in registers) and scoring
//     every tile of the split in two 32-key steps with its own online softmax, so no data moves between waves; two
//     workgroups share a CU, so their tile loops interleave on the SIMDs (the waves of one workgroup meet at a
//     barrier every tile and would otherwise run their MFMA and softmax phases in lockstep). The row-group kernel
//     (small batches) splits each stage's keys over its waves instead and combines them at the end.
//   * Transposed contractions on v_mfma_f32_16x16x32_bf16:  S^T = K Q^T  (M = tokens, N = rows, K = head dim) and
//     O^T = V^T P^T  (M = head dim, N = rows, K = tokens). A lane then owns one query row per N-tile, so the online
//     softmax max is two xor-shuffles and the row sum stays lane-local until the end. The P^T operand is the lane's
//     own S^T values; the token order inside the K=32 step is permuted identically on the V^T side, so no data
//     moves between lanes.
//   * K tiles live in LDS as [token][D] with an XOR swizzle of the 16-byte chunks (conflict-free 16-row reads);
//     V pages are stored token-minor ([D][16] per page) in HBM, so the V^T operand is two 8-byte LDS reads.
//   * Tiles stream straight from global memory into LDS (global_load_lds_dwordx4; no staging registers) through a
//     ring of 2 one-tile slots per workgroup: tile i + 1 is in flight while tile i is computed (and the CU's other
//     workgroup streams its own), one workgroup barrier per tile, each wave waiting for its own loads of tile i. The
//     loads are issued from inline assembly so the compiler does not add a wait for every in-flight LDS load before
//     each LDS read. The split's page ids are read once into LDS.
//   * Grid order is XCD-aware: the grid enumerates only the units that hold keys (each workgroup finds its unit from
//     the device-side lengths), consecutive units go to different XCDs (ragged batches balance), the row groups of
//     one unit to the same XCD (their repeated K/V reads hit its L2).
//   * Keys are tiled by absolute position (window rows take the positions after the prefix); the split size, the
//     tile -> split -> wave assignment and the kernel come from the caller's plan (gss_attn_plan) only, never
//     from W, the prefix length or the row grouping, and every combine runs in a fixed order. Results therefore do not
//     depend on where a key comes from or on how many rows are in the window: a verify row reproduces the AR step
//     of the same token bit for bit. With several splits, the normalized partial O (bf16) and (m, l) (fp32) of each
//     split go to the caller's workspace and the merge kernel combines the valid splits of every row.
#include "gss_common.h"

#include <type_traits>

namespace {

constexpr int PAGE = 16;
constexpr int TILE = 64;        // KV tokens per tile (4 pages)
constexpr int RW_MAX = 4;       // row waves per workgroup: <= 8 waves, 2 per SIMD
constexpr int NGW_MAX = 3;      // N-tiles (16 query rows) per row wave
constexpr int MAX_TPS = 256;    // tiles per split (page ids of a split in LDS: 4 * MAX_TPS ints)
constexpr int MAX_SPLIT = 256;
constexpr float LOG2E = 1.4426950408889634f;
// a row's reference max may trail its running max by up to this (log2 domain): P^T <= 2^8, O and l stay far from
// fp32 overflow, and the rescale of O runs only when a max jumps by more
constexpr float RESCALE_SLACK = 8.f;
// the row-group kernel (small batches): stages of RG_LANES tiles, a wave per (tile lane, key half), RG_NTG N-tiles
// per workgroup
constexpr int RG_LANES = 4;
constexpr int RG_NTG = 3;
constexpr int RG_THREADS = 64 * 2 * RG_LANES;

typedef __attribute__((address_space(1))) void gvoid_t;  // global memory (direct-to-LDS load source)
typedef __attribute__((address_space(3))) void lvoid_t;  // LDS (its destination)

struct AttnParams {
  const uint16_t* q;
  const uint16_t* k_pages;
  const uint16_t* v_pages;
  const int32_t* page_table;
  const int32_t* prefix_len;
  const uint16_t* k_win;
  const uint16_t* v_win;
  uint16_t* out;
  uint16_t* ws_o;  // [bs, Hkv, n_split, R, D] bf16: O / l of each split
  float* ws_ml;    // [bs, Hkv, R, n_split, 2]:      (m, l) of each split (log2 domain max, sum)
  int bs, pt_stride, prefix_extra, W, n_causal, Hq, Hkv, G, R, n_split, RW, TPG, RG, n_units, tps;
  int cap;  // prefix lengths are clamped to this: min(plan capacity, what a page-table row addresses)
  float scale_log2;
};

template <int D>
struct Lds {  // the wide kernel: a 2-slot ring and the split's page ids, so two workgroups fit a CU
  static constexpr int TILE_EL = TILE * D;          // elements of one K (or V) tile
  static constexpr int NSLOT = 2;                   // one-tile slots of the load ring
  static constexpr int SLOT_EL = 2 * TILE_EL;       // a slot: K [TILE][D] swizzled, then V [4][D][16]
  static constexpr int BUF_BYTES = NSLOT * SLOT_EL * 2;  // the ring (bytes)
  static constexpr int TOTAL = BUF_BYTES + 4 * MAX_TPS * 4;  // then the split's page ids (4 pages per tile)
  static_assert(2 * TOTAL <= 160 * 1024, "two workgroups per CU");
};

template <int D>
struct LdsRG {
  static constexpr int TILE_EL = TILE * D;          // elements of one K (or V) tile
  static constexpr int V_OFF = RG_LANES * TILE_EL;     // K stage [RG_LANES][TILE][D] swizzled, then V [RG_LANES][4][D][16]
  static constexpr int BYTES = 2 * RG_LANES * TILE_EL * 2;         // the K/V stage
  static constexpr int MAX_BYTES = RG_THREADS / 64 * RG_NTG * 16 * 4;  // row-max exchange [waves][NG][16] after it
  static constexpr int TOTAL = BYTES + MAX_BYTES;
  // combine scratch (reuses the K/V stage): per (wave, N-tile) O as bf16 [DT][64 lanes] x 4 + l [16 rows]
  static constexpr int SCR_BYTES = (D / 16) * 64 * 8 + 16 * 4;
  static_assert(RG_THREADS / 64 * RG_NTG * SCR_BYTES <= BYTES, "combine scratch exceeds the K/V stage");
  static_assert(TOTAL <= 160 * 1024, "LDS budget");
};


template <int D>
GSS_DEV int k_lds_index(int tok, int chunk) {
  // 16-byte chunk `chunk` of token row `tok`, XOR-swizzled over the D/8 chunks of a row
  return (tok * (D / 8) + (chunk ^ (tok & (D / 8 - 1)))) * 8;
}

// V tile layout [page][d][16 tokens]: the two 8-token halves of a (page, d) row are swapped when bit 3 of d is set,
// so the 8-byte V^T reads of head dims d and d + 8 land in different LDS banks.
GSS_DEV int v_lds_index(int pi, int d, int h, int D) { return (pi * D + d) * PAGE + ((h ^ ((d >> 3) & 1)) * 8); }

// Round-to-nearest-even fp32 pair -> packed bf16 in one instruction (v_cvt_pk_bf16_f32 on gfx950).
GSS_DEV uint32_t cvt_pk_bf16(float lo, float hi) {
  typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
  const bf16x2_t v = {static_cast<__bf16>(lo), static_cast<__bf16>(hi)};
  return __builtin_bit_cast(uint32_t, v);
}

// 2^x with one v_exp_f32 (libm's exp2f wraps it in a denormal range fix-up of five more instructions). Every
// argument here is <= 0 (a score minus its running max) or -inf; results below 2^-126 flush to zero, far below the
// resolution of the bf16 probabilities and the fp32 row sums they feed.
GSS_DEV float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// Direct global -> LDS load of 16 bytes per lane (global_load_lds_dwordx4: lane i writes its 16 bytes at LDS address
// `lds` + 16 i; `lds` is wave-uniform and goes through M0). Written as inline assembly so that the compiler does not
// see an LDS store in flight: it would otherwise wait for every outstanding one (vmcnt(0)) before the next LDS read,
// including the loads of a stage being prefetched while the current one is computed. The kernels order these loads
// themselves: s_waitcnt vmcnt on the issuing wave, then a workgroup barrier, before any wave reads the data. The
// source is a wave-uniform base held in scalar registers plus a 32-bit per-lane byte offset: no 64-bit address
// arithmetic per lane.
GSS_DEV void dma16s(const void* sbase, uint32_t voff, uint32_t lds) {
  asm volatile("global_load_lds_dwordx4 %0, %1" ::"v"(voff), "s"(sbase), "{m0}"(lds) : "memory");
}

// A pointer that is the same in every lane, moved to scalar registers (no-op when it already is there).
GSS_DEV const char* uniform_ptr(const void* p) {
  const uint64_t a = reinterpret_cast<uint64_t>(p);
  const uint32_t lo = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(a));
  const uint32_t hi = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(a >> 32));
  return reinterpret_cast<const char*>((static_cast<uint64_t>(hi) << 32) | lo);
}

// Boundary tiles ts..te-1 of a stage held in LDS (tile t's K at lds_k + (t - ts) * TILE * D, V likewise), t0 the
// first tile that reaches past the prefix L: window row j < W (position L + j) comes from k_win / v_win, positions
// past L + W are zero, and the V chunk that straddles L keeps only its prefix tokens. The thread's first window
// loads are issued before the LDS pass that clears everything past the prefix, so the whole fix costs about one
// memory round trip; a workgroup barrier separates the clearing from the window writes, and the caller follows
// with another before the tiles are read.
template <int D, bool RETIRE = false>
GSS_DEV void fix_boundary(uint16_t* lds_k, uint16_t* lds_v, int ts, int t0, int te, int L, int W,
                          const uint16_t* k_win, const uint16_t* v_win, int64_t win_base, int Hkv, int tid,
                          int nthr) {
  constexpr int CH = D / 8, TILE_EL = TILE * D;
  const int j0 = max(0, t0 * TILE - L), j1 = min(W, te * TILE - L);  // window rows inside these tiles
  const int n_win = max(0, j1 - j0) * CH;                             // their 16-byte chunks (8 dims of a row)
  auto win_addr = [&](int c) { return (win_base + static_cast<int64_t>(j0 + c / CH) * Hkv) * D + (c % CH) * 8; };
  u32x4_t kw = {0u, 0u, 0u, 0u}, vw = {0u, 0u, 0u, 0u};
  if (tid < n_win) {
    kw = *reinterpret_cast<const u32x4_t*>(k_win + win_addr(tid));
    vw = *reinterpret_cast<const u32x4_t*>(v_win + win_addr(tid));
  }
  for (int c = tid; c < (te - t0) * TILE * CH; c += nthr) {  // K chunks past the prefix -> 0
    const int t = t0 + c / (TILE * CH), r = c % (TILE * CH), tok = r / CH, part = r % CH;
    if (t * TILE + tok >= L)
      *reinterpret_cast<u32x4_t*>(&lds_k[(t - ts) * TILE_EL + k_lds_index<D>(tok, part)]) = u32x4_t{0u, 0u, 0u, 0u};
  }
  for (int c = tid; c < (te - t0) * TILE * CH; c += nthr) {  // V tokens past the prefix -> 0
    const int t = t0 + c / (TILE * CH), r = c % (TILE * CH);
    const int pi = r / (2 * D), r2 = r % (2 * D), d = r2 >> 1, h = r2 & 1;
    const int first = t * TILE + pi * PAGE + h * 8;  // absolute position of the chunk's first token
    if (first + 8 <= L) continue;
    uint16_t* dst = &lds_v[(t - ts) * TILE_EL + v_lds_index(pi, d, h, D)];
    u32x4_t v = {0u, 0u, 0u, 0u};
    const int keep = L - first;  // tokens of the chunk inside the prefix (loaded from the page)
    if (keep > 0) {
      v = *reinterpret_cast<const u32x4_t*>(dst);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const uint32_t lo = (2 * e < keep) ? 0x0000ffffu : 0u, hi = (2 * e + 1 < keep) ? 0xffff0000u : 0u;
        v[e] &= (lo | hi);
      }
    }
    *reinterpret_cast<u32x4_t*>(dst) = v;
  }
  __syncthreads();
  for (int c = tid; c < n_win; c += nthr) {  // window rows -> K chunks and V columns
    if (c != tid) {
      kw = *reinterpret_cast<const u32x4_t*>(k_win + win_addr(c));
      vw = *reinterpret_cast<const u32x4_t*>(v_win + win_addr(c));
    }
    const int pos = L + j0 + c / CH, part = c % CH;
    const int t = pos / TILE, tok = pos % TILE;
    *reinterpret_cast<u32x4_t*>(&lds_k[(t - ts) * TILE_EL + k_lds_index<D>(tok, part)]) = kw;
    const int pi = tok / PAGE, h = (tok % PAGE) / 8, e0 = tok % 8;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const int d = part * 8 + e;
      lds_v[(t - ts) * TILE_EL + v_lds_index(pi, d, h, D) + e0] =
          static_cast<uint16_t>((e & 1) ? (vw[e >> 1] >> 16) : (vw[e >> 1] & 0xffffu));
    }
  }
  // RETIRE (callers that keep loads of their own in flight across this call): the window loads of lanes past n_win
  // were never consumed; retire them here (a wait the compiler accounts for), so no load the compiler tracks is
  // pending when the caller's loop continues (it would otherwise wait for every vector memory operation before
  // reusing their registers, prefetched tiles included)
  if (RETIRE) __builtin_amdgcn_s_waitcnt(0);
}

GSS_DEV int valid_splits(int L, int W, int tps) {
  const int n_tiles = (L + W + TILE - 1) / TILE;
  return (n_tiles + tps - 1) / tps;
}

template <int D, int NGW, int RWT>
__global__ void __launch_bounds__(64 * RWT, 2) attn_split_kernel(AttnParams p) {
  using LY = Lds<D>;
  constexpr int NW = RWT;  // waves per workgroup: one per row wave
  constexpr int KS = D / 32;   // MFMA K-steps over the head dim
  constexpr int DT = D / 16;   // 16-row tiles of the head dim (O^T M-tiles)
  constexpr int CH = D / 8;    // 16-byte chunks per K row
  constexpr int TILE_EL = LY::TILE_EL;
  constexpr int TILE_INSTR = TILE * CH / 64;    // direct-load instructions per K (or V) tile
  constexpr int PAGE_INSTR = PAGE * CH / 64;    // instructions per (page, head) block of K (or V)
  extern __shared__ __attribute__((aligned(16))) uint16_t smem[];

  // Grid order: workgroups are dealt to the 8 XCDs round-robin by linear index. The grid enumerates only the units
  // (sequence, kv head, split) that hold keys: unit v of that list (sequence-major, split fastest) runs as workgroups
  // (v / 8) * 8 * RG + rg * 8 + v % 8 for its RG row groups, all of them on XCD v % 8, dispatched back to back (so
  // they share that XCD's L2 for the unit's K/V), and consecutive units on different XCDs. Ragged sequences (whose
  // late splits are empty) thus spread their work evenly over the XCDs; numbering all units instead would put
  // split s of every sequence on XCD s % 8. Each workgroup finds its unit from the device-side lengths (wave 0 scans
  // the valid split counts of the batch), so the host needs no length and the launch stays graph-capturable.
  // the kernel arguments of the exits, the unit scan and the first loads in one scalar batch before the first
  // branch (loaded where first used, they came in dependent round trips)
  asm volatile("" ::"s"(p.RG), "s"(p.n_units), "s"(p.bs), "s"(p.prefix_len), "s"(p.prefix_extra), "s"(p.cap),
               "s"(p.n_split), "s"(p.W), "s"(p.tps), "s"(p.Hkv), "s"(p.q), "s"(p.k_pages), "s"(p.v_pages),
               "s"(p.page_table), "s"(p.pt_stride), "s"(p.TPG), "s"(p.RW), "s"(p.R));
  const int r8 = blockIdx.x % (8 * p.RG);
  const int v = blockIdx.x / (8 * p.RG) * 8 + r8 % 8, rg = r8 / 8;
  if (v >= p.n_units) return;  // padding of the last group of 8 units
  const int tid = threadIdx.x, lane = tid & 63;
  const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
  __shared__ int s_unit[4];  // (sequence, kv head, split, prefix length) of unit v; sequence -1: past the valid units
  if (wv == 0) {
    int base = 0;  // valid units of the sequences before this 64-sequence chunk
    int found = -1, fh = 0, fs = 0, fl = 0;
    for (int c = 0; c < p.bs && found < 0 && base <= v; c += 64) {
      const int bb = c + lane;
      int nvb = 0, Lb = 0;  // valid splits and committed prefix length of sequence bb
      if (bb < p.bs) {
        Lb = min(max(p.prefix_len[bb] + p.prefix_extra, 0), p.cap);
        nvb = min(p.n_split, valid_splits(Lb, p.W, p.tps));
      }
      int inc = nvb * p.Hkv;  // inclusive prefix sum of the chunk's unit counts
#pragma unroll
      for (int o = 1; o < 64; o <<= 1) {
        const int t = __shfl_up(inc, o, 64);
        if (lane >= o) inc += t;
      }
      const int lo = base + inc - nvb * p.Hkv;
      const bool mine = bb < p.bs && v >= lo && v < base + inc;
      const unsigned long long bal = __ballot(mine);
      if (bal) {
        const int src = __builtin_ctzll(bal);
        const int r = __shfl(v - lo, src, 64), nv = __shfl(nvb, src, 64);
        fl = __shfl(Lb, src, 64);
        found = c + src;
        fh = r / nv;
        fs = r % nv;
      }
      base += __shfl(inc, 63, 64);
    }
    if (lane == 0) {
      s_unit[0] = found;
      s_unit[1] = fh;
      s_unit[2] = fs;
      s_unit[3] = fl;
    }
  }
  __syncthreads();
  // workgroup-uniform (readfirstlane keeps them and every address derived from them in scalar registers)
  const int b = __builtin_amdgcn_readfirstlane(s_unit[0]), kvh = __builtin_amdgcn_readfirstlane(s_unit[1]),
            s = __builtin_amdgcn_readfirstlane(s_unit[2]);
  if (b < 0) return;  // past the last valid unit
  const int rw = wv;  // row wave
  const int l16 = lane & 15, g4 = lane >> 4;
  // committed prefix length (from the scan above); clamped to the plan's capacity and to what the page-table row
  // can address, so every key falls in one of the plan's splits and every page-table read is in bounds
  const int L = __builtin_amdgcn_readfirstlane(s_unit[3]);
  const int W = p.W, nc = p.n_causal;
  const int n_tiles = (L + W + TILE - 1) / TILE;
  const int t_beg = s * p.tps, t_end = min(n_tiles, t_beg + p.tps);
  if (t_beg >= t_end) return;  // no key of this sequence in this split (the merge counts only valid splits)
  const int32_t* pt = p.page_table + static_cast<int64_t>(b) * p.pt_stride;
  const int64_t head_stride = static_cast<int64_t>(PAGE) * D;          // elements per (page, kv head) block
  const int64_t win_base = static_cast<int64_t>(b) * W * p.Hkv + kvh;  // window row j: (win_base + j*Hkv)*D
  // this kv head's block of page 0 in the K and V pools; page pg's block is page_stride elements further
  const uint16_t* kp_head = p.k_pages + kvh * head_stride;
  const uint16_t* vp_head = p.v_pages + kvh * head_stride;
  const int64_t page_stride = p.Hkv * head_stride;

  // ---- this wave's query fragments (the B operand of S^T = K Q^T), in registers for the whole kernel: N-tiles
  // nt0 .. nt0 + ng - 1 (ng <= NGW, wave-uniform) of the sequence's R = G*W rows. Rows past R have zero queries and
  // are never written; N-tiles g >= ng are skipped (never computed).
  const int tb_base = p.TPG / p.RW, tb_extra = p.TPG % p.RW;
  const int ng = tb_base + (rw < tb_extra ? 1 : 0);
  __builtin_assume(ng >= NGW - 1 && ng <= NGW);  // the host deals NGW or NGW - 1 tiles to every row wave
  const int nt0 = rg * p.TPG + rw * tb_base + min(rw, tb_extra);
  // the split's page ids -> LDS, once; issued right after the query loads, so both are in flight together
  int* spages = reinterpret_cast<int*>(reinterpret_cast<char*>(smem) + LY::BUF_BYTES);
  auto load_pages = [&]() {
    for (int i = tid; i < (t_end - t_beg) * (TILE / PAGE); i += blockDim.x) {
      const int pos = t_beg * TILE + i * PAGE;
      spages[i] = pos < L ? pt[pos / PAGE] : 0;
    }
  };

  // ---- tile loads, global -> LDS directly (dma16s: lane i of an instruction writes the 16 bytes at the
  // instruction's LDS base + 16 i) into a ring of NSLOT one-tile slots, each K [TILE][D] (XOR-swizzled 16-byte
  // chunks) then V [4 pages][D][16]. Instruction ib of the K (or V) tile covers the 64 chunks of pattern
  // pat = ib % PAGE_INSTR of page ib / PAGE_INSTR, so its page id is wave-uniform. A wave issues one instruction
  // every few clocks at best, so the issue code is kept to scalar work plus at most two VALU operations per load: the
  // per-lane byte offsets of pattern 0 are computed once; pattern pat adds pat * 1024 bytes (in the scalar base) and,
  // for K, XORs (pat * 64 / CH) % CH into the lane's swizzled chunk index. Loads are unconditional: pages past the
  // prefix read page 0 (in bounds) and the boundary fix overwrites those positions after the loads have landed.
  constexpr int NSLOT = LY::NSLOT;
  constexpr int N_INSTR = 2 * TILE_INSTR;                // K then V instructions of a tile
  constexpr int PER_WAVE = (N_INSTR + NW - 1) / NW;      // this wave's: wv, wv + NW, ...
  const uint32_t ktok0 = lane / CH;                      // the lane's token within a K pattern
  const uint32_t kc0 = (lane % CH) ^ (ktok0 & (CH - 1));  // its swizzled chunk index, pattern 0
  const uint32_t k_lane = ktok0 * D * 2;
  const uint32_t v_lane = ((lane >> 1) * PAGE + ((lane & 1) ^ ((lane >> 4) & 1)) * 8) * 2;  // (d, half) chunk
  const char* k_base = uniform_ptr(kp_head);
  const char* v_base = uniform_ptr(vp_head);
  const uint32_t page_bytes = static_cast<uint32_t>(page_stride * 2);
  const uint32_t lds0 = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(reinterpret_cast<uintptr_t>(smem)));
  auto issue_tile = [&](int i) __attribute__((always_inline)) {  // tile t_beg + i -> slot i % NSLOT
    const uint32_t slot = lds0 + (i % NSLOT) * (LY::SLOT_EL * 2);
    const int pgv = lane < TILE / PAGE ? spages[i * (TILE / PAGE) + lane] : 0;
    // the per-instruction scalars are a few operations from wv; kept opaque here so the compiler recomputes them
    // per tile instead of holding a register for each across the tile loop
    uint32_t w = static_cast<uint32_t>(wv);
    asm volatile("" : "+s"(w));
    __builtin_assume(w < NW);
#pragma unroll
    for (uint32_t k = 0; k < PER_WAVE; ++k) {
      const uint32_t ii = w + k * NW;
      if (PER_WAVE * NW != N_INSTR && ii >= N_INSTR) break;  // wave-uniform; only when NW does not divide it
      const bool is_v = ii >= TILE_INSTR;
      const uint32_t ib = is_v ? ii - TILE_INSTR : ii;
      const uint32_t pblk = ib / PAGE_INSTR, pat = ib % PAGE_INSTR;
      const uint32_t page = __builtin_amdgcn_readlane(pgv, pblk);
      const char* sb = (is_v ? v_base : k_base) + (static_cast<uint64_t>(page) * page_bytes + pat * 1024);
      const uint32_t xr = (pat * (64 / CH)) & (CH - 1);
      dma16s(sb, is_v ? v_lane : k_lane + ((kc0 ^ xr) << 4), slot + (is_v ? TILE_EL * 2 : 0) + ib * 1024);
    }
  };
  // Tile i reaching past the prefix: K rows and V columns of positions >= L get the window rows (staging) or zero,
  // and the V chunk that straddles L keeps only its prefix tokens.
  auto fix_tile = [&](int i) {
    const int t = t_beg + i;
    if ((t + 1) * TILE <= L) return false;
    uint16_t* lds_k = smem + (i % NSLOT) * LY::SLOT_EL;
    fix_boundary<D, true>(lds_k, lds_k + TILE_EL, t, t, t + 1, L, W, p.k_win, p.v_win, win_base, p.Hkv, tid,
                          blockDim.x);
    return true;
  };
  const int hsw = (l16 >> 3) & 1;  // the V half swap of head dims d with bit 3 set (d = dt*16 + l16)
  const int vrd = ((g4 >> 1) ^ hsw) * 8 + (g4 & 1) * 4;
  
  const int n_t = t_end - t_beg;

  // The wave's work for its NG N-tiles, NG a compile-time count (NGW or NGW - 1, dealt by the host), so the MFMA
  // sequence has no per-tile branches. Both instantiations run the same workgroup barriers in the same order.
  auto body = [&](auto ngc) {
    constexpr int NG = decltype(ngc)::value;
    // ---- query fragments (the B operand of S^T = K Q^T), in registers for the whole kernel: N-tiles
    // nt0 .. nt0 + NG - 1 of the sequence's R = G*W rows. Rows past R have zero queries and are never written.
    bf16x8_t qf[NG][KS];
#pragma unroll
    for (int g = 0; g < NG; ++g) {
      const int n = (nt0 + g) * 16 + l16;
      const int nn = n < p.R ? n : 0;  // padding rows read row 0 (in bounds) and are zeroed
      const uint16_t* qrow = p.q + ((static_cast<int64_t>(b) * W + nn / p.G) * p.Hq + kvh * p.G + nn % p.G) * D;
#pragma unroll
      for (int ks = 0; ks < KS; ++ks)
        qf[g][ks] = n < p.R ? *reinterpret_cast<const bf16x8_t*>(qrow + ks * 32 + g4 * 8) : bf16x8_t{};
    }
    load_pages();
    // queries pre-scaled by scale * log2(e) (fp32 product rounded to bf16), so the MFMA yields log2-domain scores
#pragma unroll
    for (int g = 0; g < NG; ++g)
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
        const u32x4_t u = __builtin_bit_cast(u32x4_t, qf[g][ks]);
        u32x4_t r;
#pragma unroll
        for (int e = 0; e < 4; ++e)
          r[e] = cvt_pk_bf16(__uint_as_float(u[e] << 16) * p.scale_log2,
                             __uint_as_float(u[e] & 0xffff0000u) * p.scale_log2);
        qf[g][ks] = __builtin_bit_cast(bf16x8_t, r);
      }
    __syncthreads();

    // ---- online softmax, private to the wave: it scores the two key halves hh of every tile of the split (32
    // keys, m-tiles 2 hh and 2 hh + 1, one step each) for its NG N-tiles. Scores come out of the MFMA in the log2
    // domain (the queries are pre-scaled). Each row keeps a reference max m that trails its running max by at most
    // RESCALE_SLACK, and P^T = 2^(s - m) <= 2^RESCALE_SLACK; only when some row's max exceeds its reference by more
    // than the slack (rare after the first tiles) does the wave take the row maxima (two xor-shuffles over the row's
    // lanes), move the references and rescale O and l. P^T is packed to bf16 in the lane that scored it, and
    // O^T += V^T P^T over one K-step of 32 keys.
    floatx4_t o[NG][DT];
    float m_run[NG], l_run[NG];
#pragma unroll
    for (int g = 0; g < NG; ++g) {
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) o[g][dt] = floatx4_t{0.f, 0.f, 0.f, 0.f};
      m_run[g] = -INFINITY;
      l_run[g] = 0.f;
    }
    // nothing the compiler tracks may be outstanding when the tile loop starts: a load or spill store still pending
    // at the loop header would make it wait for every vector memory operation inside the loop, the prefetched tiles
    // included (a real s_waitcnt, which the compiler's wait insertion accounts for)
    __builtin_amdgcn_s_waitcnt(0);
    static_assert(NSLOT == 2, "one tile in flight: the wait below is for every load");
    issue_tile(0);
    for (int i = 0; i < n_t; ++i) {
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // this wave's loads of tile i (the only ones in flight)
      __syncthreads();  // every wave's loads of tile i have landed; every wave is done with tile i - 1's slot
      if (fix_tile(i)) __syncthreads();  // block-uniform condition
      if (i + NSLOT - 1 < n_t) issue_tile(i + NSLOT - 1);  // into the slot of tile i - 1
      const int tb = (t_beg + i) * TILE;
      const uint16_t* tk = smem + (i % NSLOT) * LY::SLOT_EL;
      const uint16_t* tv = tk + TILE_EL;
#pragma unroll 1
      for (int hh = 0; hh < 2; ++hh) {  // the tile's two key halves (32 keys each), one online-softmax step each
        // scores: the half's K fragments (2 m-tiles x KS K-steps) are read in two batches, the second in flight
        // under the first batch's MFMAs; K-step outer and m-tile inner, each accumulator over the K-steps in order
        floatx4_t sacc[NG][2];
#pragma unroll
        for (int g = 0; g < NG; ++g) sacc[g][0] = sacc[g][1] = floatx4_t{0.f, 0.f, 0.f, 0.f};
        constexpr int KB = KS;  // fragments per batch (i2 = ks * 2 + mt)
        auto kfrag = [&](int i2) {
          return *reinterpret_cast<const bf16x8_t*>(
              &tk[k_lds_index<D>((2 * hh + (i2 & 1)) * 16 + l16, (i2 >> 1) * 4 + g4)]);
        };
        bf16x8_t kf[2][KB];
#pragma unroll
        for (int j = 0; j < KB; ++j) kf[0][j] = kfrag(j);
#pragma unroll
        for (int bt = 0; bt < 2; ++bt) {
          if (bt == 0) {
#pragma unroll
            for (int j = 0; j < KB; ++j) kf[1][j] = kfrag(KB + j);
          }
#pragma unroll
          for (int j = 0; j < KB; ++j) {
            const int i2 = bt * KB + j;
#pragma unroll
            for (int g = 0; g < NG; ++g)
              sacc[g][i2 & 1] =
                  __builtin_amdgcn_mfma_f32_16x16x32_bf16(kf[bt][j], qf[g][i2 >> 1], sacc[g][i2 & 1], 0, 0, 0);
          }
        }
        // the V^T fragments do not depend on the scores: the first half is read now, under the softmax, the rest
        // under the first half's MFMAs
        bf16x8_t vf[DT];
        auto vfrag = [&](int dt) {
          const int d = dt * 16 + l16;
          const u32x2_t v0 = *reinterpret_cast<const u32x2_t*>(&tv[((2 * hh) * D + d) * PAGE + vrd]);
          const u32x2_t v1 = *reinterpret_cast<const u32x2_t*>(&tv[((2 * hh + 1) * D + d) * PAGE + vrd]);
          return __builtin_bit_cast(bf16x8_t, u32x4_t{v0[0], v0[1], v1[0], v1[1]});
        };
#pragma unroll
        for (int dt = 0; dt < DT / 2; ++dt) vf[dt] = vfrag(dt);
        if (tb + TILE > L) {  // keys past the prefix: the window mask (wave-uniform branch)
#pragma unroll
          for (int g = 0; g < NG; ++g) {
            const int n = (nt0 + g) * 16 + l16;
            const int roww = (n < p.R ? n : 0) / p.G;  // the row's window index
#pragma unroll
            for (int mt = 0; mt < 2; ++mt)
#pragma unroll
              for (int e = 0; e < 4; ++e) {
                const int pos = tb + (2 * hh + mt) * 16 + g4 * 4 + e;
                const int wj = pos - L;
                const bool vis = pos < L || (wj < W && (roww >= nc || wj <= roww));
                if (!vis) sacc[g][mt][e] = -INFINITY;
              }
          }
        }
        bf16x8_t pb[NG];
#pragma unroll
        for (int g = 0; g < NG; ++g) {
          // the lane's own max over its 8 scores of the row; a row's reference moves only when its max exceeds it by
          // more than the slack (or on its first visible keys, m_run = -inf), so the row max over the row's 4 lanes
          // (two xor-shuffles) is needed only when some lane's own max does: the wave votes first. Keys that are all
          // masked (mx = -inf) never move a reference.
          float mx = fmaxf(fmaxf(fmaxf(sacc[g][0][0], sacc[g][0][1]), fmaxf(sacc[g][0][2], sacc[g][0][3])),
                           fmaxf(fmaxf(sacc[g][1][0], sacc[g][1][1]), fmaxf(sacc[g][1][2], sacc[g][1][3])));
          if (__any(mx > m_run[g] + RESCALE_SLACK)) {  // wave-uniform: rescale O and l of the rows that moved
            mx = fmaxf(mx, lane_xor(mx, 16));
            mx = fmaxf(mx, lane_xor(mx, 32));
            const float m_new = mx > m_run[g] + RESCALE_SLACK ? mx : m_run[g];
            // 1 for rows that keep their reference (also -inf: no visible key yet, where -inf - -inf would be NaN),
            // 0 on a row's first visible keys
            const float alpha = m_new == m_run[g] ? 1.f : fast_exp2(m_run[g] - m_new);
            m_run[g] = m_new;
            l_run[g] *= alpha;
#pragma unroll
            for (int dt = 0; dt < DT; ++dt) o[g][dt] = o[g][dt] * alpha;
          }
          const float m_use = m_run[g] == -INFINITY ? 0.f : m_run[g];  // a row with no visible key yet: P = 0
          uint32_t pk[4];
          float ls = 0.f;
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            const floatx4_t& sv = sacc[g][j >> 1];
            const float p0 = fast_exp2(sv[(2 * j) & 3] - m_use);
            const float p1 = fast_exp2(sv[(2 * j + 1) & 3] - m_use);
            ls += p0 + p1;
            pk[j] = cvt_pk_bf16(p0, p1);
          }
          l_run[g] += ls;
          pb[g] = __builtin_bit_cast(bf16x8_t, u32x4_t{pk[0], pk[1], pk[2], pk[3]});
        }
#pragma unroll
        for (int dt = DT / 2; dt < DT; ++dt) vf[dt] = vfrag(dt);
#pragma unroll
        for (int dt = 0; dt < DT; ++dt)
#pragma unroll
          for (int g = 0; g < NG; ++g)
            o[g][dt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(vf[dt], pb[g], o[g][dt], 0, 0, 0);
      }
    }

    // ---- the wave's rows: the row sums over the 4 lane groups, then O / l (bf16) and (m, l), or the output
#pragma unroll
    for (int g = 0; g < NG; ++g) {
      l_run[g] += lane_xor(l_run[g], 16);
      l_run[g] += lane_xor(l_run[g], 32);
      const int n = (nt0 + g) * 16 + l16;
      if (n >= p.R) continue;
      const float inv = l_run[g] > 0.f ? 1.f / l_run[g] : 0.f;
      uint16_t* orow;
      if (p.n_split == 1) {
        orow = p.out + ((static_cast<int64_t>(b) * W + n / p.G) * p.Hq + kvh * p.G + n % p.G) * D;
      } else {
        const int64_t rowid = (static_cast<int64_t>(b) * p.Hkv + kvh) * p.R + n;  // (m, l): [bs, Hkv, R, n_split]
        orow = p.ws_o + ((static_cast<int64_t>(b) * p.Hkv + kvh) * p.n_split + s) * p.R * D +
               static_cast<int64_t>(n) * D;
        if (g4 == 0) {
          p.ws_ml[(rowid * p.n_split + s) * 2 + 0] = m_run[g];
          p.ws_ml[(rowid * p.n_split + s) * 2 + 1] = l_run[g];
        }
      }
#pragma unroll
      for (int dt = 0; dt < DT; ++dt)
        *reinterpret_cast<u32x2_t*>(orow + dt * 16 + g4 * 4) = u32x2_t{
            cvt_pk_bf16(o[g][dt][0] * inv, o[g][dt][1] * inv), cvt_pk_bf16(o[g][dt][2] * inv, o[g][dt][3] * inv)};
    }
  };
  static_assert(NGW >= 2, "row waves take NGW or NGW - 1 >= 1 N-tiles");
  if (ng == NGW)
    body(std::integral_constant<int, NGW>{});
  else
    body(std::integral_constant<int, NGW - 1>{});
}

// Row-group kernel for small batches (bs * Hkv below the wide threshold), where the chip must be filled from few
// key splits: the R rows are cut into row groups of up to RG_NTG N-tiles, each its own workgroup (the groups of a
// unit share its K/V through the XCD's L2), 8 waves = (tile lane, key half) pairs over stages of RG_LANES tiles, one
// running max per row shared by the waves through LDS, and the 8 partial (O, l) summed in wave order.
template <int D, int NG>
__global__ void __launch_bounds__(RG_THREADS, 1) attn_rowgroup_kernel(AttnParams p) {
  constexpr int KS = D / 32;   // MFMA K-steps over the head dim
  constexpr int DT = D / 16;   // 16-row tiles of the head dim (O^T M-tiles)
  constexpr int CH = D / 8;    // 16-byte chunks per K row
  constexpr int TILE_EL = LdsRG<D>::TILE_EL;
  constexpr int TILE_INSTR = TILE * CH / 64;    // direct-load instructions per K (or V) tile
  constexpr int STAGE_INSTR = RG_LANES * TILE_INSTR;
  constexpr int PAGE_INSTR = PAGE * CH / 64;    // instructions per (page, head) block of K (or V)
  constexpr int NW = RG_THREADS / 64;
  extern __shared__ __attribute__((aligned(16))) uint16_t smem[];
  uint16_t* lds_k = smem;
  uint16_t* lds_v = smem + LdsRG<D>::V_OFF;

  // The kernel arguments the exits and the first loads need, in one batch before the first branch: loaded where
  // first used, they came in three dependent scalar round trips ahead of the prefix length's own.
  asm volatile("" ::"s"(p.RG), "s"(p.n_units), "s"(p.n_split), "s"(p.Hkv), "s"(p.prefix_len), "s"(p.prefix_extra),
               "s"(p.cap), "s"(p.tps), "s"(p.W), "s"(p.q), "s"(p.k_pages), "s"(p.v_pages), "s"(p.page_table),
               "s"(p.pt_stride));
  // grid order: as attn_split_kernel (units spread over the XCDs, the row groups of a unit on one XCD)
  const int r8 = blockIdx.x % (8 * p.RG);
  const int u = blockIdx.x / (8 * p.RG) * 8 + r8 % 8, rg = r8 / 8;
  if (u >= p.n_units) return;  // padding of the last group of 8 units
  const int s = u % p.n_split, kvh = (u / p.n_split) % p.Hkv, b = u / (p.n_split * p.Hkv);
  const int tid = threadIdx.x, lane = tid & 63;
  const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int kq = wv >> 1, half = wv & 1;                      // tile lane, key half (32 keys) of this wave
  const int l16 = lane & 15, g4 = lane >> 4;
  // committed prefix length; clamped to the plan's capacity and to what the page-table row can address, so every
  // key falls in one of the plan's splits and every page-table read is in bounds
  const int L = min(max(p.prefix_len[b] + p.prefix_extra, 0), p.cap);
  const int W = p.W, nc = p.n_causal;
  const int n_tiles = (L + W + TILE - 1) / TILE;
  const int t_beg = s * p.tps, t_end = min(n_tiles, t_beg + p.tps);
  if (t_beg >= t_end) return;  // no key of this sequence in this split (the merge counts only valid splits)
  const int32_t* pt = p.page_table + static_cast<int64_t>(b) * p.pt_stride;
  const int64_t head_stride = static_cast<int64_t>(PAGE) * D;          // elements per (page, kv head) block
  const int64_t win_base = static_cast<int64_t>(b) * W * p.Hkv + kvh;  // window row j: (win_base + j*Hkv)*D

  // ---- this row group's query fragments (the B operand of S^T = K Q^T), in registers for the whole kernel.
  // NG = min(NTG, N-tiles of the window) is a compile-time count: every row group computes NG N-tiles (rows past R
  // have zero queries and are not written), so the MFMA sequence has no data-dependent branches.
  const int row0 = rg * NG * 16;
  bf16x8_t qf[NG][KS];
  int roww[NG];
#pragma unroll
  for (int g = 0; g < NG; ++g) {
    const int n = row0 + g * 16 + l16;
    const int nn = n < p.R ? n : 0;  // padding rows read row 0 (in bounds) and are zeroed
    roww[g] = nn / p.G;
    const uint16_t* qrow = p.q + ((static_cast<int64_t>(b) * W + nn / p.G) * p.Hq + kvh * p.G + nn % p.G) * D;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks)
      qf[g][ks] = n < p.R ? *reinterpret_cast<const bf16x8_t*>(qrow + ks * 32 + g4 * 8) : bf16x8_t{};
  }

  // ---- stage loads, global -> LDS directly (global_load_lds_dwordx4: lane i of an instruction writes the 16 bytes
  // at the instruction's LDS base + 16 i). Every instruction covers 64 chunks of one (page, head) block, so its page
  // id is wave-uniform (lane j of `pgv` holds the id of the stage's page j; readlane broadcasts it), and since the
  // waves take the instructions round-robin and NW is a multiple of PAGE_INSTR, a wave always covers the same 64
  // chunks of a block: its per-lane source offsets (with the K swizzle and the V half swap) are computed once.
  // Chunks of positions >= L are not loaded.
  static_assert(NW % PAGE_INSTR == 0, "a wave's chunk pattern must not change between instructions");
  const int pat = wv % PAGE_INSTR;
  const int kr = pat * 64 + lane, ktok = kr / CH;                       // token within the page block (< 16)
  const int koff = ktok * D + ((kr % CH) ^ (ktok & (CH - 1))) * 8;      // elements within the (page, head) block
  const int vr = kr % (2 * D), vd = vr >> 1, vh = (vr & 1) ^ ((vd >> 3) & 1);
  const int voff = vd * PAGE + vh * 8;
  auto stage_pages = [&](int st) {
    const int pos = (t_beg + st * RG_LANES) * TILE + lane * PAGE;
    return (lane < RG_LANES * (TILE / PAGE) && pos < L) ? pt[pos / PAGE] : 0;
  };
  // A wave issues one instruction every few clocks at best, so each load is a handful of scalar operations on
  // wave-uniform values (the page base in scalar registers, the lane's byte offset computed once above).
  const uint32_t koff_b = koff * 2, voff_b = voff * 2;
  const char* k_base = uniform_ptr(p.k_pages + kvh * head_stride);
  const char* v_base = uniform_ptr(p.v_pages + kvh * head_stride);
  const uint32_t page_bytes = static_cast<uint32_t>(p.Hkv * head_stride * 2);
  const uint32_t lds0 = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(reinterpret_cast<uintptr_t>(smem)));
  auto issue_stage = [&](int st, int pgv) __attribute__((always_inline)) {
    // the page ids (and the queries) have landed before the first load is issued: the compiler does not count the
    // direct-to-LDS loads, so a wait it placed for pgv between them would also wait for every load issued before it
    __builtin_amdgcn_s_waitcnt(0);
    // the per-instruction scalars are a few operations from wv; kept opaque so they are not held across stages
    uint32_t w = static_cast<uint32_t>(wv);
    asm volatile("" : "+s"(w));
    __builtin_assume(w < NW);
#pragma unroll
    for (uint32_t i = 0; i < 2 * STAGE_INSTR / NW; ++i) {
      const uint32_t ii = i * NW + w;
      const bool is_v = ii >= STAGE_INSTR;
      const uint32_t iv = is_v ? ii - STAGE_INSTR : ii;
      const int t = t_beg + st * RG_LANES + static_cast<int>(iv / TILE_INSTR);
      if (t >= t_end) continue;
      const uint32_t pblk = iv / PAGE_INSTR;                                 // page of the stage (tile * 4 + page)
      const int pos0 = t * TILE + static_cast<int>(pblk % (TILE / PAGE)) * PAGE;  // first position of that page
      const uint32_t page = __builtin_amdgcn_readlane(pgv, pblk);
      const char* sb = (is_v ? v_base : k_base) + static_cast<uint64_t>(page) * page_bytes;
      const uint32_t lds = lds0 + (is_v ? LdsRG<D>::V_OFF * 2 : 0) + iv * 1024;
      // chunks of positions >= L are not loaded (the lane's first position in the page is below PAGE, so this one
      // compare also keeps every chunk of a page that lies inside the prefix)
      if (pos0 + (is_v ? vh * 8 : ktok) < L) dma16s(sb, is_v ? voff_b : koff_b, lds);
    }
  };
  // Tiles that reach past the prefix: K rows and V columns of positions >= L get the window rows (staging) or zero,
  // and the V chunk that straddles L keeps only its prefix tokens.
  auto fix_stage = [&](int st) {
    const int ts = t_beg + st * RG_LANES, te = min(t_end, ts + RG_LANES);
    const int t0 = max(ts, L / TILE);
    if (t0 >= te) return false;
    fix_boundary<D>(lds_k, lds_v, ts, t0, te, L, W, p.k_win, p.v_win, win_base, p.Hkv, tid, RG_THREADS);
    return true;
  };

  // ---- softmax with one running max per row shared by the whole workgroup -----------------------------------
  // Each stage: every wave scores its 32 keys (tile lane kq, key half `half`; m-tiles 2*half, 2*half+1) for the NG
  // N-tiles, the waves exchange their row maxima through LDS, and all of them rescale (from the second stage on)
  // and accumulate against the same running max. The 8 partial (O, l) of the workgroup are then on one scale and
  // combine by plain sums in a fixed order. Every K and V fragment read from LDS feeds the MFMAs of all NG N-tiles.
  float* smax = reinterpret_cast<float*>(reinterpret_cast<char*>(smem) + LdsRG<D>::BYTES);  // [NW][NG][16]
  floatx4_t o[NG][DT];
  float m_run[NG], l_run[NG];
#pragma unroll
  for (int g = 0; g < NG; ++g) {
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) o[g][dt] = floatx4_t{0.f, 0.f, 0.f, 0.f};
    m_run[g] = -INFINITY;
    l_run[g] = 0.f;
  }
  const uint16_t* tk = lds_k + kq * TILE_EL;
  const uint16_t* tv = lds_v + kq * TILE_EL;
  const int hsw = (l16 >> 3) & 1;  // the V half swap of head dims d with bit 3 set (d = dt*16 + l16)
  const int vrd = ((g4 >> 1) ^ hsw) * 8 + (g4 & 1) * 4;

  const int n_stages = (t_end - t_beg + RG_LANES - 1) / RG_LANES;
  int pgv = stage_pages(0);
  for (int st = 0; st < n_stages; ++st) {
    if (st > 0) __syncthreads();  // the previous stage's compute is done with LDS
    issue_stage(st, pgv);
    if (st + 1 < n_stages) pgv = stage_pages(st + 1);
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    if (fix_stage(st)) __syncthreads();  // block-uniform condition
    const int tb = (t_beg + st * RG_LANES + kq) * TILE;
    const bool has_tile = tb < t_end * TILE;  // wave-uniform
    floatx4_t sacc[NG][2];
#pragma unroll
    for (int g = 0; g < NG; ++g)
#pragma unroll
      for (int mt = 0; mt < 2; ++mt) sacc[g][mt] = floatx4_t{-INFINITY, -INFINITY, -INFINITY, -INFINITY};
    if (has_tile) {
#pragma unroll
      for (int g = 0; g < NG; ++g)
#pragma unroll
        for (int mt = 0; mt < 2; ++mt) sacc[g][mt] = floatx4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
        bf16x8_t a[2];
#pragma unroll
        for (int mt = 0; mt < 2; ++mt)
          a[mt] = *reinterpret_cast<const bf16x8_t*>(&tk[k_lds_index<D>((2 * half + mt) * 16 + l16, ks * 4 + g4)]);
#pragma unroll
        for (int g = 0; g < NG; ++g)
#pragma unroll
          for (int mt = 0; mt < 2; ++mt)
            sacc[g][mt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[mt], qf[g][ks], sacc[g][mt], 0, 0, 0);
      }
      if (tb + TILE > L) {  // keys past the prefix: the window mask (wave-uniform branch)
#pragma unroll
        for (int g = 0; g < NG; ++g)
#pragma unroll
          for (int mt = 0; mt < 2; ++mt)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
              const int pos = tb + (2 * half + mt) * 16 + g4 * 4 + i;
              const int wj = pos - L;
              const bool vis = pos < L || (wj < W && (roww[g] >= nc || wj <= roww[g]));
              if (!vis) sacc[g][mt][i] = -INFINITY;
            }
      }
    }
    // row maxima of this wave's keys -> LDS; the stage maximum of every row over the 8 waves (in wave order)
#pragma unroll
    for (int g = 0; g < NG; ++g) {
      float mx = fmaxf(fmaxf(fmaxf(sacc[g][0][0], sacc[g][0][1]), fmaxf(sacc[g][0][2], sacc[g][0][3])),
                       fmaxf(fmaxf(sacc[g][1][0], sacc[g][1][1]), fmaxf(sacc[g][1][2], sacc[g][1][3])));
      mx = fmaxf(mx, lane_xor(mx, 16));
      mx = fmaxf(mx, lane_xor(mx, 32));
      if (g4 == 0) smax[(wv * NG + g) * 16 + l16] = mx;
    }
    __syncthreads();
#pragma unroll
    for (int g = 0; g < NG; ++g) {
      float mx = smax[g * 16 + l16];
#pragma unroll
      for (int w = 1; w < NW; ++w) mx = fmaxf(mx, smax[(w * NG + g) * 16 + l16]);
      const float m_new = fmaxf(m_run[g], mx * p.scale_log2);
      const float m_use = m_new == -INFINITY ? 0.f : m_new;
      if (st > 0) {  // rescale to the new running max (the first stage starts from zero)
        const float alpha = fast_exp2(m_run[g] - m_use);
        l_run[g] *= alpha;
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) o[g][dt] = o[g][dt] * alpha;
      }
      m_run[g] = m_new;
      if (has_tile) {
        const float nm = -m_use;
        float ls = 0.f;
        uint32_t pk[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const float p0 = fast_exp2(__builtin_fmaf(sacc[g][j >> 1][(2 * j) & 3], p.scale_log2, nm));
          const float p1 = fast_exp2(__builtin_fmaf(sacc[g][j >> 1][(2 * j + 1) & 3], p.scale_log2, nm));
          ls += p0 + p1;
          pk[j] = cvt_pk_bf16(p0, p1);
        }
        l_run[g] += ls;
        // P^T operand: slots 0..3 = m-tile 2*half values, slots 4..7 = m-tile 2*half+1 values
        const bf16x8_t pb = __builtin_bit_cast(bf16x8_t, u32x4_t{pk[0], pk[1], pk[2], pk[3]});
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) {
          const int d = dt * 16 + l16;
          const u32x2_t v0 = *reinterpret_cast<const u32x2_t*>(&tv[((2 * half) * D + d) * PAGE + vrd]);
          const u32x2_t v1 = *reinterpret_cast<const u32x2_t*>(&tv[((2 * half + 1) * D + d) * PAGE + vrd]);
          const bf16x8_t va = __builtin_bit_cast(bf16x8_t, u32x4_t{v0[0], v0[1], v1[0], v1[1]});
          o[g][dt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(va, pb, o[g][dt], 0, 0, 0);
        }
      }
    }
  }

  // ---- combine: every partial is on the workgroup's running max, so the 8 waves' (O, l) add up. Each wave stores
  // its O (bf16) and l; then the waves share the (N-tile, 16-dim block) sums, each over the 8 waves in wave order.
#pragma unroll
  for (int g = 0; g < NG; ++g) {
    l_run[g] += lane_xor(l_run[g], 16);
    l_run[g] += lane_xor(l_run[g], 32);
  }
  __syncthreads();  // every wave is done with the K/V stage: reuse it as scratch
  char* scr = reinterpret_cast<char*>(smem);
#pragma unroll
  for (int g = 0; g < NG; ++g) {
    char* slot = scr + (wv * NG + g) * LdsRG<D>::SCR_BYTES;
    u32x2_t* so = reinterpret_cast<u32x2_t*>(slot);
#pragma unroll
    for (int dt = 0; dt < DT; ++dt)
      so[dt * 64 + lane] = u32x2_t{cvt_pk_bf16(o[g][dt][0], o[g][dt][1]), cvt_pk_bf16(o[g][dt][2], o[g][dt][3])};
    if (g4 == 0) reinterpret_cast<float*>(slot + DT * 64 * 8)[l16] = l_run[g];
  }
  __syncthreads();
  for (int blk = wv; blk < NG * DT; blk += NW) {
    const int g = blk / DT, dt = blk % DT;
    floatx4_t acc = {0.f, 0.f, 0.f, 0.f};
    float lc = 0.f;
#pragma unroll
    for (int w = 0; w < NW; ++w) {
      const char* slot = scr + (w * NG + g) * LdsRG<D>::SCR_BYTES;
      const u32x2_t u = reinterpret_cast<const u32x2_t*>(slot)[dt * 64 + lane];
      acc += floatx4_t{__uint_as_float(u[0] << 16), __uint_as_float(u[0] & 0xffff0000u), __uint_as_float(u[1] << 16),
                       __uint_as_float(u[1] & 0xffff0000u)};
      lc += reinterpret_cast<const float*>(slot + DT * 64 * 8)[l16];
    }
    const int n = row0 + g * 16 + l16;
    if (n >= p.R) continue;
    float mc = m_run[0];  // the running max of N-tile g's rows (the same in every wave of the workgroup)
#pragma unroll
    for (int k = 1; k < NG; ++k)
      if (k == g) mc = m_run[k];
    const float inv = lc > 0.f ? 1.f / lc : 0.f;
    uint16_t* orow;
    if (p.n_split == 1) {
      orow = p.out + ((static_cast<int64_t>(b) * W + n / p.G) * p.Hq + kvh * p.G + n % p.G) * D;
    } else {
      const int64_t rowid = (static_cast<int64_t>(b) * p.Hkv + kvh) * p.R + n;  // (m, l): [bs, Hkv, R, n_split]
      orow = p.ws_o + ((static_cast<int64_t>(b) * p.Hkv + kvh) * p.n_split + s) * p.R * D +
             static_cast<int64_t>(n) * D;
      if (dt == 0 && g4 == 0) {
        p.ws_ml[(rowid * p.n_split + s) * 2 + 0] = mc;
        p.ws_ml[(rowid * p.n_split + s) * 2 + 1] = lc;
      }
    }
    *reinterpret_cast<u32x2_t*>(orow + dt * 16 + g4 * 4) =
        u32x2_t{cvt_pk_bf16(acc[0] * inv, acc[1] * inv), cvt_pk_bf16(acc[2] * inv, acc[3] * inv)};
  }
}


// Combine the valid splits of each (sequence, kv head, row): one wave (and workgroup) per row. A split's partial
// row is D bf16 = D/8 chunks of 16 bytes, so the wave reads SGW = 64 / (D/8) split rows per instruction (lane =
// split group sg x chunk dc) and issues the loads of up to PRE * SGW splits before it waits; the row's (m, l) of every
// split (stored contiguously per row) are read in the same round, one split per lane. Weights w_s = l_s * 2^(m_s - M)
// follow from one wave max; lane (sg, dc) sums w_s * O_s over s = sg mod SGW with fused multiply-adds in split order,
// and the split groups combine by xor-shuffles in a fixed order. Splits past the valid count hold whatever an earlier
// call left in the workspace and are neither loaded nor weighted. A split that holds none of the row's visible keys
// has w_s = 0 exactly.
template <int D>
__global__ void __launch_bounds__(64) window_attn_merge(AttnParams p) {
  constexpr int CPL = D / 8, SGW = 64 / CPL, PRE = 16, MLR = MAX_SPLIT / 64;
  static_assert(PRE * SGW <= MAX_SPLIT, "the first round's splits must have weights");
  const int lane = threadIdx.x & 63;
  const int64_t rid = blockIdx.x;  // (b * Hkv + kvh) * R + n
  const int n = static_cast<int>(rid % p.R), bh = static_cast<int>(rid / p.R), kvh = bh % p.Hkv, b = bh / p.Hkv;
  const int sg = lane / CPL, dc = lane % CPL;
  const int ns = p.n_split;
  const float2* ml = reinterpret_cast<const float2*>(p.ws_ml) + rid * ns;
  const uint16_t* obase = p.ws_o + static_cast<int64_t>(bh) * ns * p.R * D + static_cast<int64_t>(n) * D + dc * 8;
  const int64_t ostride = static_cast<int64_t>(p.R) * D;
  // one round of loads: the length, and (m, l) and the first PRE * SGW partial rows of every split of the workspace
  // (in bounds whatever the length); the valid count masks them afterwards
  const int L = min(max(p.prefix_len[b] + p.prefix_extra, 0), p.cap);
  // The loads are unconditional (splits past the workspace read split 0, which every row with keys has written), so
  // no loaded value joins a branch: a register copy at such a join made the compiler wait for every load issued
  // before it, splitting the round in two.
  float2 mlv[MLR];
#pragma unroll
  for (int k = 0; k < MLR; ++k) {
    const int sp = lane + 64 * k;
    mlv[k] = ml[sp < ns ? sp : 0];
  }
  u32x4_t u[PRE];
#pragma unroll
  for (int k = 0; k < PRE; ++k) {
    const int sp = sg + k * SGW;
    u[k] = *reinterpret_cast<const u32x4_t*>(obase + (sp < ns ? sp : 0) * ostride);
  }
  const int nv = min(ns, valid_splits(L, p.W, p.tps));
  float mx = lane < nv ? mlv[0].x : -INFINITY;
#pragma unroll
  for (int k = 1; k < MLR; ++k) mx = fmaxf(mx, lane + 64 * k < nv ? mlv[k].x : -INFINITY);
  const float M = wave_max(mx);
  const float Mu = M == -INFINITY ? 0.f : M;
  float wk[MLR];  // weight of split lane + 64 k (0 past the valid count)
  float den = 0.f;
#pragma unroll
  for (int k = 0; k < MLR; ++k) {
    wk[k] = lane + 64 * k < nv ? mlv[k].y * exp2f(mlv[k].x - Mu) : 0.f;
    den += wk[k];
  }
  den = wave_sum(den);
  auto weight = [&](int sp) {  // w of split sp (< MAX_SPLIT), from lane sp % 64
    float w = 0.f;
#pragma unroll
    for (int k = 0; k < MLR; ++k) {
      const float t = __shfl(wk[k], sp & 63, 64);
      if ((sp >> 6) == k) w = t;
    }
    return w;
  };
  float acc[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) acc[e] = 0.f;
  auto fma_row = [&](float w, const u32x4_t& x) {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      acc[2 * e] = __builtin_fmaf(w, __uint_as_float(x[e] << 16), acc[2 * e]);
      acc[2 * e + 1] = __builtin_fmaf(w, __uint_as_float(x[e] & 0xffff0000u), acc[2 * e + 1]);
    }
  };
#pragma unroll
  for (int k = 0; k < PRE; ++k) {  // split sg + k SGW: its weight sits in register (k SGW) / 64 of lane (sp % 64)
    const int sp = sg + k * SGW;
    const float w = __shfl(wk[(k * SGW) >> 6], sp & 63, 64);
    if (sp < nv) fma_row(w, u[k]);
  }
  for (int sp0 = PRE * SGW; sp0 < nv; sp0 += SGW) {  // more than PRE * SGW splits: the rest, in the same order
    const int sp = sp0 + sg;
    const float w = weight(sp < MAX_SPLIT ? sp : 0);
    if (sp < nv) fma_row(w, *reinterpret_cast<const u32x4_t*>(obase + sp * ostride));
  }
#pragma unroll
  for (int o = CPL; o < 64; o <<= 1)
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[e] += lane_xor(acc[e], o);
  if (sg != 0) return;
  const float inv = den > 0.f ? 1.f / den : 0.f;
  uint16_t* orow = p.out + ((static_cast<int64_t>(b) * p.W + n / p.G) * p.Hq + kvh * p.G + n % p.G) * D + dc * 8;
  *reinterpret_cast<u32x4_t*>(orow) = u32x4_t{cvt_pk_bf16(acc[0] * inv, acc[1] * inv), cvt_pk_bf16(acc[2] * inv, acc[3] * inv),
                                             cvt_pk_bf16(acc[4] * inv, acc[5] * inv), cvt_pk_bf16(acc[6] * inv, acc[7] * inv)};
}

// Default plan (gss_attn_make_plan with zeros): about DEF_TARGET_WGS / (bs * Hkv) key splits per sequence and kv
// head, each at least DEF_MIN_TILES tiles; batches with bs * Hkv >= DEF_WIDE_MIN run the wide kernel. At bs = 1 the
// minimum decides (short splits fill the chip); a large batch gets few long splits, which keeps the partial traffic
// and the merge small (32 ragged sequences of up to 12K keys with a 17-row window: 14 splits of 14 tiles, 87 us per
// call, against 90 us for 12 of 17, 122 us for 8 of 25 and 107-113 us for 15 or 16 splits of 13).
constexpr int DEF_TARGET_WGS = 896, DEF_MIN_TILES = 4, DEF_WIDE_MIN = 16;

// The plan fixes the key partition (tiles by absolute position, tiles_per_split of them per split) and the kernel;
// both depend on the arguments here only, never on W or on the lengths of a call.
int make_plan(int bs, int Hkv, int max_kv_len, int target_wgs, int min_tiles, int wide_min, gss_attn_plan* plan) {
  if (!plan || bs <= 0 || Hkv <= 0 || max_kv_len < 0 || target_wgs < 0 || min_tiles < 0 || wide_min < 0)
    return GSS_ERR_ARG;
  if (min_tiles > MAX_TPS) return GSS_ERR_ARG;
  if (target_wgs == 0) target_wgs = DEF_TARGET_WGS;
  if (min_tiles == 0) min_tiles = DEF_MIN_TILES;
  if (wide_min == 0) wide_min = DEF_WIDE_MIN;
  const int tiles = (max_kv_len + TILE + TILE - 1) / TILE;  // the capacity plus a full window
  const int by_chip = max(1, (target_wgs + bs * Hkv - 1) / (bs * Hkv));
  int t = max(min_tiles, (tiles + by_chip - 1) / by_chip);
  int ns = (tiles + t - 1) / t;
  if (ns > MAX_SPLIT) {
    ns = MAX_SPLIT;
    t = (tiles + ns - 1) / ns;
  }
  if (t > MAX_TPS) return GSS_ERR_UNSUPPORTED;
  plan->kernel = bs * Hkv >= wide_min ? GSS_ATTN_WIDE : GSS_ATTN_ROWGROUP;
  plan->tiles_per_split = t;
  plan->n_split = (tiles + t - 1) / t;
  plan->max_kv_len = max_kv_len;
  return GSS_OK;
}

// A caller-filled plan is accepted when its splits cover the capacity plus a full window.
int check_plan(const gss_attn_plan* plan) {
  if (!plan) return GSS_ERR_ARG;
  if (plan->kernel != GSS_ATTN_ROWGROUP && plan->kernel != GSS_ATTN_WIDE) return GSS_ERR_ARG;
  if (plan->tiles_per_split < 1 || plan->tiles_per_split > MAX_TPS || plan->n_split < 1 ||
      plan->n_split > MAX_SPLIT || plan->max_kv_len < 0)
    return GSS_ERR_ARG;
  const int64_t tiles = (static_cast<int64_t>(plan->max_kv_len) + TILE + TILE - 1) / TILE;
  if (static_cast<int64_t>(plan->n_split) * plan->tiles_per_split < tiles) return GSS_ERR_ARG;
  return GSS_OK;
}

int validate(int bs, int W, int Hq, int Hkv, int D, int page) {
  if (bs <= 0 || W <= 0 || Hq <= 0 || Hkv <= 0) return GSS_ERR_ARG;
  if (Hq % Hkv != 0) return GSS_ERR_UNSUPPORTED;
  if (D != 64 && D != 128) return GSS_ERR_UNSUPPORTED;
  if (page != PAGE || W > TILE) return GSS_ERR_UNSUPPORTED;
  return GSS_OK;
}

template <int D>
int set_lds_limits() {
  static bool done = false;  // allow the dynamic LDS beyond the default 64 KB (set once, before use)
  if (!done) {
    const void* wide[] = {reinterpret_cast<const void*>(&attn_split_kernel<D, 2, 1>),
                          reinterpret_cast<const void*>(&attn_split_kernel<D, 2, 2>),
                          reinterpret_cast<const void*>(&attn_split_kernel<D, 2, 3>),
                          reinterpret_cast<const void*>(&attn_split_kernel<D, 2, 4>),
                          reinterpret_cast<const void*>(&attn_split_kernel<D, 3, 4>)};
    for (const void* f : wide)
      if (hipFuncSetAttribute(f, hipFuncAttributeMaxDynamicSharedMemorySize, Lds<D>::TOTAL) != hipSuccess)
        return GSS_ERR_LAUNCH;
    const void* rg[] = {reinterpret_cast<const void*>(&attn_rowgroup_kernel<D, 1>),
                        reinterpret_cast<const void*>(&attn_rowgroup_kernel<D, 2>),
                        reinterpret_cast<const void*>(&attn_rowgroup_kernel<D, 3>)};
    for (const void* f : rg)
      if (hipFuncSetAttribute(f, hipFuncAttributeMaxDynamicSharedMemorySize, LdsRG<D>::TOTAL) != hipSuccess)
        return GSS_ERR_LAUNCH;
    done = true;
  }
  return GSS_OK;
}

// ng: N-tiles per row wave (wide kernel) or per workgroup (row-group kernel)
template <int D>
int launch_d(const AttnParams& p, int bs, bool wide, int ng, hipStream_t st) {
  if (set_lds_limits<D>() != GSS_OK) return GSS_ERR_LAUNCH;
  const dim3 grid((p.n_units + 7) / 8 * 8 * p.RG);
  if (wide) {
    const dim3 block(64 * p.RW);
    constexpr size_t lds = Lds<D>::TOTAL;
    // row waves x N-tiles per row wave: 1..4 x <= 2 (one N-tile per wave runs on the two-tile instantiation, only
    // its first tile computed), or 4 x 3
    if (ng > 2)
      hipLaunchKernelGGL((attn_split_kernel<D, 3, 4>), grid, block, lds, st, p);
    else if (p.RW == 4)
      hipLaunchKernelGGL((attn_split_kernel<D, 2, 4>), grid, block, lds, st, p);
    else if (p.RW == 3)
      hipLaunchKernelGGL((attn_split_kernel<D, 2, 3>), grid, block, lds, st, p);
    else if (p.RW == 2)
      hipLaunchKernelGGL((attn_split_kernel<D, 2, 2>), grid, block, lds, st, p);
    else
      hipLaunchKernelGGL((attn_split_kernel<D, 2, 1>), grid, block, lds, st, p);
  } else {
    constexpr size_t lds = LdsRG<D>::TOTAL;
    if (ng == 1)
      hipLaunchKernelGGL((attn_rowgroup_kernel<D, 1>), grid, dim3(RG_THREADS), lds, st, p);
    else if (ng == 2)
      hipLaunchKernelGGL((attn_rowgroup_kernel<D, 2>), grid, dim3(RG_THREADS), lds, st, p);
    else
      hipLaunchKernelGGL((attn_rowgroup_kernel<D, 3>), grid, dim3(RG_THREADS), lds, st, p);
  }
  if (p.n_split > 1)
    hipLaunchKernelGGL((window_attn_merge<D>), dim3(bs * p.Hkv * p.R), dim3(64), 0, st, p);
  return gss_launch_status();
}

size_t ws_bytes(int bs, int Hkv, int R, int D, int n_split) {
  return n_split > 1 ? static_cast<size_t>(bs) * Hkv * n_split * R * (D * sizeof(uint16_t) + 2 * sizeof(float)) : 0;
}

int attn_entry(const void* q, const void* k_pages, const void* v_pages, const int32_t* page_table, int pt_stride,
               const int32_t* prefix_len, int prefix_extra, const void* k_win, const void* v_win, void* out, int bs,
               int W, int n_causal, int Hq, int Hkv, int D, int page, float scale, const gss_attn_plan* plan,
               void* workspace, size_t workspace_bytes, hipStream_t st) {
  int rc = validate(bs, W, Hq, Hkv, D, page);
  if (rc != GSS_OK) return rc;
  if ((rc = check_plan(plan)) != GSS_OK) return rc;
  if (!q || !k_pages || !v_pages || !page_table || !prefix_len || !k_win || !v_win || !out) return GSS_ERR_ARG;
  if (n_causal < 0 || pt_stride <= 0) return GSS_ERR_ARG;
  AttnParams p;
  p.q = static_cast<const uint16_t*>(q);
  p.k_pages = static_cast<const uint16_t*>(k_pages);
  p.v_pages = static_cast<const uint16_t*>(v_pages);
  p.page_table = page_table;
  p.prefix_len = prefix_len;
  p.k_win = static_cast<const uint16_t*>(k_win);
  p.v_win = static_cast<const uint16_t*>(v_win);
  p.out = static_cast<uint16_t*>(out);
  p.pt_stride = pt_stride;
  p.prefix_extra = prefix_extra;
  p.W = W;
  p.n_causal = n_causal;
  p.Hq = Hq;
  p.Hkv = Hkv;
  p.G = Hq / Hkv;
  p.R = p.G * W;
  p.n_split = plan->n_split;
  p.tps = plan->tiles_per_split;
  p.cap = static_cast<int>(min(static_cast<int64_t>(plan->max_kv_len), static_cast<int64_t>(pt_stride) * PAGE));
  p.bs = bs;
  p.n_units = bs * Hkv * p.n_split;
  // kernel: the plan's (never a function of W), so every window size of one batch runs the same one
  const bool wide = plan->kernel == GSS_ATTN_WIDE;
  const int NT = (p.R + 15) / 16;
  int ng;
  if (wide) {
    // rows: NT N-tiles of 16 in RG row groups of TPG tiles (as even as the group count allows; tiles past NT are
    // padding), dealt to RW row waves (the first TPG % RW take one more): 1 -> one wave of 1, 9 (17-row window) ->
    // 3,2,2,2, 17 (33-row window) -> two groups of 9 (3,2,2,2; the last tile padding) rather than 12 and 5, whose
    // padding would triple the second group's work
    p.RG = (NT + RW_MAX * NGW_MAX - 1) / (RW_MAX * NGW_MAX);
    p.TPG = (NT + p.RG - 1) / p.RG;
    p.RW = min(RW_MAX, p.TPG);
    ng = (p.TPG + p.RW - 1) / p.RW;
  } else {
    // row groups of ng <= RG_NTG N-tiles, one workgroup each
    ng = min(RG_NTG, NT);
    p.RW = p.TPG = 0;
    p.RG = (NT + ng - 1) / ng;
  }
  p.scale_log2 = scale * LOG2E;
  p.ws_o = nullptr;
  p.ws_ml = nullptr;
  if (p.n_split > 1) {
    const size_t need = ws_bytes(bs, Hkv, p.R, D, p.n_split);
    if (!workspace || workspace_bytes < need) return GSS_ERR_WORKSPACE;
    p.ws_o = static_cast<uint16_t*>(workspace);
    p.ws_ml = reinterpret_cast<float*>(static_cast<char*>(workspace) +
                                       static_cast<size_t>(bs) * Hkv * p.n_split * p.R * D * sizeof(uint16_t));
  }
  return D == 128 ? launch_d<128>(p, bs, wide, ng, st) : launch_d<64>(p, bs, wide, ng, st);
}

}  // namespace

extern "C" int gss_attn_make_plan(int bs, int Hkv, int max_kv_len, int target_wgs, int min_tiles, int wide_min,
                                  gss_attn_plan* plan) {
  return make_plan(bs, Hkv, max_kv_len, target_wgs, min_tiles, wide_min, plan);
}

extern "C" int gss_attn_workspace_size(int bs, int Hq, int Hkv, int D, int W, const gss_attn_plan* plan,
                                       size_t* bytes) {
  if (!bytes) return GSS_ERR_ARG;
  int rc = validate(bs, W, Hq, Hkv, D, PAGE);
  if (rc != GSS_OK) return rc;
  if ((rc = check_plan(plan)) != GSS_OK) return rc;
  *bytes = ws_bytes(bs, Hkv, (Hq / Hkv) * W, D, plan->n_split);
  return GSS_OK;
}

extern "C" int gss_draft_attn(const void* q, const void* k_pages, const void* v_pages, const int32_t* page_table,
                              int pt_stride, const int32_t* prefix_len, int prefix_extra, const void* k_win,
                              const void* v_win, void* out, int bs, int W, int n_causal, int Hq, int Hkv, int D,
                              int page, float scale, const gss_attn_plan* plan, void* workspace,
                              size_t workspace_bytes, gss_stream_t stream) {
  return attn_entry(q, k_pages, v_pages, page_table, pt_stride, prefix_len, prefix_extra, k_win, v_win, out, bs, W,
                    n_causal, Hq, Hkv, D, page, scale, plan, workspace, workspace_bytes,
                    static_cast<hipStream_t>(stream));
}

extern "C" int gss_verify_attn(const void* q, const void* k_pages, const void* v_pages, const int32_t* page_table,
                               int pt_stride, const int32_t* prefix_len, int prefix_extra, const void* k_win,
                               const void* v_win, void* out, int bs, int W, int Hq, int Hkv, int D, int page,
                               float scale, const gss_attn_plan* plan, void* workspace, size_t workspace_bytes,
                               gss_stream_t stream) {
  return attn_entry(q, k_pages, v_pages, page_table, pt_stride, prefix_len, prefix_extra, k_win, v_win, out, bs, W,
                    W, Hq, Hkv, D, page, scale, plan, workspace, workspace_bytes, static_cast<hipStream_t>(stream));
}
