// (a) draft and (b) verify attention of the self-spec round: W window query rows of each sequence attend to the
// committed prefix (paged K/V, 16-token pages) plus the window's own K/V (staging), with the draft
// (n_causal leading causal rows, the rest bidirectional) or verify (causal) window mask.
//
// gfx950 design
//   * GQA packing: the G = Hq/Hkv query heads of one KV head and the W window rows form R = G*W query rows that
//     share every K/V byte read (row n = w*G + g); rows are MFMA N-tiles of 16. A workgroup owns a row group of up
//     to NTG = 3 N-tiles, so the MFMA work of one key tile is spread over ceil(R/48) workgroups. Those row groups
//     of a split are launched on the same XCD (grid x = row_group * S8 + split with S8 a multiple of 8, and
//     workgroups are dealt to the 8 XCDs round-robin), so their repeated K/V reads hit that XCD's L2.
//   * Transposed contractions on v_mfma_f32_16x16x32_bf16:  S^T = K Q^T  (M = tokens, N = rows, K = head dim) and
//     O^T = V^T P^T  (M = head dim, N = rows, K = tokens). A lane then owns one query row per N-tile, so the online
//     softmax max is two xor-shuffles and the row sum stays lane-local until the end. The P^T operand is the lane's
//     own S^T values; the token order inside the K=32 step is permuted identically on the V^T side, so no data
//     moves between lanes.
//   * K tiles live in LDS as [token][D] with an XOR swizzle of the 16-byte chunks (conflict-free 16-row reads);
//     V pages are stored token-minor ([D][16] per page) in HBM, so the V^T operand is two 8-byte LDS reads.
//   * A split's tiles are processed in stages of LANES = 4 tiles: the page ids of the whole split are read once
//     into LDS, then every K/V load of a stage is issued at once, straight from global memory into LDS
//     (global_load_lds_dwordx4; no staging registers). Tile j of a split belongs to tile lane j % 4; the compute waves
//     of a row group are (N-tile, lane) pairs, each keeps its own online softmax, and the 4 lanes are combined in
//     lane order at the end.
//   * Keys are tiled by absolute position (window rows take the positions after the prefix); the split size and
//     the tile -> split -> lane assignment depend only on the capacity max_kv_len and on fixed constants, never on
//     W, the prefix length or the row grouping, and every combine runs in a fixed order. Results therefore do not
//     depend on where a key comes from or on how many rows are in the window: a verify row reproduces the AR step
//     of the same token bit for bit. With several splits, the normalized partial O (bf16) and (m, l) (fp32) of each
//     split go to the caller's workspace and the merge kernel combines the valid splits of every row.
#include "gss_common.h"

namespace {

constexpr int PAGE = 16;
constexpr int TILE = 64;        // KV tokens per tile (4 pages)
constexpr int LANES = 4;        // tiles per stage; tile j of a split goes to lane j % LANES
constexpr int NTG = 3;          // query N-tiles (16 rows) per workgroup
constexpr int NTHREADS = 64 * 2 * LANES;  // a wave per (tile lane, key half): 8 waves, 2 per SIMD
constexpr int MAX_TPS = 256;    // tiles per split (page ids of a split in LDS: 4 * MAX_TPS ints)
constexpr int MAX_SPLIT = 256;
constexpr float LOG2E = 1.4426950408889634f;

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
  int pt_stride, prefix_extra, W, n_causal, Hq, Hkv, G, R, n_split, S8, tps;
  float scale_log2;
};

template <int D>
struct Lds {
  static constexpr int TILE_EL = TILE * D;          // elements of one K (or V) tile
  static constexpr int V_OFF = LANES * TILE_EL;     // K stage [LANES][TILE][D] swizzled, then V [LANES][4][D][16]
  static constexpr int BYTES = 2 * LANES * TILE_EL * 2;         // the K/V stage
  static constexpr int MAX_BYTES = NTHREADS / 64 * NTG * 16 * 4;  // row-max exchange [waves][NG][16] after it
  static constexpr int TOTAL = BYTES + MAX_BYTES;
  // combine scratch (reuses the K/V stage): per (wave, N-tile) O as bf16 [DT][64 lanes] x 4 + l [16 rows]
  static constexpr int SCR_BYTES = (D / 16) * 64 * 8 + 16 * 4;
  static_assert(NTHREADS / 64 * NTG * SCR_BYTES <= BYTES, "combine scratch exceeds the K/V stage");
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

GSS_DEV int valid_splits(int L, int W, int tps) {
  const int n_tiles = (L + W + TILE - 1) / TILE;
  return (n_tiles + tps - 1) / tps;
}

template <int D, int NG>
__global__ void __launch_bounds__(NTHREADS, 1) window_attn_kernel(AttnParams p) {
  constexpr int KS = D / 32;   // MFMA K-steps over the head dim
  constexpr int DT = D / 16;   // 16-row tiles of the head dim (O^T M-tiles)
  constexpr int CH = D / 8;    // 16-byte chunks per K row
  constexpr int TILE_EL = Lds<D>::TILE_EL;
  constexpr int TILE_INSTR = TILE * CH / 64;    // direct-load instructions per K (or V) tile
  constexpr int STAGE_INSTR = LANES * TILE_INSTR;
  constexpr int PAGE_INSTR = PAGE * CH / 64;    // instructions per (page, head) block of K (or V)
  constexpr int NW = NTHREADS / 64;
  extern __shared__ __attribute__((aligned(16))) uint16_t smem[];
  uint16_t* lds_k = smem;
  uint16_t* lds_v = smem + Lds<D>::V_OFF;

  const int s = blockIdx.x % p.S8, rg = blockIdx.x / p.S8;  // split, row group
  if (s >= p.n_split) return;                                 // XCD-alignment padding
  const int kvh = blockIdx.y, b = blockIdx.z;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int kq = wv >> 1, half = wv & 1;                      // tile lane, key half (32 keys) of this wave
  const int l16 = lane & 15, g4 = lane >> 4;
  // committed prefix length; clamped to what the page-table row can address so every page-table read is in bounds
  const int L = min(max(p.prefix_len[b] + p.prefix_extra, 0), p.pt_stride * PAGE);
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
    const int pos = (t_beg + st * LANES) * TILE + lane * PAGE;
    return (lane < LANES * (TILE / PAGE) && pos < L) ? pt[pos / PAGE] : 0;
  };
  auto issue_stage = [&](int st, int pgv) {
#pragma unroll 4
    for (int i = 0; i < 2 * STAGE_INSTR / NW; ++i) {
      const int ii = i * NW + wv;
      const bool is_v = ii >= STAGE_INSTR;
      const int iv = is_v ? ii - STAGE_INSTR : ii;
      const int t = t_beg + st * LANES + iv / TILE_INSTR;
      if (t >= t_end) continue;
      const int pblk = iv / PAGE_INSTR;                         // page of the stage (tile * 4 + page in tile)
      const int pos0 = t * TILE + (pblk % (TILE / PAGE)) * PAGE;  // first position of that page
      const int64_t page = __builtin_amdgcn_readlane(pgv, pblk);
      const uint16_t* base = (is_v ? p.v_pages : p.k_pages) + (page * p.Hkv + kvh) * head_stride;
      const bool in_prefix = pos0 + PAGE <= L || (is_v ? pos0 + vh * 8 < L : pos0 + ktok < L);
      if (in_prefix)
        __builtin_amdgcn_global_load_lds((gvoid_t*)(base + (is_v ? voff : koff)),
                                         (lvoid_t*)(smem + (is_v ? Lds<D>::V_OFF : 0) + iv * 512), 16, 0, 0);
    }
  };
  // Tiles that reach past the prefix: K rows and V columns of positions >= L get the window rows (staging) or zero,
  // and the V chunk that straddles L keeps only its prefix tokens.
  auto fix_stage = [&](int st) {
    const int ts = t_beg + st * LANES, te = min(t_end, ts + LANES);
    const int t0 = max(ts, L / TILE);
    if (t0 >= te) return false;
    for (int c = tid; c < (te - t0) * TILE * CH; c += NTHREADS) {  // K chunks of the boundary tiles
      const int t = t0 + c / (TILE * CH), r = c % (TILE * CH), tok = r / CH, part = r % CH;
      const int pos = t * TILE + tok;
      if (pos < L) continue;
      u32x4_t v = {0u, 0u, 0u, 0u};
      if (pos < L + W)
        v = *reinterpret_cast<const u32x4_t*>(p.k_win + (win_base + static_cast<int64_t>(pos - L) * p.Hkv) * D +
                                              part * 8);
      *reinterpret_cast<u32x4_t*>(&lds_k[(t - ts) * TILE_EL + k_lds_index<D>(tok, part)]) = v;
    }
    for (int c = tid; c < (te - t0) * TILE * CH; c += NTHREADS) {  // V chunks of the boundary tiles
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
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const int pos = first + e;
        if (pos >= L && pos < L + W) {
          const uint32_t x = p.v_win[(win_base + static_cast<int64_t>(pos - L) * p.Hkv) * D + d];
          v[e >> 1] |= (e & 1) ? (x << 16) : x;
        }
      }
      *reinterpret_cast<u32x4_t*>(dst) = v;
    }
    return true;
  };

  // ---- softmax with one running max per row shared by the whole workgroup -----------------------------------
  // Each stage: every wave scores its 32 keys (tile lane kq, key half `half`; m-tiles 2*half, 2*half+1) for the NG
  // N-tiles, the waves exchange their row maxima through LDS, and all of them rescale (from the second stage on)
  // and accumulate against the same running max. The 8 partial (O, l) of the workgroup are then on one scale and
  // combine by plain sums in a fixed order. Every K and V fragment read from LDS feeds the MFMAs of all NG N-tiles.
  float* smax = reinterpret_cast<float*>(reinterpret_cast<char*>(smem) + Lds<D>::BYTES);  // [NW][NG][16]
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

  const int n_stages = (t_end - t_beg + LANES - 1) / LANES;
  int pgv = stage_pages(0);
  for (int st = 0; st < n_stages; ++st) {
    if (st > 0) __syncthreads();  // the previous stage's compute is done with LDS
    issue_stage(st, pgv);
    if (st + 1 < n_stages) pgv = stage_pages(st + 1);
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    if (fix_stage(st)) __syncthreads();  // block-uniform condition
    const int tb = (t_beg + st * LANES + kq) * TILE;
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
      mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
      mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
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
        const float alpha = exp2f(m_run[g] - m_use);
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
          const float p0 = exp2f(__builtin_fmaf(sacc[g][j >> 1][(2 * j) & 3], p.scale_log2, nm));
          const float p1 = exp2f(__builtin_fmaf(sacc[g][j >> 1][(2 * j + 1) & 3], p.scale_log2, nm));
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
    l_run[g] += __shfl_xor(l_run[g], 16, 64);
    l_run[g] += __shfl_xor(l_run[g], 32, 64);
  }
  __syncthreads();  // every wave is done with the K/V stage: reuse it as scratch
  char* scr = reinterpret_cast<char*>(smem);
#pragma unroll
  for (int g = 0; g < NG; ++g) {
    char* slot = scr + (wv * NG + g) * Lds<D>::SCR_BYTES;
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
      const char* slot = scr + (w * NG + g) * Lds<D>::SCR_BYTES;
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

// Combine the valid splits of each (sequence, kv head, row): block = one query row, 256 threads = (D/2 dim pairs) x
// (SG split groups). All loads are issued in one round: the prefix length, the row's (m, l) of every split (stored
// contiguously per row; splits past the valid count are masked), and each thread's partial-O pairs. Weights
// w_s = l_s * 2^(m_s - M) follow from one wave-wide max; thread (dp, sg) sums w_s * O_s over s = sg mod SG with
// fused multiply-adds in split order, and the SG groups and the weights are reduced in a fixed order. A split that
// holds none of the row's visible keys has w_s = 0 exactly.
template <int D>
__global__ void __launch_bounds__(256) window_attn_merge(AttnParams p) {
  constexpr int DP = D / 2, SG = 256 / DP, PRE = 16;  // PRE: partial-O loads per thread issued up front
  const int n = blockIdx.x, kvh = blockIdx.y, b = blockIdx.z;
  const int tid = threadIdx.x, dp = tid % DP, sg = tid / DP;
  const int ns = p.n_split;
  const int64_t rowid = (static_cast<int64_t>(b) * p.Hkv + kvh) * p.R + n;
  const float2* ml = reinterpret_cast<const float2*>(p.ws_ml) + rowid * ns;
  const uint16_t* obase = p.ws_o + (static_cast<int64_t>(b) * p.Hkv + kvh) * ns * p.R * D +
                          static_cast<int64_t>(n) * D + 2 * dp;
  const int64_t ostride = static_cast<int64_t>(p.R) * D;
  __shared__ float sw[MAX_SPLIT];
  __shared__ float red[4];
  __shared__ float2 sacc[SG][DP];
  // every independent load in one round: prefix length, (m, l) of split tid, this thread's first PRE O pairs
  const int L = min(max(p.prefix_len[b] + p.prefix_extra, 0), p.pt_stride * PAGE);
  const float2 mlv = tid < ns ? ml[tid] : float2{-INFINITY, 0.f};
  uint32_t u[PRE];
#pragma unroll
  for (int k = 0; k < PRE; ++k) {
    const int s = sg + k * SG;
    u[k] = s < ns ? *reinterpret_cast<const uint32_t*>(obase + s * ostride) : 0u;
  }
  const int nv = min(ns, valid_splits(L, p.W, p.tps));
  float mloc = wave_max(tid < nv ? mlv.x : -INFINITY);
  if ((tid & 63) == 0) red[tid >> 6] = mloc;
  __syncthreads();
  const float M = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  const float Mu = M == -INFINITY ? 0.f : M;
  sw[tid] = tid < nv ? mlv.y * exp2f(mlv.x - Mu) : 0.f;
  __syncthreads();
  float ax = 0.f, ay = 0.f;
#pragma unroll
  for (int k = 0; k < PRE; ++k) {  // splits sg, sg + SG, ... in order, with fused multiply-adds
    const int s = sg + k * SG;
    // splits past the valid count hold whatever an earlier call left in the workspace: drop the value, not just
    // its weight (0 * inf would be NaN)
    const float w = s < nv ? sw[s] : 0.f;
    const uint32_t v = s < nv ? u[k] : 0u;
    ax = __builtin_fmaf(w, __uint_as_float(v << 16), ax);
    ay = __builtin_fmaf(w, __uint_as_float(v & 0xffff0000u), ay);
  }
  for (int s = sg + PRE * SG; s < nv; s += SG) {  // more than PRE * SG splits: the rest, in the same order
    const uint32_t v = *reinterpret_cast<const uint32_t*>(obase + s * ostride);
    const float w = sw[s];
    ax = __builtin_fmaf(w, __uint_as_float(v << 16), ax);
    ay = __builtin_fmaf(w, __uint_as_float(v & 0xffff0000u), ay);
  }
  sacc[sg][dp] = float2{ax, ay};
  __syncthreads();
  if (sg != 0) return;
  float den = 0.f;
  for (int k = 0; k < nv; ++k) den += sw[k];
  for (int g = 1; g < SG; ++g) {
    ax += sacc[g][dp].x;
    ay += sacc[g][dp].y;
  }
  const float inv = den > 0.f ? 1.f / den : 0.f;
  const int w = n / p.G, gq = n % p.G;
  uint16_t* orow = p.out + ((static_cast<int64_t>(b) * p.W + w) * p.Hq + kvh * p.G + gq) * D;
  *reinterpret_cast<uint32_t*>(orow + 2 * dp) = cvt_pk_bf16(ax * inv, ay * inv);
}

// Split sizing: tiles per split from the capacity (max_kv_len plus a full window) and bs * Hkv only, so every call
// on the same cache and batch size partitions the keys identically: about target_wgs / (bs * Hkv) splits per
// sequence and kv head, each at least min_tiles tiles (gss_attn_set_split_policy). At bs = 1 the minimum decides
// (short splits fill the chip); a large batch gets few long splits, which keeps the partial traffic and the merge
// small (32 ragged sequences of up to 12K keys: 8 splits of 25 tiles, 1.8x faster than 4 splits of 49).
int g_target_wgs = 512, g_min_tiles = 4;

int attn_plan(int bs, int Hkv, int max_kv_len, int* n_split, int* tps) {
  const int tiles = (max(max_kv_len, 0) + TILE + TILE - 1) / TILE;
  const int by_chip = max(1, (g_target_wgs + bs * Hkv - 1) / (bs * Hkv));
  int t = max(g_min_tiles, (tiles + by_chip - 1) / by_chip);
  int ns = (tiles + t - 1) / t;
  if (ns > MAX_SPLIT) {
    ns = MAX_SPLIT;
    t = (tiles + ns - 1) / ns;
  }
  if (t > MAX_TPS) return GSS_ERR_UNSUPPORTED;
  *n_split = (tiles + t - 1) / t;
  *tps = t;
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
int launch_d(const AttnParams& p, int bs, int NT, hipStream_t st) {
  static bool lds_attr_set = false;  // allow the dynamic LDS beyond the default 64 KB (set once, before use)
  if (!lds_attr_set) {
    const void* fns[] = {reinterpret_cast<const void*>(&window_attn_kernel<D, 1>),
                         reinterpret_cast<const void*>(&window_attn_kernel<D, 2>),
                         reinterpret_cast<const void*>(&window_attn_kernel<D, 3>)};
    for (const void* f : fns)
      if (hipFuncSetAttribute(f, hipFuncAttributeMaxDynamicSharedMemorySize, Lds<D>::TOTAL) != hipSuccess)
        return GSS_ERR_LAUNCH;
    lds_attr_set = true;
  }
  const int NG = min(NTG, NT), RG = (NT + NG - 1) / NG;
  const dim3 grid(p.S8 * RG, p.Hkv, bs);
  if (NG == 1)
    hipLaunchKernelGGL((window_attn_kernel<D, 1>), grid, dim3(NTHREADS), Lds<D>::TOTAL, st, p);
  else if (NG == 2)
    hipLaunchKernelGGL((window_attn_kernel<D, 2>), grid, dim3(NTHREADS), Lds<D>::TOTAL, st, p);
  else
    hipLaunchKernelGGL((window_attn_kernel<D, 3>), grid, dim3(NTHREADS), Lds<D>::TOTAL, st, p);
  if (p.n_split > 1) hipLaunchKernelGGL((window_attn_merge<D>), dim3(p.R, p.Hkv, bs), dim3(256), 0, st, p);
  return gss_launch_status();
}

size_t ws_bytes(int bs, int Hkv, int R, int D, int n_split) {
  return n_split > 1 ? static_cast<size_t>(bs) * Hkv * n_split * R * (D * sizeof(uint16_t) + 2 * sizeof(float)) : 0;
}

int attn_entry(const void* q, const void* k_pages, const void* v_pages, const int32_t* page_table, int pt_stride,
               const int32_t* prefix_len, int prefix_extra, const void* k_win, const void* v_win, void* out, int bs,
               int W, int n_causal, int Hq, int Hkv, int D, int page, float scale, int max_kv_len, void* workspace,
               size_t workspace_bytes, hipStream_t st) {
  int rc = validate(bs, W, Hq, Hkv, D, page);
  if (rc != GSS_OK) return rc;
  if (!q || !k_pages || !v_pages || !page_table || !prefix_len || !k_win || !v_win || !out) return GSS_ERR_ARG;
  if (n_causal < 0 || max_kv_len < 0 || pt_stride <= 0) return GSS_ERR_ARG;
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
  rc = attn_plan(bs, Hkv, max_kv_len, &p.n_split, &p.tps);
  if (rc != GSS_OK) return rc;
  p.S8 = (p.n_split + 7) / 8 * 8;
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
  const int NT = (p.R + 15) / 16;
  return D == 128 ? launch_d<128>(p, bs, NT, st) : launch_d<64>(p, bs, NT, st);
}

}  // namespace

extern "C" int gss_attn_workspace_size(int bs, int Hq, int Hkv, int D, int W, int max_kv_len, size_t* bytes) {
  if (!bytes) return GSS_ERR_ARG;
  int rc = validate(bs, W, Hq, Hkv, D, PAGE);
  if (rc != GSS_OK) return rc;
  if (max_kv_len < 0) return GSS_ERR_ARG;
  int ns, tps;
  rc = attn_plan(bs, Hkv, max_kv_len, &ns, &tps);
  if (rc != GSS_OK) return rc;
  *bytes = ws_bytes(bs, Hkv, (Hq / Hkv) * W, D, ns);
  return GSS_OK;
}

extern "C" int gss_draft_attn(const void* q, const void* k_pages, const void* v_pages, const int32_t* page_table,
                              int pt_stride, const int32_t* prefix_len, int prefix_extra, const void* k_win,
                              const void* v_win, void* out, int bs, int W, int n_causal, int Hq, int Hkv, int D,
                              int page, float scale, int max_kv_len, void* workspace, size_t workspace_bytes,
                              gss_stream_t stream) {
  return attn_entry(q, k_pages, v_pages, page_table, pt_stride, prefix_len, prefix_extra, k_win, v_win, out, bs, W,
                    n_causal, Hq, Hkv, D, page, scale, max_kv_len, workspace, workspace_bytes,
                    static_cast<hipStream_t>(stream));
}

extern "C" int gss_verify_attn(const void* q, const void* k_pages, const void* v_pages, const int32_t* page_table,
                               int pt_stride, const int32_t* prefix_len, int prefix_extra, const void* k_win,
                               const void* v_win, void* out, int bs, int W, int Hq, int Hkv, int D, int page,
                               float scale, int max_kv_len, void* workspace, size_t workspace_bytes,
                               gss_stream_t stream) {
  return attn_entry(q, k_pages, v_pages, page_table, pt_stride, prefix_len, prefix_extra, k_win, v_win, out, bs, W,
                    W, Hq, Hkv, D, page, scale, max_kv_len, workspace, workspace_bytes,
                    static_cast<hipStream_t>(stream));
}

extern "C" int gss_attn_set_split_policy(int target_wgs, int min_tiles) {
  if (target_wgs < 1 || min_tiles < 1 || min_tiles > MAX_TPS) return GSS_ERR_ARG;
  g_target_wgs = target_wgs;
  g_min_tiles = min_tiles;
  return GSS_OK;
}
