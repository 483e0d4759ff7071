// (a) draft and (b) verify attention of the self-spec round: W window query rows of each sequence attend to the
// committed prefix (paged K/V, 16-token pages) plus the window's own K/V (staging), with the draft
// (n_causal leading causal rows, the rest bidirectional) or verify (causal) window mask.
//
// gfx950 design
//   * GQA packing: the G = Hq/Hkv query heads of one KV head and the W window rows form R = G*W query rows that
//     share every K/V byte read; rows are MFMA N-tiles of 16 (row n = w*G + g).
//   * Transposed contractions on v_mfma_f32_16x16x32_bf16:  S^T = K Q^T  (M = tokens, N = rows, K = head dim) and
//     O^T = V^T P^T  (M = head dim, N = rows, K = tokens). A lane then owns one query row per N-tile, so the online
//     softmax max is two xor-shuffles and the row sum stays lane-local until the end. The P^T operand is the lane's
//     own S^T values; the token order inside the K=32 step is permuted identically on the V^T side, so no data
//     moves between lanes.
//   * K tiles live in LDS as [token][D] with an XOR swizzle of the 16-byte chunks (conflict-free 16-row reads);
//     V pages are stored token-minor ([D][16] per page) in HBM, so the V^T operand is two 8-byte LDS reads.
//   * Keys are tiled by absolute position (window rows take the positions after the prefix), and split-KV
//     partitions the tiles by capacity (grid = splits x Hkv x bs), so results do not depend on where a key comes
//     from or on the prefix length: verify rows reproduce AR steps bit for bit. Partial (m, l, O) go to the
//     caller's workspace and a merge kernel combines them in a fixed order.
#include "gss_common.h"

namespace {

constexpr int PAGE = 16;
constexpr int TILE = 64;  // KV tokens per LDS tile (4 pages)
constexpr int MAX_WAVES = 12;  // 768 threads: 3 waves per SIMD, 168 VGPRs per lane
constexpr int MIN_WAVES = 4;   // extra waves only load tiles
constexpr int MAX_NT = 24;  // query-row tiles per kv head (LDS: 32 KB K/V + MAX_NT * 16 * D * 2 B of Q)
constexpr float LOG2E = 1.4426950408889634f;

struct AttnParams {
  const uint16_t* q;
  const uint16_t* k_pages;
  const uint16_t* v_pages;
  const int32_t* page_table;
  const int32_t* prefix_len;
  const uint16_t* k_win;
  const uint16_t* v_win;
  uint16_t* out;
  float* ws_o;   // [bs, Hkv, n_split, R, D]
  float* ws_ml;  // [bs, Hkv, n_split, R, 2]
  int pt_stride, prefix_extra, W, n_causal, Hq, Hkv, G, R, NT, n_split, tps;  // tps: 64-token tiles per split
  float scale_log2;
};

template <int D>
GSS_DEV int k_lds_index(int tok, int chunk) {
  // 16-byte chunk `chunk` of token row `tok`, XOR-swizzled over the D/8 chunks of a row
  return (tok * (D / 8) + (chunk ^ (tok & (D / 8 - 1)))) * 8;
}

template <int D, int TPW, int CPT>
__global__ void __launch_bounds__(64 * MAX_WAVES)
window_attn_kernel(AttnParams p) {
  constexpr int KS = D / 32;   // MFMA K-steps over the head dim
  constexpr int DT = D / 16;   // 16-row tiles of the head dim (O^T M-tiles)
  __shared__ __attribute__((aligned(16))) uint16_t lds_k[TILE * D];
  __shared__ __attribute__((aligned(16))) uint16_t lds_v[TILE * D];  // [4 pages][D][16]
  extern __shared__ __attribute__((aligned(16))) uint16_t lds_q[];    // [NT*16 rows][D], swizzled like lds_k

  const int s = blockIdx.x, kvh = blockIdx.y, b = blockIdx.z;
  const int tid = threadIdx.x, nthr = blockDim.x;
  const int lane = tid & 63, wv = tid >> 6;
  const int l16 = lane & 15, g4 = lane >> 4;
  // committed prefix length; clamped to what the page-table row can address so every page-table read is in bounds
  const int L = min(max(p.prefix_len[b] + p.prefix_extra, 0), p.pt_stride * PAGE);

  // ---- the R = G*W query rows of this kv head into LDS (row n = w*G + g; rows >= R are zero) ------------------
  for (int c = tid; c < p.NT * 16 * (D / 8); c += nthr) {
    const int n = c / (D / 8), part = c % (D / 8);
    u32x4_t v = {0u, 0u, 0u, 0u};
    if (n < p.R) {
      const int w = n / p.G, gq = n % p.G;
      v = *reinterpret_cast<const u32x4_t*>(p.q + ((static_cast<int64_t>(b) * p.W + w) * p.Hq + kvh * p.G + gq) * D +
                                            part * 8);
    }
    *reinterpret_cast<u32x4_t*>(&lds_q[k_lds_index<D>(n, part)]) = v;
  }

  // ---- this wave's accumulators: N-tiles wv*TPW .. wv*TPW+TPW-1 ------------------------------------------------
  floatx4_t o[TPW][DT];
  float m_run[TPW], l_run[TPW];
#pragma unroll
  for (int t = 0; t < TPW; ++t) {
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) o[t][dt] = floatx4_t{0.f, 0.f, 0.f, 0.f};
    m_run[t] = -INFINITY;
    l_run[t] = 0.f;
  }

  // Online-softmax update of one 64-token tile held in LDS. `visible(row_w, tok)` decides the mask.
  auto compute_tile = [&](auto visible) {
#pragma unroll
    for (int t = 0; t < TPW; ++t) {
      const int nt = wv * TPW + t;
      if (nt < p.NT) {  // wave-uniform
        floatx4_t sacc[4];
#pragma unroll
        for (int mt = 0; mt < 4; ++mt) sacc[mt] = floatx4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) {
          const bf16x8_t qb = *reinterpret_cast<const bf16x8_t*>(&lds_q[k_lds_index<D>(nt * 16 + l16, ks * 4 + g4)]);
#pragma unroll
          for (int mt = 0; mt < 4; ++mt) {
            const bf16x8_t a = *reinterpret_cast<const bf16x8_t*>(&lds_k[k_lds_index<D>(mt * 16 + l16, ks * 4 + g4)]);
            sacc[mt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, qb, sacc[mt], 0, 0, 0);
          }
        }
        const int n = nt * 16 + l16;
        const int roww = n < p.R ? n / p.G : 0;
        float mx = -INFINITY;
#pragma unroll
        for (int mt = 0; mt < 4; ++mt)
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const int tok = mt * 16 + g4 * 4 + i;
            const float x = visible(roww, tok) ? sacc[mt][i] * p.scale_log2 : -INFINITY;
            sacc[mt][i] = x;
            mx = fmaxf(mx, x);
          }
        mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
        mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
        const float m_new = fmaxf(m_run[t], mx);
        const float m_use = m_new == -INFINITY ? 0.f : m_new;
        const float alpha = exp2f(m_run[t] - m_use);
        m_run[t] = m_new;
        float ls = 0.f;
        uint32_t pk[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const float p0 = exp2f(sacc[j >> 1][(2 * j) & 3] - m_use);
          const float p1 = exp2f(sacc[j >> 1][(2 * j + 1) & 3] - m_use);
          ls += p0 + p1;
          pk[j] = pack_bf16x2(p0, p1);
        }
        l_run[t] = l_run[t] * alpha + ls;
        // P^T operand of K-step kk: slots 0..3 = m-tile 2kk values, slots 4..7 = m-tile 2kk+1 values
        const bf16x8_t pb0 = __builtin_bit_cast(bf16x8_t, u32x4_t{pk[0], pk[1], pk[2], pk[3]});
        const bf16x8_t pb1 = __builtin_bit_cast(bf16x8_t, u32x4_t{pk[4], pk[5], pk[6], pk[7]});
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) {
          floatx4_t acc = o[t][dt] * alpha;
          const int d = dt * 16 + l16;
          const u32x2_t v00 = *reinterpret_cast<const u32x2_t*>(&lds_v[((0 * D) + d) * PAGE + g4 * 4]);
          const u32x2_t v01 = *reinterpret_cast<const u32x2_t*>(&lds_v[((1 * D) + d) * PAGE + g4 * 4]);
          acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
              __builtin_bit_cast(bf16x8_t, u32x4_t{v00[0], v00[1], v01[0], v01[1]}), pb0, acc, 0, 0, 0);
          const u32x2_t v10 = *reinterpret_cast<const u32x2_t*>(&lds_v[((2 * D) + d) * PAGE + g4 * 4]);
          const u32x2_t v11 = *reinterpret_cast<const u32x2_t*>(&lds_v[((3 * D) + d) * PAGE + g4 * 4]);
          acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
              __builtin_bit_cast(bf16x8_t, u32x4_t{v10[0], v10[1], v11[0], v11[1]}), pb1, acc, 0, 0, 0);
          o[t][dt] = acc;
        }
      }
    }
  };

  // ---- the key sequence in absolute positions --------------------------------------------------------------
  // Keys are positions 0 .. L+W-1: positions < L come from the pages, positions L .. L+W-1 are the window rows
  // (staging). Tiles are the 64-position blocks [64t, 64t+64) and split s owns tiles [s*tps, (s+1)*tps) (tps depends
  // only on the capacity max_kv_len). A query's visible keys therefore sit in the same tiles, accumulated in the same
  // order, whether they are window rows or already in the pages: a verify row and the AR step of the same token
  // compute bit-identical attention.
  const int W = p.W, nc = p.n_causal;
  const int n_tiles = (L + W + TILE - 1) / TILE;
  const int t_beg = s * p.tps, t_end = min(n_tiles, t_beg + p.tps);
  const int32_t* pt = p.page_table + static_cast<int64_t>(b) * p.pt_stride;
  const int64_t head_stride = static_cast<int64_t>(PAGE) * D;  // elements per (page, kv head) block
  const int64_t win_base = static_cast<int64_t>(b) * W * p.Hkv + kvh;  // row j of the window: (win_base + j*Hkv)*D

  // Tile loads go through registers: tile i+1's global loads are issued before tile i is computed, so HBM latency
  // overlaps the MFMA work. Each thread owns chunks c = tid + k*nthr (k < CPT) of the K tile ([64 tok][D], 16 B
  // each) and of the V tile ([4 pages][D][16 tok], 8 tokens of one dim each).
  constexpr int NCH = TILE * D / 8;  // 16-byte chunks per K tile (and per V tile)
  u32x4_t pk[CPT], pv[CPT];
  auto load_tile = [&](int tb) {
    int pg[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) pg[i] = (tb + i * PAGE < L) ? pt[tb / PAGE + i] : 0;
#pragma unroll
    for (int k = 0; k < CPT; ++k) {
      const int c = tid + k * nthr;
      pk[k] = u32x4_t{0u, 0u, 0u, 0u};
      pv[k] = u32x4_t{0u, 0u, 0u, 0u};
      if (c < NCH) {
        const int j = c / (D / 8), part = c % (D / 8);
        const int pos = tb + j;
        if (pos < L)
          pk[k] = *reinterpret_cast<const u32x4_t*>(
              p.k_pages + (static_cast<int64_t>(pg[j / PAGE]) * p.Hkv + kvh) * head_stride + (j % PAGE) * D + part * 8);
        else if (pos < L + W)
          pk[k] = *reinterpret_cast<const u32x4_t*>(p.k_win + (win_base + static_cast<int64_t>(pos - L) * p.Hkv) * D +
                                                    part * 8);
        const int pi = c / (D * 2), rem = c % (D * 2), d = rem >> 1, h = rem & 1;
        const int t0 = tb + pi * PAGE + h * 8;  // absolute position of the chunk's first token
        u32x4_t v = {0u, 0u, 0u, 0u};
        if (t0 < L) {
          v = *reinterpret_cast<const u32x4_t*>(
              p.v_pages + (static_cast<int64_t>(pg[pi]) * p.Hkv + kvh) * head_stride + d * PAGE + h * 8);
          const int keep = L - t0;  // tokens of the chunk inside the prefix
          if (keep < 8) {
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              const uint32_t lo = (2 * e < keep) ? 0x0000ffffu : 0u, hi = (2 * e + 1 < keep) ? 0xffff0000u : 0u;
              v[e] &= (lo | hi);
            }
          }
        }
        if (t0 + 8 > L && t0 < L + W) {  // window rows inside this chunk (token-minor: one element per row)
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            const int pos = t0 + e;
            if (pos >= L && pos < L + W) {
              const uint32_t x = p.v_win[(win_base + static_cast<int64_t>(pos - L) * p.Hkv) * D + d];
              v[e >> 1] |= (e & 1) ? (x << 16) : x;
            }
          }
        }
        pv[k] = v;
      }
    }
  };
  auto store_tile = [&]() {
#pragma unroll
    for (int k = 0; k < CPT; ++k) {
      const int c = tid + k * nthr;
      if (c < NCH) {
        *reinterpret_cast<u32x4_t*>(&lds_k[k_lds_index<D>(c / (D / 8), c % (D / 8))]) = pk[k];
        const int pi = c / (D * 2), rem = c % (D * 2), d = rem >> 1, h = rem & 1;
        *reinterpret_cast<u32x4_t*>(&lds_v[(pi * D + d) * PAGE + h * 8]) = pv[k];
      }
    }
  };

  if (t_beg < t_end) load_tile(t_beg * TILE);
  for (int t = t_beg; t < t_end; ++t) {
    const int tb = t * TILE;
    __syncthreads();            // the previous tile's compute is done with LDS
    store_tile();
    __syncthreads();
    if (t + 1 < t_end) load_tile(tb + TILE);
    compute_tile([tb, L, W, nc](int roww, int tok) {
      const int pos = tb + tok;
      if (pos < L) return true;
      const int wj = pos - L;  // window row of this key
      return wj < W && (roww >= nc || wj <= roww);
    });
  }

  // ---- epilogue ------------------------------------------------------------------------------------------------
#pragma unroll
  for (int t = 0; t < TPW; ++t) {
    const int nt = wv * TPW + t;
    if (nt >= p.NT) break;
    float lt = l_run[t];
    lt += __shfl_xor(lt, 16, 64);
    lt += __shfl_xor(lt, 32, 64);
    const int n = nt * 16 + l16;
    if (n >= p.R) continue;
    if (p.n_split == 1) {
      const float inv = 1.f / lt;
      const int w = n / p.G, gq = n % p.G;
      uint16_t* orow = p.out + ((static_cast<int64_t>(b) * p.W + w) * p.Hq + kvh * p.G + gq) * D;
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) {
        const floatx4_t v = o[t][dt];
        *reinterpret_cast<u32x2_t*>(orow + dt * 16 + g4 * 4) =
            u32x2_t{pack_bf16x2(v[0] * inv, v[1] * inv), pack_bf16x2(v[2] * inv, v[3] * inv)};
      }
    } else {
      const int64_t base = ((static_cast<int64_t>(b) * p.Hkv + kvh) * p.n_split + s) * p.R + n;
      float* orow = p.ws_o + base * D;
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) *reinterpret_cast<floatx4_t*>(orow + dt * 16 + g4 * 4) = o[t][dt];
      if (g4 == 0) {
        p.ws_ml[base * 2 + 0] = m_run[t];
        p.ws_ml[base * 2 + 1] = lt;
      }
    }
  }
}

// Combine the splits of each (sequence, kv head, row). Block = one query row; thread (dg, sg) owns 4 head dims
// and the splits sg, sg + SG, ...; the SG groups are combined through LDS in group order (deterministic).
template <int D>
__global__ void __launch_bounds__(256) window_attn_merge(AttnParams p) {
  constexpr int DG = D / 4, SG = 256 / DG;
  const int n = blockIdx.x, kvh = blockIdx.y, b = blockIdx.z;
  const int dg = threadIdx.x % DG, sg = threadIdx.x / DG;
  const int64_t hb = (static_cast<int64_t>(b) * p.Hkv + kvh) * p.n_split;
  float M = -INFINITY, den = 0.f;
  floatx4_t acc = {0.f, 0.f, 0.f, 0.f};
  for (int s = sg; s < p.n_split; s += SG) {
    const int64_t r = (hb + s) * p.R + n;
    const float ms = p.ws_ml[r * 2];
    if (ms == -INFINITY) continue;
    const float ls = p.ws_ml[r * 2 + 1];
    const floatx4_t os = *reinterpret_cast<const floatx4_t*>(p.ws_o + r * D + dg * 4);
    const float Mn = fmaxf(M, ms);
    const float a = exp2f(M - Mn), c = exp2f(ms - Mn);
    den = den * a + ls * c;
    acc = acc * a + os * c;
    M = Mn;
  }
  __shared__ float sm[SG][DG], sd[SG][DG];
  __shared__ floatx4_t sa[SG][DG];
  sm[sg][dg] = M;
  sd[sg][dg] = den;
  sa[sg][dg] = acc;
  __syncthreads();
  if (sg != 0) return;
  float Mt = sm[0][dg];
  for (int g = 1; g < SG; ++g) Mt = fmaxf(Mt, sm[g][dg]);
  float dt = 0.f;
  floatx4_t at = {0.f, 0.f, 0.f, 0.f};
  for (int g = 0; g < SG; ++g) {
    if (sm[g][dg] == -INFINITY) continue;
    const float c = exp2f(sm[g][dg] - Mt);
    dt += sd[g][dg] * c;
    at += sa[g][dg] * c;
  }
  const float inv = 1.f / dt;
  const int w = n / p.G, gq = n % p.G;
  uint16_t* orow = p.out + ((static_cast<int64_t>(b) * p.W + w) * p.Hq + kvh * p.G + gq) * D;
  *reinterpret_cast<u32x2_t*>(orow + dg * 4) =
      u32x2_t{pack_bf16x2(at[0] * inv, at[1] * inv), pack_bf16x2(at[2] * inv, at[3] * inv)};
}

// Split count: about target_wgs (sequence, kv head, split) workgroups, each split at least min_tiles 64-token
// tiles of the longest prefix (gss_attn_set_split_policy).
int g_target_wgs = 512, g_min_tiles = 2;

int attn_splits(int bs, int Hkv, int max_kv_len) {
  const int target_wgs = g_target_wgs, min_tiles = g_min_tiles;
  const int tiles = (max(max_kv_len, 1) + TILE - 1) / TILE;
  int by_chip = (target_wgs + bs * Hkv - 1) / (bs * Hkv);
  int by_len = (tiles + min_tiles - 1) / min_tiles;
  int s = min(by_chip, by_len);
  return max(1, min(s, 256));
}

int choose_tpw(int NT, int* nw) {
  const int tpw = NT <= MAX_WAVES ? 1 : 2;
  *nw = max(MIN_WAVES, (NT + tpw - 1) / tpw);
  return tpw;
}

int validate(int bs, int W, int Hq, int Hkv, int D, int page) {
  if (bs <= 0 || W <= 0 || Hq <= 0 || Hkv <= 0) return GSS_ERR_ARG;
  if (Hq % Hkv != 0) return GSS_ERR_UNSUPPORTED;
  if (D != 64 && D != 128) return GSS_ERR_UNSUPPORTED;
  if (page != PAGE || W > TILE) return GSS_ERR_UNSUPPORTED;
  const int R = (Hq / Hkv) * W, NT = (R + 15) / 16;
  if (NT > MAX_NT) return GSS_ERR_UNSUPPORTED;
  return GSS_OK;
}

template <int D, int TPW>
void launch_kernel(const AttnParams& p, dim3 grid, int nw, size_t lds_q, hipStream_t st) {
  constexpr int NCH = TILE * D / 8;
  const int cpt = (NCH + 64 * nw - 1) / (64 * nw);
  if (cpt <= 2)
    hipLaunchKernelGGL((window_attn_kernel<D, TPW, 2>), grid, dim3(64 * nw), lds_q, st, p);
  else
    hipLaunchKernelGGL((window_attn_kernel<D, TPW, 4>), grid, dim3(64 * nw), lds_q, st, p);
}

template <int D>
int launch_d(const AttnParams& p, int bs, int tpw, int nw, hipStream_t st) {
  const dim3 grid(p.n_split, p.Hkv, bs);
  const size_t lds_q = static_cast<size_t>(p.NT) * 16 * D * sizeof(uint16_t);
  static bool lds_attr_set = false;  // allow the dynamic Q tile beyond the default 64 KB (set once, before use)
  if (!lds_attr_set) {
    const int max_dyn = MAX_NT * 16 * D * static_cast<int>(sizeof(uint16_t));
    const void* fns[] = {reinterpret_cast<const void*>(&window_attn_kernel<D, 1, 2>),
                         reinterpret_cast<const void*>(&window_attn_kernel<D, 1, 4>),
                         reinterpret_cast<const void*>(&window_attn_kernel<D, 2, 2>),
                         reinterpret_cast<const void*>(&window_attn_kernel<D, 2, 4>)};
    for (const void* f : fns)
      if (hipFuncSetAttribute(f, hipFuncAttributeMaxDynamicSharedMemorySize, max_dyn) != hipSuccess)
        return GSS_ERR_LAUNCH;
    lds_attr_set = true;
  }
  if (tpw == 1)
    launch_kernel<D, 1>(p, grid, nw, lds_q, st);
  else
    launch_kernel<D, 2>(p, grid, nw, lds_q, st);
  if (p.n_split > 1) hipLaunchKernelGGL((window_attn_merge<D>), dim3(p.R, p.Hkv, bs), dim3(256), 0, st, p);
  return gss_launch_status();
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
  p.NT = (p.R + 15) / 16;
  p.n_split = attn_splits(bs, Hkv, max_kv_len);
  const int tiles_max = (max_kv_len + W + TILE - 1) / TILE;  // tiles of the longest key sequence
  p.tps = (tiles_max + p.n_split - 1) / p.n_split;
  p.scale_log2 = scale * LOG2E;
  p.ws_o = nullptr;
  p.ws_ml = nullptr;
  if (p.n_split > 1) {
    size_t need = 0;
    gss_attn_workspace_size(bs, Hq, Hkv, D, W, max_kv_len, &need);
    if (!workspace || workspace_bytes < need) return GSS_ERR_WORKSPACE;
    p.ws_o = static_cast<float*>(workspace);
    p.ws_ml = p.ws_o + static_cast<size_t>(bs) * Hkv * p.n_split * p.R * D;
  }
  int nw;
  const int tpw = choose_tpw(p.NT, &nw);
  return D == 128 ? launch_d<128>(p, bs, tpw, nw, st) : launch_d<64>(p, bs, tpw, nw, st);
}

}  // namespace

extern "C" int gss_attn_workspace_size(int bs, int Hq, int Hkv, int D, int W, int max_kv_len, size_t* bytes) {
  if (!bytes) return GSS_ERR_ARG;
  const int rc = validate(bs, W, Hq, Hkv, D, PAGE);
  if (rc != GSS_OK) return rc;
  const int R = (Hq / Hkv) * W;
  const int ns = attn_splits(bs, Hkv, max_kv_len);
  *bytes = ns > 1 ? static_cast<size_t>(bs) * Hkv * ns * R * (D + 2) * sizeof(float) : 0;
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
  if (target_wgs < 1 || min_tiles < 1) return GSS_ERR_ARG;
  g_target_wgs = target_wgs;
  g_min_tiles = min_tiles;
  return GSS_OK;
}
