// Skinny GEMM for the decode forwards: Y[M, N] = X[M, Kd] . W[N, Kd]^T with M = bs * window rows, bf16 operands,
// fp32 accumulation. Weight streaming is the whole cost at M <= 64 (N*Kd*2 bytes per call), so the kernel is built
// to keep many 16-byte weight loads in flight and to touch every weight byte exactly once. Batched windows (M > 64)
// run on a tiled kernel (gemm_tiled_kernel) that computes every element with the same sequence of operations.
//
// Layout on v_mfma_f32_16x16x32_bf16: A = 16 weight rows x 32 k (lane: row l%16, k 8*(l/16)..+7, one 16-byte
// load), B = 32 k x 16 activation rows (lane: activation row l%16, same k), C = Y^T tile (lane: 4 consecutive
// features of one activation row). A workgroup owns FT*16 output features; its waves split the k-steps into
// contiguous ranges and reduce their partial tiles through LDS in wave order.
//
// Batch invariance: an output element is always the same sequence of MFMA k-steps and the same wave-order
// reduction, whatever M is, whichever kernel runs it and wherever its row sits, so a row computed in a 17-row verify
// forward or a 544-row batched verify is bit-identical to the same row computed alone (a 1-row AR step). Decode parity between speculative and AR decoding rests on it.
//
// Fused epilogues (the GEMM output is rounded to bf16 first, as a bf16 torch linear writes it):
//   EPI_PLAIN   Y bf16 (or fp32) [M, ldy]
//   EPI_ROPE    N = (Hq + 2 Hkv) * D q|k|v projection -> RoPE on q and k (interleaved pairs of the first rot_dim dims,
//               position = seq_lens[b] + pos_delta[b] + w), written as q [bs, W, Hq, D] and window K/V [bs, W, Hkv, D]
//   EPI_SWIGLU  N = 2F with gate/up rows interleaved (row 2i = gate_i, 2i+1 = up_i) -> act[M, F] = up * silu(gate)
//   EPI_PARTS   the k splits' fp32 partial sums [S][M][N], summed in split order (then rounded to bf16) by the
//               consumer: no handoff between the splits, the kernel boundary orders them
#include "gss_common.h"

namespace {

enum { EPI_PLAIN = 0, EPI_ROPE = 1, EPI_SWIGLU = 2, EPI_PARTS = 3 };

struct GemmParams {
  const uint16_t* x;
  int64_t ldx;
  const uint16_t* w;
  int64_t ldw;
  void* y;
  int64_t ldy;
  int M, N, Kd;
  int out_f32;
  // EPI_ROPE
  const int32_t* seq_lens;
  const int32_t* pos_delta;
  const float* inv_freq;
  int rot_dim, W, Hq, Hkv, D;
  uint16_t* q_out;
  uint16_t* k_out;
  uint16_t* v_out;
  // prologue (PRO_ADDNORM): x = rmsnorm(h') * w_next with h' = h_in + rmsnorm(a) * w_post (a == nullptr: h' = h_in);
  // workgroup (0, 0) stores h' to h_out (never h_in: other workgroups still read it)
  const uint16_t* pa;
  const float* pa_parts;  // or a given as n_parts fp32 partial sums [n_parts][M][Kd] (a = bf16 of their sum)
  int n_parts;
  const uint16_t* h_in;
  uint16_t* h_out;
  const uint16_t* w_post;
  const uint16_t* w_next;
  float eps;
  // split-K over workgroups (blockIdx.y = split): fp32 partials [ksplit][M][N] and per-column-tile counters
  int ksplit, kps;  // splits, k-steps per split
  float* part;
  uint32_t* tile_ctr;
  // post-norm epilogue (gss_norm_epilogue): the last column tile to finish runs, on every row,
  // h = h + rmsnorm(Y) * w_post; x = rmsnorm(h) * w_next
  uint16_t* post_h;
  const uint16_t* post_wp;
  const uint16_t* post_wn;
  uint16_t* post_x;
  float post_eps;
  uint32_t* done_ctr;
};

constexpr int MAX_NW = 12;  // waves per workgroup (768 threads: 168 VGPRs per lane)
constexpr size_t MAX_LDS = 160 * 1024;  // LDS per workgroup on gfx950
constexpr size_t MAX_DYN_LDS = MAX_LDS - 1024;  // dynamic part of it (the kernels' static LDS is a few bytes)

// Wave w owns the contiguous k-steps [w*ksw, (w+1)*ksw) and walks them in passes of UNR steps; every weight and
// activation load of a pass is issued before the pass's first MFMA, so each wave keeps UNR*(FT+NT) 16-byte loads
// in flight and a workgroup needs ceil(ksw / UNR) HBM round trips for its whole weight slice.
enum { PRO_NONE = 0, PRO_ADDNORM = 1 };
constexpr int XPAD = 8;  // bf16 elements of padding per LDS activation row (spreads rows over the LDS banks)

typedef __attribute__((address_space(1))) void gvoid_t;  // global memory (direct-to-LDS load source)
typedef __attribute__((address_space(3))) void lvoid_t;  // LDS (its destination)

// Activation staging (XS): a vector memory instruction costs the CU's address unit about the same whatever its
// active lanes, so a fragment load of a partly filled row tile (17 rows: the second tile has one live row) costs as
// much as a full one. Instead each wave copies its own k-range of all M rows into LDS with full-lane direct-to-LDS
// loads (64 x 16-byte chunks per instruction) and reads its B fragments from there. Chunk c (16 bytes) of row r of
// the wave's range sits at slot r * CPR + (c ^ (r & 15)), CPR = 16-byte chunks per row (a multiple of 16): the 16
// rows of one fragment read land in 16 different bank groups.
GSS_DEV int xs_slot(int r, int c, int cpr) { return r * cpr + (c ^ (r & 15)); }

// global -> LDS, 16 bytes per lane, from a wave-uniform base held in scalar registers plus a 32-bit per-lane byte
// offset, into the wave-uniform LDS byte address lds + 16 * lane: no 64-bit address arithmetic per lane
GSS_DEV void dma16s(const void* sbase, uint32_t voff, uint32_t lds) {
  asm volatile("global_load_lds_dwordx4 %0, %1" ::"v"(voff), "s"(sbase), "{m0}"(lds) : "memory");
}

// a pointer that is the same in every lane, moved to scalar registers (no-op when it already is there)
GSS_DEV const char* uniform_ptr(const void* ptr) {
  const uint64_t a = reinterpret_cast<uint64_t>(ptr);
  const uint32_t lo = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(a));
  const uint32_t hi = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(a >> 32));
  return reinterpret_cast<const char*>((static_cast<uint64_t>(hi) << 32) | lo);
}

// s_waitcnt immediate (gfx9 encoding) that waits until at most n vector memory operations are outstanding and
// leaves the other counters free: vmcnt[3:0] in bits 3:0, expcnt 7 in bits 6:4, lgkmcnt 15 in bits 11:8. The
// builtin form lets the compiler's own wait counting see the direct-to-LDS loads complete.
constexpr int waitcnt_vm(int n) { return (n & 15) | (7 << 4) | (15 << 8) | ((n >> 4) << 14); }

// Prologue: the normalized activation rows x (bf16) go to LDS. One wavefront per row; lane l owns the E = Kd/64
// consecutive elements [l*E, (l+1)*E); the arithmetic and rounding points are gss_add_rmsnorm's, so the fused and
// unfused paths agree bit for bit.
template <int E>
GSS_DEV void addnorm_row(const GemmParams& p, int row, int lane, uint16_t* xs, bool store_h) {
  constexpr int KD = 64 * E;
  const int64_t off = static_cast<int64_t>(row) * KD + lane * E;
  float hv[E], av[E], wn[E], wp[E];
#pragma unroll
  for (int c = 0; c < E / 8; ++c) {
    const u32x4_t qh = *reinterpret_cast<const u32x4_t*>(p.h_in + off + c * 8);
    const u32x4_t qn = *reinterpret_cast<const u32x4_t*>(p.w_next + lane * E + c * 8);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      hv[c * 8 + 2 * e] = __uint_as_float(qh[e] << 16);
      hv[c * 8 + 2 * e + 1] = __uint_as_float(qh[e] & 0xffff0000u);
      wn[c * 8 + 2 * e] = __uint_as_float(qn[e] << 16);
      wn[c * 8 + 2 * e + 1] = __uint_as_float(qn[e] & 0xffff0000u);
    }
    if (p.pa_parts != nullptr) {
      // a = bf16 of the partial sums, added in part order (gss_add_rmsnorm_parts' arithmetic)
      const float* pp = p.pa_parts + off + c * 8;
      const int64_t pstride = static_cast<int64_t>(p.M) * KD;
      floatx4_t s0 = *reinterpret_cast<const floatx4_t*>(pp), s1 = *reinterpret_cast<const floatx4_t*>(pp + 4);
      for (int k = 1; k < p.n_parts; ++k) {
        s0 += *reinterpret_cast<const floatx4_t*>(pp + k * pstride);
        s1 += *reinterpret_cast<const floatx4_t*>(pp + k * pstride + 4);
      }
      const u32x4_t qp = *reinterpret_cast<const u32x4_t*>(p.w_post + lane * E + c * 8);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        av[c * 8 + e] = round_bf16(s0[e]);
        av[c * 8 + 4 + e] = round_bf16(s1[e]);
        wp[c * 8 + 2 * e] = __uint_as_float(qp[e] << 16);
        wp[c * 8 + 2 * e + 1] = __uint_as_float(qp[e] & 0xffff0000u);
      }
    } else if (p.pa != nullptr) {
      const u32x4_t qa = *reinterpret_cast<const u32x4_t*>(p.pa + off + c * 8);
      const u32x4_t qp = *reinterpret_cast<const u32x4_t*>(p.w_post + lane * E + c * 8);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        av[c * 8 + 2 * e] = __uint_as_float(qa[e] << 16);
        av[c * 8 + 2 * e + 1] = __uint_as_float(qa[e] & 0xffff0000u);
        wp[c * 8 + 2 * e] = __uint_as_float(qp[e] << 16);
        wp[c * 8 + 2 * e + 1] = __uint_as_float(qp[e] & 0xffff0000u);
      }
    }
  }
  if (p.pa != nullptr || p.pa_parts != nullptr) {
    float ss = 0.f;
#pragma unroll
    for (int e = 0; e < E; ++e) ss += av[e] * av[e];
    const float ra = 1.f / sqrtf(wave_sum(ss) / static_cast<float>(KD) + p.eps);
#pragma unroll
    for (int e = 0; e < E; ++e) hv[e] = round_bf16(hv[e] + round_bf16(wp[e] * round_bf16(av[e] * ra)));
  }
  float sh = 0.f;
#pragma unroll
  for (int e = 0; e < E; ++e) sh += hv[e] * hv[e];
  const float rh = 1.f / sqrtf(wave_sum(sh) / static_cast<float>(KD) + p.eps);
  uint16_t* xrow = xs + row * (KD + XPAD) + lane * E;
#pragma unroll
  for (int c = 0; c < E / 8; ++c) {
    float xv[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) xv[e] = wn[c * 8 + e] * round_bf16(hv[c * 8 + e] * rh);
    *reinterpret_cast<u32x4_t*>(xrow + c * 8) = u32x4_t{pack_bf16x2(xv[0], xv[1]), pack_bf16x2(xv[2], xv[3]),
                                                       pack_bf16x2(xv[4], xv[5]), pack_bf16x2(xv[6], xv[7])};
    if (store_h)
      *reinterpret_cast<u32x4_t*>(p.h_out + off + c * 8) =
          u32x4_t{pack_bf16x2(hv[c * 8], hv[c * 8 + 1]), pack_bf16x2(hv[c * 8 + 2], hv[c * 8 + 3]),
                  pack_bf16x2(hv[c * 8 + 4], hv[c * 8 + 5]), pack_bf16x2(hv[c * 8 + 6], hv[c * 8 + 7])};
  }
}

// Post-norm of one row (one wavefront; H = p.N = 64 * E with E = 8 * nc, nc <= 4): the arithmetic, order and
// rounding points of gss_add_rmsnorm, so the fused and separate norms agree bit for bit. The GEMM output rows were
// handed over through the coherence point (coherent loads); h and the weights were written before this kernel.
constexpr int POST_MAX_E = 32;
GSS_DEV void post_addnorm_row(const GemmParams& p, int row, int lane) {
  const int E = p.N / 64, nc = E / 8;
  const int64_t off = static_cast<int64_t>(row) * p.N + lane * E;
  const uint16_t* a = static_cast<const uint16_t*>(p.y) + off;
  u32x4_t qa[4];
  ld_agent_x4(nc, a, a + 8 * min(1, nc - 1), a + 8 * min(2, nc - 1), a + 8 * min(3, nc - 1), qa[0], qa[1], qa[2],
              qa[3]);
  float av[POST_MAX_E], hv[POST_MAX_E], wp[POST_MAX_E], wn[POST_MAX_E];
#pragma unroll
  for (int c = 0; c < POST_MAX_E / 8; ++c) {
    if (c < nc) {
      const u32x4_t qh = *reinterpret_cast<const u32x4_t*>(p.post_h + off + 8 * c);
      const u32x4_t qp = *reinterpret_cast<const u32x4_t*>(p.post_wp + lane * E + 8 * c);
      const u32x4_t qn = *reinterpret_cast<const u32x4_t*>(p.post_wn + lane * E + 8 * c);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        av[8 * c + 2 * e] = __uint_as_float(qa[c][e] << 16);
        av[8 * c + 2 * e + 1] = __uint_as_float(qa[c][e] & 0xffff0000u);
        hv[8 * c + 2 * e] = __uint_as_float(qh[e] << 16);
        hv[8 * c + 2 * e + 1] = __uint_as_float(qh[e] & 0xffff0000u);
        wp[8 * c + 2 * e] = __uint_as_float(qp[e] << 16);
        wp[8 * c + 2 * e + 1] = __uint_as_float(qp[e] & 0xffff0000u);
        wn[8 * c + 2 * e] = __uint_as_float(qn[e] << 16);
        wn[8 * c + 2 * e + 1] = __uint_as_float(qn[e] & 0xffff0000u);
      }
    }
  }
  float ss = 0.f;
#pragma unroll
  for (int e = 0; e < POST_MAX_E; ++e)
    if (e < E) ss += av[e] * av[e];
  const float ra = 1.f / sqrtf(wave_sum(ss) / static_cast<float>(p.N) + p.post_eps);
  float sh = 0.f;
#pragma unroll
  for (int e = 0; e < POST_MAX_E; ++e) {
    if (e < E) {
      hv[e] = round_bf16(hv[e] + round_bf16(wp[e] * round_bf16(av[e] * ra)));
      sh += hv[e] * hv[e];
    }
  }
  const float rh = 1.f / sqrtf(wave_sum(sh) / static_cast<float>(p.N) + p.post_eps);
#pragma unroll
  for (int c = 0; c < POST_MAX_E / 8; ++c) {
    if (c < nc) {
      const float* h8 = hv + 8 * c;
      float x8[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) x8[e] = wn[8 * c + e] * round_bf16(h8[e] * rh);
      *reinterpret_cast<u32x4_t*>(p.post_h + off + 8 * c) =
          u32x4_t{pack_bf16x2(h8[0], h8[1]), pack_bf16x2(h8[2], h8[3]), pack_bf16x2(h8[4], h8[5]),
                  pack_bf16x2(h8[6], h8[7])};
      *reinterpret_cast<u32x4_t*>(p.post_x + off + 8 * c) =
          u32x4_t{pack_bf16x2(x8[0], x8[1]), pack_bf16x2(x8[2], x8[3]), pack_bf16x2(x8[4], x8[5]),
                  pack_bf16x2(x8[6], x8[7])};
    }
  }
}

// RoPE factors of a lane's 4 output features (two rotated pairs): the position and inverse frequencies are fetched
// first (rope_fetch, before a kernel's weight loads, so they arrive under them), the bf16-rounded cos / sin computed
// afterwards (rope_math, while the weights are in flight), so the epilogue has neither a memory round trip nor the
// transcendental functions on its path. The same expressions as computed in place, so the same bits.
struct RopeIn {
  int s0, s1, w, d;  // seq_lens[b], pos_delta[b] (or a stand-in), window row, head dim of the first feature
  float i0, i1;      // inverse frequencies of the two pairs (clamped index)
};
struct RopeCS {
  float c[2], s[2];
};
GSS_DEV RopeIn rope_fetch(const GemmParams& p, int row, int feat) {
  // loads only, every one unconditional and in bounds (their values are used by rope_math), so no wait is forced
  // before the loads that follow
  row = min(row, p.M - 1);  // rows past M are never stored
  const int b = row / p.W;
  RopeIn r;
  r.w = row % p.W;
  r.d = feat % p.D;
  const int32_t* pd = p.pos_delta ? p.pos_delta : p.seq_lens;
  // (no rotated dims: read a valid int instead, never used)
  const float* fq = p.rot_dim >= 2 ? p.inv_freq : reinterpret_cast<const float*>(p.seq_lens);
  const int hi = max(p.rot_dim - 2, 0);
  r.s0 = p.seq_lens[b];
  r.s1 = pd[b];
  r.i0 = fq[min(r.d, hi) >> 1];
  r.i1 = fq[min(r.d + 2, hi) >> 1];
  return r;
}
GSS_DEV RopeCS rope_math(const GemmParams& p, const RopeIn& r) {
  const int pos = r.s0 + (p.pos_delta ? r.s1 : 0) + r.w;
  const float fr0 = static_cast<float>(pos) * (r.d < p.rot_dim ? r.i0 : 0.f);
  const float fr1 = static_cast<float>(pos) * (r.d + 2 < p.rot_dim ? r.i1 : 0.f);
  RopeCS cs;
  cs.c[0] = round_bf16(cosf(fr0));
  cs.s[0] = round_bf16(sinf(fr0));
  cs.c[1] = round_bf16(cosf(fr1));
  cs.s[1] = round_bf16(sinf(fr1));
  return cs;
}

// Epilogue of output tile (f, n) of the workgroup whose first feature is f0 and first row row0, on its reduced sum s
// (lane: activation row row0 + n*16 + l16, features f0 + f*16 + g4*4 .. +3). The GEMM output is rounded to bf16
// first, as a bf16 torch linear writes it. EPI_ROPE takes the lane's precomputed factors if given (pre), else
// computes them here.
template <int EPI, bool POST>
GSS_DEV void gemm_epilogue(const GemmParams& p, int f0, int row0, int f, int n, floatx4_t s, int l16, int g4,
                           const RopeCS* pre = nullptr) {
  const int row = row0 + n * 16 + l16;     // activation row
  const int feat = f0 + f * 16 + g4 * 4;   // first of this lane's 4 consecutive output features
  float y0 = s[0], y1 = s[1], y2 = s[2], y3 = s[3];
  if constexpr (EPI == EPI_PLAIN) {
    if (p.out_f32) {
      *reinterpret_cast<floatx4_t*>(static_cast<float*>(p.y) + static_cast<int64_t>(row) * p.ldy + feat) = s;
    } else if constexpr (POST) {  // the rows are handed to the workgroup that runs the norm
      uint32_t* dst = reinterpret_cast<uint32_t*>(static_cast<uint16_t*>(p.y) + static_cast<int64_t>(row) * p.ldy +
                                                  feat);
      st_agent(dst, pack_bf16x2(y0, y1));
      st_agent(dst + 1, pack_bf16x2(y2, y3));
    } else {
      *reinterpret_cast<u32x2_t*>(static_cast<uint16_t*>(p.y) + static_cast<int64_t>(row) * p.ldy + feat) =
          u32x2_t{pack_bf16x2(y0, y1), pack_bf16x2(y2, y3)};
    }
  } else if constexpr (EPI == EPI_SWIGLU) {
    // features (gate_i, up_i, gate_i+1, up_i+1), i = feat / 2
    const float g0 = round_bf16(y0), u0 = round_bf16(y1), g1 = round_bf16(y2), u1 = round_bf16(y3);
    const float s0 = round_bf16(g0 / (1.f + expf(-g0))), s1 = round_bf16(g1 / (1.f + expf(-g1)));
    *reinterpret_cast<uint32_t*>(static_cast<uint16_t*>(p.y) + static_cast<int64_t>(row) * p.ldy + feat / 2) =
        pack_bf16x2(u0 * s0, u1 * s1);
  } else {  // EPI_ROPE
    const int head = feat / p.D, d = feat % p.D;  // 4 features never straddle a head (D % 16 == 0)
    float o[4] = {round_bf16(y0), round_bf16(y1), round_bf16(y2), round_bf16(y3)};
    if (head < p.Hq + p.Hkv) {
      const RopeCS cs = pre ? *pre : rope_math(p, rope_fetch(p, row, feat));
#pragma unroll
      for (int e = 0; e < 4; e += 2) {
        if (d + e < p.rot_dim) {
          const float c = cs.c[e >> 1], sn = cs.s[e >> 1];
          const float x0 = o[e], x1 = o[e + 1];
          o[e] = round_bf16(round_bf16(x0 * c) - round_bf16(x1 * sn));
          o[e + 1] = round_bf16(round_bf16(x1 * c) + round_bf16(x0 * sn));
        }
      }
    }
    uint16_t* dst;
    if (head < p.Hq)
      dst = p.q_out + (static_cast<int64_t>(row) * p.Hq + head) * p.D + d;
    else if (head < p.Hq + p.Hkv)
      dst = p.k_out + (static_cast<int64_t>(row) * p.Hkv + (head - p.Hq)) * p.D + d;
    else
      dst = p.v_out + (static_cast<int64_t>(row) * p.Hkv + (head - p.Hq - p.Hkv)) * p.D + d;
    *reinterpret_cast<u32x2_t*>(dst) = u32x2_t{pack_bf16x2(o[0], o[1]), pack_bf16x2(o[2], o[3])};
  }
}

template <int FT, int NT, int UNR, int EPI, int PRO = PRO_NONE, int E = 8, bool POST = false, bool XS = false>
__global__ void __launch_bounds__(64 * MAX_NW) gemm_kernel(GemmParams p, int ksw) {
  // LDS: [NW][FT][NT][64] wave partials, then (PRO_ADDNORM) x rows [M][Kd + XPAD] or (XS) per wave [M][ksw * 4]
  // 16-byte chunks of its k-range
  extern __shared__ floatx4_t red[];
  // the kernel arguments of the staging, weight and RoPE loads in one scalar batch (loaded where first used, they
  // came in two dependent round trips)
  asm volatile("" ::"s"(p.x), "s"(p.ldx), "s"(p.w), "s"(p.ldw), "s"(p.M), "s"(p.N), "s"(p.Kd), "s"(p.kps),
               "s"(p.seq_lens), "s"(p.pos_delta), "s"(p.inv_freq), "s"(p.rot_dim), "s"(p.W), "s"(p.D), "s"(ksw),
               "s"(static_cast<int>(blockDim.x)));
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6, NW = blockDim.x >> 6;
  const int l16 = lane & 15, g4 = lane >> 4;
  const int f0 = blockIdx.x * FT * 16;
  const int row0 = 0, Ms = p.M;  // every row (M <= 64)
  const uint16_t* xs0 = p.x;
  const int ksteps = p.Kd / 32;
  const int ks = blockIdx.y;  // k split: k-steps [ks * kps, (ks + 1) * kps)
  const int k_end = min(ksteps, (ks + 1) * p.kps);
  const int s_beg = ks * p.kps + wv * ksw, s_end = min(k_end, s_beg + ksw);

  floatx4_t acc[FT][NT];
#pragma unroll
  for (int f = 0; f < FT; ++f)
#pragma unroll
    for (int n = 0; n < NT; ++n) acc[f][n] = floatx4_t{0.f, 0.f, 0.f, 0.f};

  const uint16_t* wrow[FT];
#pragma unroll
  for (int f = 0; f < FT; ++f) {
    const int row = min(f0 + f * 16 + l16, p.N - 1);  // rows past N repeat the last (never stored)
    wrow[f] = p.w + static_cast<int64_t>(row) * p.ldw + g4 * 8;
  }
  const uint16_t* xrow[NT];
  bool xlive[NT];
#pragma unroll
  for (int n = 0; n < NT; ++n) {
    const int r = n * 16 + l16;
    xlive[n] = r < Ms;
    xrow[n] = xs0 + static_cast<int64_t>(xlive[n] ? r : 0) * p.ldx + g4 * 8;
  }

  // RoPE factors of the output tiles this wave finishes ((f * NT + n) % NW == wv): fetched before any other load (so
  // they arrive under the weights), computed after the MFMAs
  RopeIn rin[FT][NT];
  RopeCS rcs[FT][NT];
  auto owns = [&](int f, int n) { return (f * NT + n) % NW == wv; };
  if constexpr (EPI == EPI_ROPE) {
#pragma unroll
    for (int f = 0; f < FT; ++f)
#pragma unroll
      for (int n = 0; n < NT; ++n) rin[f][n] = rope_fetch(p, row0 + n * 16 + l16, f0 + f * 16 + g4 * 4);
  }
  auto rope_prepare = [&]() {
    if constexpr (EPI == EPI_ROPE) {
#pragma unroll
      for (int f = 0; f < FT; ++f)
#pragma unroll
        for (int n = 0; n < NT; ++n)
          if (owns(f, n)) rcs[f][n] = rope_math(p, rin[f][n]);
    }
  };

  uint16_t* xs = reinterpret_cast<uint16_t*>(red + NW * FT * NT * 64);
  // XS runs only with ksw == UNR (the host checks), so a staged row holds a compile-time 4 * UNR chunks
  const int cpr = XS ? UNR * 4 : ksw * 4;
  uint16_t* xw = xs + wv * Ms * cpr * 8;  // XS: this wave's staged rows
  if constexpr (XS) {
    // one pass: rows 0..Ms-1, k-steps [s_beg, s_end) -> LDS, issued before the weight loads below. LDS slot
    // q = j * 64 + lane holds chunk (q % CPR) ^ (r & 15) of row r = q / CPR; each instruction is a few VALU
    // operations on a row offset that steps by a uniform amount (a wave issues one instruction every few clocks, and
    // these loads go out before the weights').
    constexpr int CPR = UNR * 4, DR = 64 / CPR;
    static_assert(64 % CPR == 0 && CPR >= 16, "a chunk swizzle by r & 15 must stay inside the row");
    const int n_slots = Ms * CPR, live_chunks = (s_end - s_beg) * 4;
    const char* xbase = uniform_ptr(xs0 + static_cast<int64_t>(s_beg) * 32);
    const uint32_t lds0 = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(reinterpret_cast<uintptr_t>(xw)));
    const int cl = lane % CPR;
    int r = lane / CPR;
    uint32_t rofs = static_cast<uint32_t>(r * p.ldx * 2);
    const uint32_t rstep = static_cast<uint32_t>(DR * p.ldx * 2);
#pragma unroll 1
    for (int j = 0; j * 64 < n_slots; ++j) {
      const int c = cl ^ (r & 15);
      if (j * 64 + lane < n_slots && c < live_chunks) dma16s(xbase, rofs + c * 16, lds0 + j * 1024);
      r += DR;
      rofs += rstep;
    }
  }
  // PRO_ADDNORM runs exactly one pass on every wave (the prologue has a workgroup barrier)
  const int sp_end = PRO == PRO_ADDNORM ? s_beg + 1 : s_end;
  for (int sp = s_beg; sp < sp_end; sp += UNR) {
    u32x4_t wa[UNR][FT];
    u32x4_t xb[UNR][NT];
#pragma unroll
    for (int u = 0; u < UNR; ++u) {
      const int s = sp + u;
      const bool on = s < s_end;
#pragma unroll
      for (int f = 0; f < FT; ++f)
        wa[u][f] = on ? *reinterpret_cast<const u32x4_t*>(wrow[f] + s * 32) : u32x4_t{0u, 0u, 0u, 0u};
    }
    if constexpr (PRO == PRO_ADDNORM) {
      // the weight loads above are in flight; build the normalized rows meanwhile (single pass: ksw <= UNR)
      for (int r = wv; r < p.M; r += NW)
        addnorm_row<E>(p, r, lane, xs, (blockIdx.x | blockIdx.y) == 0 && p.h_out != nullptr);
      __syncthreads();
#pragma unroll
      for (int u = 0; u < UNR; ++u) {
        const int s = sp + u;
#pragma unroll
        for (int n = 0; n < NT; ++n)
          xb[u][n] = (s < s_end && xlive[n])
                         ? *reinterpret_cast<const u32x4_t*>(xs + (n * 16 + l16) * (p.Kd + XPAD) + s * 32 + g4 * 8)
                         : u32x4_t{0u, 0u, 0u, 0u};
      }
    } else if constexpr (XS) {
      __builtin_amdgcn_s_waitcnt(waitcnt_vm(0));  // the staged rows (and the weights) have landed
#pragma unroll
      for (int u = 0; u < UNR; ++u) {
#pragma unroll
        for (int n = 0; n < NT; ++n) {
          const int r = n * 16 + l16;
          xb[u][n] = (sp + u < s_end && xlive[n])
                         ? *reinterpret_cast<const u32x4_t*>(xw + xs_slot(r, u * 4 + g4, cpr) * 8)
                         : u32x4_t{0u, 0u, 0u, 0u};
        }
      }
    } else {
#pragma unroll
      for (int u = 0; u < UNR; ++u) {
        const int s = sp + u;
#pragma unroll
        for (int n = 0; n < NT; ++n)
          xb[u][n] = (s < s_end && xlive[n]) ? *reinterpret_cast<const u32x4_t*>(xrow[n] + s * 32)
                                             : u32x4_t{0u, 0u, 0u, 0u};
      }
    }
#pragma unroll
    for (int u = 0; u < UNR; ++u) {
      if (sp + u < s_end) {
#pragma unroll
        for (int f = 0; f < FT; ++f)
#pragma unroll
          for (int n = 0; n < NT; ++n)
            acc[f][n] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, wa[u][f]),
                                                                __builtin_bit_cast(bf16x8_t, xb[u][n]), acc[f][n], 0,
                                                                0, 0);
      }
    }
  }

  rope_prepare();  // (inside the load pass, the compiler hoists it above the weight loads)

  // ---- reduce the NW wave partials in wave order --------------------------------------------------------------
#pragma unroll
  for (int f = 0; f < FT; ++f)
#pragma unroll
    for (int n = 0; n < NT; ++n) red[((wv * FT + f) * NT + n) * 64 + lane] = acc[f][n];
  __syncthreads();

  // epilogue of tile (f, n) on its reduced sum (wave v owns the tiles with (f * NT + n) % NW == v)
  auto epilogue = [&](int f, int n, floatx4_t s) {
    gemm_epilogue<EPI, POST>(p, f0, row0, f, n, s, l16, g4, EPI == EPI_ROPE ? &rcs[f][n] : nullptr);
  };
  auto reduced = [&](int f, int n) {
    floatx4_t s = red[((0 * FT + f) * NT + n) * 64 + lane];
    for (int v = 1; v < NW; ++v) s += red[((v * FT + f) * NT + n) * 64 + lane];
    return s;
  };
  auto live = [&](int f, int n) { return n * 16 + l16 < Ms && f0 + f * 16 + g4 * 4 < p.N; };
  __shared__ int last_flag;

  if constexpr (EPI == EPI_PARTS) {
    // this split's fp32 partial sums, plain stores (read by a later kernel)
#pragma unroll
    for (int f = 0; f < FT; ++f)
#pragma unroll
      for (int n = 0; n < NT; ++n)
        if ((f * NT + n) % NW == wv && live(f, n))
          *reinterpret_cast<floatx4_t*>(static_cast<float*>(p.y) +
                                        (static_cast<int64_t>(ks) * p.M + row0 + n * 16 + l16) * p.ldy + f0 + f * 16 +
                                        g4 * 4) = reduced(f, n);
    return;
  }
  if (p.ksplit == 1) {
#pragma unroll
    for (int f = 0; f < FT; ++f)
#pragma unroll
      for (int n = 0; n < NT; ++n)
        if ((f * NT + n) % NW == wv && live(f, n)) epilogue(f, n, reduced(f, n));
  } else {
    // this split's partial tile -> workspace; the last split of the column tile to arrive sums all splits in split
    // order and runs the epilogue, then resets the counter. Partials are agent-scope stores (written through to the
    // coherence point), waited for before the barrier and the counter bump; the last reads them with agent loads.
    auto part_at = [&](int k, int f, int n) {
      return reinterpret_cast<uint64_t*>(p.part + (static_cast<int64_t>(k) * p.M + row0 + n * 16 + l16) * p.N + f0 +
                                         f * 16 + g4 * 4);
    };
#pragma unroll
    for (int f = 0; f < FT; ++f)
#pragma unroll
      for (int n = 0; n < NT; ++n)
        if ((f * NT + n) % NW == wv && live(f, n)) {
          const floatx4_t r = reduced(f, n);
          uint64_t* dst = part_at(ks, f, n);
          st_agent(dst, (static_cast<uint64_t>(__float_as_uint(r[1])) << 32) | __float_as_uint(r[0]));
          st_agent(dst + 1, (static_cast<uint64_t>(__float_as_uint(r[3])) << 32) | __float_as_uint(r[2]));
        }
    wait_stores();
    __syncthreads();
    if (tid == 0) last_flag = count_arrival(&p.tile_ctr[blockIdx.x]) == static_cast<uint32_t>(p.ksplit - 1);
    __syncthreads();
    if (!last_flag) return;
#pragma unroll
    for (int f = 0; f < FT; ++f)
#pragma unroll
      for (int n = 0; n < NT; ++n) {
        if ((f * NT + n) % NW != wv || !live(f, n)) continue;
        floatx4_t s = {0.f, 0.f, 0.f, 0.f};
        for (int k0 = 0; k0 < p.ksplit; k0 += 4) {  // up to 4 partials per memory round trip, summed in split order
          const int nk = min(4, p.ksplit - k0);
          u32x4_t v[4];
          ld_agent_x4(nk, part_at(k0, f, n), part_at(min(k0 + 1, p.ksplit - 1), f, n),
                      part_at(min(k0 + 2, p.ksplit - 1), f, n), part_at(min(k0 + 3, p.ksplit - 1), f, n), v[0], v[1],
                      v[2], v[3]);
          for (int j = 0; j < nk; ++j) {
            const floatx4_t x = __builtin_bit_cast(floatx4_t, v[j]);
            s = k0 + j == 0 ? x : s + x;
          }
        }
        epilogue(f, n, s);
      }
    if (tid == 0) reset_counter(&p.tile_ctr[blockIdx.x]);
  }

  if constexpr (POST) {
    // the last column tile to finish normalizes every row (one wavefront per row), then resets the counter
    wait_stores();
    __syncthreads();
    if (tid == 0) last_flag = count_arrival(p.done_ctr) == gridDim.x - 1;
    __syncthreads();
    if (!last_flag) return;
    for (int r = wv; r < p.M; r += NW) post_addnorm_row(p, r, lane);
    if (tid == 0) reset_counter(p.done_ctr);
  }
}

// Persistent variant for shapes with many column tiles and one load pass per tile (every wave's k-steps fit one
// unrolled pass): gridDim.x workgroups (about one per CU) walk the column tiles t = blockIdx.x, + gridDim.x, ...
// The activations of a wave's k-steps are loaded once and reused for every tile; the next tile's weights are
// loaded into the other register set before the current tile's MFMAs, reduction and epilogue, so a workgroup keeps
// its weight stream in flight across tiles. The k partition over the waves and the wave-order reduction are those
// of gemm_kernel, so both produce the same bits for the same shape and every row count. With PRO_ADDNORM the
// workgroup first issues its first tile's weight loads, then builds the normalized activation rows in LDS (the
// arithmetic of gss_add_rmsnorm, as in gemm_kernel's prologue) while they are in flight.
//
// A workgroup with at most FEW_TILES 16-feature tiles (FEW: FT == 1 without the prologue, when the host sized the
// partials for it) issues every tile's weights at once, runs all their MFMAs, and reduces and finishes all its
// tiles after one barrier: its compute is small next to a memory round trip, so one wait and one reduction beat a
// chain of them (gate_up 9216 x 1536 at 17 rows: 10.4 -> 9.8 us per call; staging the activations through LDS on
// top of it gained nothing).
constexpr int FEW_TILES = 3;

template <int FT, int NT, int UNR, int EPI, int PRO = PRO_NONE, int E = 8>
__global__ void __launch_bounds__(64 * MAX_NW) gemm_stream_kernel(GemmParams p, int ksw, int n_tiles, int few) {
  // LDS: [FEW_TILES or 1][NW][FT][NT][64] wave partials, then (PRO_ADDNORM) x rows [M][Kd + XPAD]
  extern __shared__ floatx4_t red[];
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6, NW = blockDim.x >> 6;
  const int l16 = lane & 15, g4 = lane >> 4;
  const int ksteps = p.Kd / 32;
  const int s_beg = wv * ksw, s_end = min(ksteps, s_beg + ksw);  // ksw <= UNR: one pass
  constexpr bool FEW = FT == 1 && PRO == PRO_NONE;
  const int red_sets = FEW && few ? FEW_TILES : 1;

  // Every load below is unconditional (clamped indices), so the compiler can count the loads in flight and wait
  // only for the older register set: activation rows past M read row 0 (their outputs are never stored), k-steps
  // past the wave's range read its last k-step and are skipped at the MFMA.
  u32x4_t xb[UNR][NT];  // this wave's activation fragments, filled once below (after the first weight loads)
  auto load_w = [&](int t, u32x4_t(&wa)[UNR][FT]) {
#pragma unroll
    for (int f = 0; f < FT; ++f) {
      const int row = min(t * FT * 16 + f * 16 + l16, p.N - 1);  // rows past N repeat the last (never stored)
      const uint16_t* wr = p.w + static_cast<int64_t>(row) * p.ldw + g4 * 8;
#pragma unroll
      for (int u = 0; u < UNR; ++u) wa[u][f] = *reinterpret_cast<const u32x4_t*>(wr + min(s_beg + u, ksteps - 1) * 32);
    }
  };
  auto mfma_tile = [&](const u32x4_t(&wa)[UNR][FT], floatx4_t(&acc)[FT][NT]) {
#pragma unroll
    for (int f = 0; f < FT; ++f)
#pragma unroll
      for (int n = 0; n < NT; ++n) acc[f][n] = floatx4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int u = 0; u < UNR; ++u) {
      if (s_beg + u < s_end) {  // wave-uniform
#pragma unroll
        for (int f = 0; f < FT; ++f)
#pragma unroll
          for (int n = 0; n < NT; ++n)
            acc[f][n] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, wa[u][f]),
                                                                __builtin_bit_cast(bf16x8_t, xb[u][n]), acc[f][n], 0,
                                                                0, 0);
      }
    }
  };
  // partials of tile t (in set `set` of the partial area) -> LDS; then its reduction in wave order and epilogue
  auto post = [&](int set, const floatx4_t(&acc)[FT][NT]) {
#pragma unroll
    for (int f = 0; f < FT; ++f)
#pragma unroll
      for (int n = 0; n < NT; ++n) red[(((set * NW + wv) * FT + f) * NT + n) * 64 + lane] = acc[f][n];
  };
  auto finish = [&](int set, int t) {
    const int f0 = t * FT * 16;
#pragma unroll
    for (int f = 0; f < FT; ++f)
#pragma unroll
      for (int n = 0; n < NT; ++n) {
        if (((set * FT + f) * NT + n) % NW != wv || n * 16 + l16 >= p.M || f0 + f * 16 + g4 * 4 >= p.N) continue;
        floatx4_t s = red[(((set * NW + 0) * FT + f) * NT + n) * 64 + lane];
        for (int v = 1; v < NW; ++v) s += red[(((set * NW + v) * FT + f) * NT + n) * 64 + lane];
        gemm_epilogue<EPI, false>(p, f0, 0, f, n, s, l16, g4);
      }
  };
  auto tile = [&](int t, const u32x4_t(&wa)[UNR][FT]) {
    floatx4_t acc[FT][NT];
    mfma_tile(wa, acc);
    __syncthreads();  // the previous tile's partials have been read
    post(0, acc);
    __syncthreads();
    finish(0, t);
  };
  const int G = gridDim.x;
  const int n_my = (n_tiles - static_cast<int>(blockIdx.x) + G - 1) / G;  // tiles of this workgroup (>= 1)
  auto tile_at = [&](int i) { return static_cast<int>(blockIdx.x) + i * G; };
  u32x4_t wa[UNR][FT], wb[UNR][FT], wc[UNR][FT];  // wc: the few-tile path's third tile
  uint16_t* xs = reinterpret_cast<uint16_t*>(red + red_sets * NW * FT * NT * 64);
  // the arguments of the weight loads and of the prologue in one scalar batch (read where first used, the
  // prologue's came in two more dependent round trips after the weight loads)
  if constexpr (PRO == PRO_ADDNORM)
    asm volatile("" ::"s"(p.w), "s"(p.ldw), "s"(p.N), "s"(p.Kd), "s"(p.M), "s"(p.h_in), "s"(p.w_next),
                 "s"(p.pa_parts), "s"(p.n_parts), "s"(p.pa), "s"(p.w_post), "s"(p.eps), "s"(p.h_out));
  load_w(tile_at(0), wa);
  if constexpr (PRO == PRO_ADDNORM) {
    // the normalized rows, one wavefront per row, into LDS; workgroup 0 also stores the updated residual
    for (int r = wv; r < p.M; r += NW) addnorm_row<E>(p, r, lane, xs, blockIdx.x == 0 && p.h_out != nullptr);
    __syncthreads();
#pragma unroll
    for (int n = 0; n < NT; ++n) {
      const int r = n * 16 + l16;
#pragma unroll
      for (int u = 0; u < UNR; ++u)
        xb[u][n] = *reinterpret_cast<const u32x4_t*>(xs + (r < p.M ? r : 0) * (p.Kd + XPAD) +
                                                     min(s_beg + u, ksteps - 1) * 32 + g4 * 8);
    }
  } else {
#pragma unroll
    for (int n = 0; n < NT; ++n) {
      const int r = n * 16 + l16;
      const uint16_t* xr = p.x + static_cast<int64_t>(r < p.M ? r : 0) * p.ldx + g4 * 8;
#pragma unroll
      for (int u = 0; u < UNR; ++u)
        xb[u][n] = *reinterpret_cast<const u32x4_t*>(xr + min(s_beg + u, ksteps - 1) * 32);
    }
  }
  if constexpr (FEW) {
    if (few) {  // n_my <= FEW_TILES: all weights in flight, all MFMAs, one reduction
      if (n_my > 1) load_w(tile_at(1), wb);
      if (n_my > 2) load_w(tile_at(2), wc);
      floatx4_t acc[FT][NT];
      mfma_tile(wa, acc);
      post(0, acc);
      if (n_my > 1) {
        mfma_tile(wb, acc);
        post(1, acc);
      }
      if (n_my > 2) {
        mfma_tile(wc, acc);
        post(2, acc);
      }
      __syncthreads();
      for (int i = 0; i < n_my; ++i) finish(i, tile_at(i));
      return;
    }
  }
  // Two register sets, alternating: while one tile is computed, the next one's weights stream into the other set.
  // The steady state (two tiles per iteration) always has a next tile, so its loads are issued unconditionally and
  // the compiler counts the loads in flight.
  int i = 0;
  for (; i + 2 < n_my; i += 2) {
    load_w(tile_at(i + 1), wb);
    tile(tile_at(i), wa);
    load_w(tile_at(i + 2), wa);
    tile(tile_at(i + 1), wb);
  }
  if (i + 1 < n_my) {
    load_w(tile_at(i + 1), wb);
    tile(tile_at(i), wa);
    tile(tile_at(i + 1), wb);
  } else {
    tile(tile_at(i), wa);
  }
}

// Launch shape: the most k splits over workgroups of a plain GEMM (1 = none). Like every other launch-shape choice
// it is a function of the weight shape (and the device's CU count) only: it fixes the reduction order, so it is a
// constant, never a setting that could differ between two calls on the same weights.
constexpr int MAX_KSPLIT = 2;
constexpr int MAX_ROWS = 65536;  // rows of one call
constexpr bool kStageX = true;  // stage the activations through LDS where it applies (gemm_kernel)

// Dynamic LDS beyond the default 64 KB for kernel K (once per process, before its first launch).
template <auto K>
bool allow_full_lds() {
  static const bool ok = hipFuncSetAttribute(reinterpret_cast<const void*>(K),
                                             hipFuncAttributeMaxDynamicSharedMemorySize, MAX_DYN_LDS) == hipSuccess;
  return ok;
}

// workgroups of the persistent kernel: one per CU of the current device (queried once)
int stream_wgs() {
  static int cus = 0;
  if (cus == 0) {
    int dev = 0, n = 0;
    if (hipGetDevice(&dev) != hipSuccess || hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) !=
                                                hipSuccess || n <= 0)
      n = 256;
    cus = n;
  }
  return cus;
}

// Workspace: per-column-tile counters and the post-norm counter at a fixed offset (so calls of every shape share one
// workspace), then the split-K partials.
constexpr int CTR_TILES = 8192;
constexpr size_t CTR_BYTES = (CTR_TILES + 64) * sizeof(uint32_t);

// k splits of a (N, Kd) shape: more workgroups (up to ~384) when the column tiles alone leave CUs idle and every
// split keeps at least 64 k-steps; below that the split's handoff (partials through the coherence point and a
// counter) costs more than the extra streaming width buys. A function of the weight shape only, so every M runs the
// same reduction order. For the 1536-hidden decoder: down (Kd 4608) splits in 2, the other projections do not.
int gemm_ksplit(int n_tiles, int ksteps) {
  int ks = max(1, min(MAX_KSPLIT, 384 / max(1, n_tiles)));
  return max(1, min(ks, ksteps / 64));
}

// features per workgroup / 16: 1 unless that makes more than ~8 workgroups per CU (the LM head)
int gemm_ft(int N) { return N / 16 <= 2048 ? 1 : 2; }

// k splits of the partial-sum output (EPI_PARTS): up to 2, as many as keep the column tiles x splits within one
// workgroup per CU, each split at least 4 k-steps. A function of the weight shape only (the reduction order).
int gemm_parts_split(int n_tiles, int ksteps) {
  const int ks = max(1, min(2, stream_wgs() / max(1, n_tiles)));
  return ksteps / ks >= 4 ? ks : 1;
}

// The partials serve the skinny kernel (M <= 64); the tiled kernel folds its splits in registers, so a workspace
// sized for 64 rows serves every larger M.
size_t gemm_ws_bytes(int M, int N, int Kd) {
  const int ft = gemm_ft(N), n_tiles = (N + ft * 16 - 1) / (ft * 16);
  const int ks = gemm_ksplit(n_tiles, Kd / 32);
  return CTR_BYTES + (ks > 1 ? static_cast<size_t>(ks) * min(M, 64) * N * sizeof(float) : 0);
}

// ---- batched windows (M > 64): a tiled kernel with gemm_kernel's arithmetic ---------------------------------------
// Each output element of gemm_kernel is, for every k split ks (in order), the left fold over the waves v = 0..nw-1 of
// P_v = the MFMA chain (v_mfma_f32_16x16x32_bf16, weights as A, activations as B, accumulating from zero) over the
// k-steps [ks*kps + v*ksw, ks*kps + (v+1)*ksw) clipped to the split; the splits are then written as parts or
// folded in split order. This kernel computes exactly that sequence of operations per element, but with a GEMM
// tiling: a workgroup owns a BF-feature x BM-row block, its GF x GM waves a WF x WN grid of 16x16 tiles each, and
// every wave walks all k-steps of the split itself, restarting its accumulator P at each wave-range boundary (ksw
// k-steps, a multiple of the LDS chunk) and folding it into S. Weights and activations stream through a ring of NB
// LDS buffers of TKC k-steps each (direct-to-LDS loads from a scalar base plus precomputed per-lane offsets, issued
// NB - 1 chunks ahead; a wave waits only for its loads of the chunk it is about to read, the later chunks stay in
// flight), rows XOR-swizzled by 16-byte chunk so the 16 rows of a fragment read hit distinct banks; the next k-step's
// fragments are read while the current one's MFMAs run. Every weight byte is read once per row block instead of once
// per 64 rows, and every activation byte once per feature block.
GSS_DEV void dma16_lds(const void* g, const void* lds) {
  const uint32_t la = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(reinterpret_cast<uintptr_t>(lds)));
  asm volatile("global_load_lds_dwordx4 %0, off" ::"v"(g), "{m0}"(la) : "memory");
}

// the same load from a wave-uniform base (in SGPRs) plus a 32-bit per-lane byte offset: no 64-bit address math per lane
GSS_DEV void dma16_lds_s(const void* sbase, uint32_t voff, const void* lds) {
  const uint32_t la = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(reinterpret_cast<uintptr_t>(lds)));
  asm volatile("global_load_lds_dwordx4 %0, %1" ::"v"(voff), "s"(sbase), "{m0}"(la) : "memory");
}

// s_waitcnt on the vector-memory counter alone (at most N of this wave's loads still in flight)
template <int N>
GSS_DEV void wait_vm() {
  static_assert(N >= 0 && N < 64, "vmcnt has 6 bits");
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

template <int EPI, int GF, int GM, int WF, int WN, int TKC, int NB, bool MULTI>
__global__ void __launch_bounds__(64 * GF * GM) gemm_tiled_kernel(GemmParams p, int ksw) {
  static_assert(4 % TKC == 0 && NB >= 2 && NB <= 4, "chunks divide the 4-k-step wave-range unit; ring of 2..4");
  constexpr int NW = GF * GM;                    // waves: GF along the features x GM along the rows
  constexpr int BF = GF * WF * 16, BM = GM * WN * 16, ROWS = BF + BM;
  constexpr int CH = TKC * 4;                   // 16-byte chunks per LDS row
  constexpr int PER_WAVE = ROWS * CH / 64 / NW;  // direct-to-LDS instructions per wave per chunk
  static_assert(ROWS * CH % (64 * NW) == 0 && BF * CH % (64 * NW) == 0, "whole instructions, weight rows first");
  extern __shared__ __attribute__((aligned(16))) u32x4_t tl[];  // [NB][ROWS][CH]
  const int tid = threadIdx.x, lane = tid & 63;
  const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wf = wv % GF, wn = wv / GF;
  const int l16 = lane & 15, g4 = lane >> 4;
  const int fb = blockIdx.x * BF, rb = blockIdx.y * BM;
  const int ksteps = p.Kd / 32;
  // splits this workgroup computes: one (EPI_PARTS: blockIdx.z) or all of them, folded in split order
  const int ks_lo = EPI == EPI_PARTS ? static_cast<int>(blockIdx.z) : 0;
  const int ks_hi = EPI == EPI_PARTS ? ks_lo + 1 : p.ksplit;
  // chunk list: split by split, TKC k-steps each from the split's first k-step (the last chunk of a split may be
  // shorter); wave-range boundaries fall on chunk starts because ksw is a multiple of TKC
  auto split_beg = [&](int ks) { return ks * p.kps; };
  auto split_end = [&](int ks) { return min(ksteps, (ks + 1) * p.kps); };
  int n_chunks = 0;
  for (int ks = ks_lo; ks < ks_hi; ++ks) n_chunks += (max(0, split_end(ks) - split_beg(ks)) + TKC - 1) / TKC;
  // a chunk cursor (split, first k-step): past the end of a split it moves to the next split's first k-step
  auto settle = [&](int& kq, int& sq) {
    while (kq < ks_hi && sq >= split_end(kq)) {
      ++kq;
      if (kq < ks_hi) sq = split_beg(kq);
    }
  };

  // per-lane byte offsets of a chunk's loads from the matrix base at the chunk's first k-step (row * ld + the lane's
  // 16 bytes of the row's TKC k-steps); instruction j < JW loads weight rows, the rest activation rows. Rows past
  // N or M repeat the last one (their results are never stored).
  constexpr int JW = BF * CH / (64 * NW);
  uint32_t off[PER_WAVE];
#pragma unroll
  for (int j = 0; j < PER_WAVE; ++j) {
    const int slot = (j * NW + wv) * 64 + lane;  // slot of this lane's 16 bytes in the chunk's LDS image
    const int r = slot / CH, cp = slot % CH;    // LDS row, physical chunk
    const int c = cp ^ (r & (CH - 1));          // the logical chunk stored there: k-step c / 4, 8 elements c % 4
    const int64_t row = j < JW ? min(fb + r, p.N - 1) : min(rb + r - BF, p.M - 1);
    off[j] = static_cast<uint32_t>(row * (j < JW ? p.ldw : p.ldx) * 2 + (c / 4) * 64 + (c % 4) * 16);
  }
  auto issue = [&](int ks, int s0, int buf) {
    const int kend = split_end(ks);
    u32x4_t* base = tl + buf * ROWS * CH;
    if (s0 + TKC <= kend) {  // a full chunk: scalar base + the per-lane offsets
      const char* bw = reinterpret_cast<const char*>(p.w) + s0 * 64;
      const char* bx = reinterpret_cast<const char*>(p.x) + s0 * 64;
#pragma unroll
      for (int j = 0; j < PER_WAVE; ++j) dma16_lds_s(j < JW ? bw : bx, off[j], base + (j * NW + wv) * 64);
      return;
    }
    // the last, shorter chunk of a split: k-steps past the split repeat its last one (never used)
#pragma unroll
    for (int j = 0; j < PER_WAVE; ++j) {
      const int slot = (j * NW + wv) * 64 + lane;
      const int r = slot / CH, cp = slot % CH;
      const int c = cp ^ (r & (CH - 1));
      const int s = min(s0 + c / 4, kend - 1);
      const uint16_t* src;
      if (r < BF) {
        const int f = min(fb + r, p.N - 1);
        src = p.w + static_cast<int64_t>(f) * p.ldw + s * 32 + (c % 4) * 8;
      } else {
        const int m = min(rb + r - BF, p.M - 1);
        src = p.x + static_cast<int64_t>(m) * p.ldx + s * 32 + (c % 4) * 8;
      }
      dma16_lds(src, base + (j * NW + wv) * 64);
    }
  };

  // P: the running range's MFMA chain (restarted by an MFMA on a zero C operand at every range start); S: the
  // split's fold over the ranges; T: the fold over the splits (MULTI only). S and T start at -0.0, so the first
  // fold S = -0.0 + P_0 is P_0 exactly (also for a zero of either sign) and no fold needs a select.
  const floatx4_t nz = {-0.f, -0.f, -0.f, -0.f}, z4 = {0.f, 0.f, 0.f, 0.f};
  floatx4_t P[WF][WN], S[WF][WN], T[WF][WN];
#pragma unroll
  for (int f = 0; f < WF; ++f)
#pragma unroll
    for (int n = 0; n < WN; ++n) {
      P[f][n] = z4;
      S[f][n] = nz;
      if constexpr (MULTI) T[f][n] = nz;
    }
  const int fr0 = wf * WF * 16 + l16;          // this lane's A row (feature) in the block, tile 0
  const int mr0 = BF + wn * WN * 16 + l16;     // its B row (activation) in the LDS image, tile 0
  const int sw = l16 & (CH - 1);               // the swizzle of both (rows = l16 mod 16)

  // the ring: chunks 0 .. NB-2 in flight before the loop, then one more per iteration
  int ki = ks_lo, si = split_beg(ks_lo), issued = 0;
  settle(ki, si);
#pragma unroll
  for (int q = 0; q < NB - 1; ++q)
    if (issued < n_chunks) {
      issue(ki, si, issued % NB);
      ++issued;
      si += TKC;
      settle(ki, si);
    }
  int ks = ks_lo, s0 = split_beg(ks_lo), v_done = 0;  // compute cursor, ranges folded into S
  settle(ks, s0);
  for (int i = 0; i < n_chunks; ++i) {
    // chunk i has landed once at most (issued - 1 - i) later chunks of this wave are in flight
    switch (issued - 1 - i) {
      case 0: wait_vm<0>(); break;
      case 1: wait_vm<(NB > 2 ? PER_WAVE : 0)>(); break;
      default: wait_vm<(NB > 3 ? 2 * PER_WAVE : 0)>(); break;
    }
    __syncthreads();  // every wave's loads of chunk i landed; every wave is done reading chunk i - 1's buffer
    if (issued < n_chunks) {  // into the buffer chunk i - 1 used
      issue(ki, si, issued % NB);
      ++issued;
      si += TKC;
      settle(ki, si);
    }
    const int kb = split_beg(ks), kend = split_end(ks), nk = min(TKC, kend - s0);
    // a range starts at this chunk (ksw is a multiple of TKC): fold the finished one (none at the split's start)
    const bool restart = (s0 - kb) % ksw == 0;
    if (restart && s0 != kb) {
#pragma unroll
      for (int f = 0; f < WF; ++f)
#pragma unroll
        for (int n = 0; n < WN; ++n) S[f][n] = S[f][n] + P[f][n];
      ++v_done;
    }
    const u32x4_t* buf = tl + (i % NB) * ROWS * CH;
    bf16x8_t a[2][WF], b[2][WN];  // fragments of k-step u in set u & 1; k-step u + 1 is read during u's MFMAs
    auto read = [&](int u, bf16x8_t(&af)[WF], bf16x8_t(&bf)[WN]) {
#pragma unroll
      for (int f = 0; f < WF; ++f)
        af[f] = __builtin_bit_cast(bf16x8_t, buf[(fr0 + f * 16) * CH + ((u * 4 + g4) ^ sw)]);
#pragma unroll
      for (int n = 0; n < WN; ++n)
        bf[n] = __builtin_bit_cast(bf16x8_t, buf[(mr0 + n * 16) * CH + ((u * 4 + g4) ^ sw)]);
    };
    read(0, a[0], b[0]);
#pragma unroll
    for (int u = 0; u < TKC; ++u) {
      if (u < nk) {  // workgroup-uniform
        if (u + 1 < nk) read(u + 1, a[(u + 1) & 1], b[(u + 1) & 1]);
        if (u == 0 && restart) {
#pragma unroll
          for (int f = 0; f < WF; ++f)
#pragma unroll
            for (int n = 0; n < WN; ++n)
              P[f][n] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[0][f], b[0][n], z4, 0, 0, 0);
        } else {
#pragma unroll
          for (int f = 0; f < WF; ++f)
#pragma unroll
            for (int n = 0; n < WN; ++n)
              P[f][n] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[u & 1][f], b[u & 1][n], P[f][n], 0, 0, 0);
        }
      }
    }
    if (s0 + TKC >= kend) {
      // the split's last chunk: fold the last range, then the empty ones of gemm_kernel's last split (+0.0 each:
      // only the sign of a zero can change), then the split's sum
      const int nw = (p.kps + ksw - 1) / ksw;
#pragma unroll
      for (int f = 0; f < WF; ++f)
#pragma unroll
        for (int n = 0; n < WN; ++n) {
          S[f][n] = S[f][n] + P[f][n];
          if (v_done + 1 < nw) S[f][n] = S[f][n] + z4;
        }
      if constexpr (EPI == EPI_PARTS) {
#pragma unroll
        for (int f = 0; f < WF; ++f)
#pragma unroll
          for (int n = 0; n < WN; ++n) {
            const int row = rb + wn * WN * 16 + n * 16 + l16, feat = fb + wf * WF * 16 + f * 16 + g4 * 4;
            if (row < p.M && feat < p.N)
              *reinterpret_cast<floatx4_t*>(static_cast<float*>(p.y) +
                                            (static_cast<int64_t>(ks) * p.M + row) * p.ldy + feat) = S[f][n];
          }
      } else if constexpr (MULTI) {
#pragma unroll
        for (int f = 0; f < WF; ++f)
#pragma unroll
          for (int n = 0; n < WN; ++n) {
            T[f][n] = T[f][n] + S[f][n];
            S[f][n] = nz;
          }
      }
      v_done = 0;
    }
    s0 += TKC;
    settle(ks, s0);
  }
  if constexpr (EPI != EPI_PARTS) {
#pragma unroll
    for (int f = 0; f < WF; ++f)
#pragma unroll
      for (int n = 0; n < WN; ++n) {
        const int row = rb + wn * WN * 16 + n * 16 + l16, feat = fb + wf * WF * 16 + f * 16 + g4 * 4;
        if (row < p.M && feat < p.N)
          gemm_epilogue<EPI, false>(p, fb + wf * WF * 16, rb + wn * WN * 16, f, n, MULTI ? T[f][n] : S[f][n], l16,
                                    g4);
      }
  }
}

template <int EPI, int GF, int GM, int WF, int WN, int TKC, int NB, bool MULTI>
int launch_tiled_k(GemmParams& p, int ksw, hipStream_t st) {
  constexpr int BF = GF * WF * 16, BM = GM * WN * 16;
  constexpr size_t lds = static_cast<size_t>(NB) * (BF + BM) * TKC * 4 * sizeof(u32x4_t);
  constexpr auto kern = gemm_tiled_kernel<EPI, GF, GM, WF, WN, TKC, NB, MULTI>;
  if constexpr (lds > 64 * 1024) {
    if (!allow_full_lds<kern>()) return GSS_ERR_LAUNCH;
  }
  const dim3 grid((p.N + BF - 1) / BF, (p.M + BM - 1) / BM, EPI == EPI_PARTS ? p.ksplit : 1);
  hipLaunchKernelGGL(kern, grid, dim3(64 * GF * GM), lds, st, p, ksw);
  return gss_launch_status();
}

// several splits folded in the kernel (not EPI_PARTS, which writes each split) take the variant with T
template <int EPI, int GF, int GM, int WF, int WN, int TKC, int NB>
int launch_tiled_cfg(GemmParams& p, int ksw, hipStream_t st) {
  if (EPI != EPI_PARTS && p.ksplit > 1) return launch_tiled_k<EPI, GF, GM, WF, WN, TKC, NB, true>(p, ksw, st);
  return launch_tiled_k<EPI, GF, GM, WF, WN, TKC, NB, false>(p, ksw, st);
}

// The tiled kernel for M > 64, by how many blocks each tiling makes (any tiling computes the same bits; only the
// speed depends on it): 256 x 128 blocks of 8 waves (64 x 64 per wave, two waves per SIMD, a 3-deep ring of
// 2-k-step chunks) when they give about two thirds of the CUs a workgroup (not with several splits folded in the
// kernel: the extra accumulators would spill), else 128 x 128 blocks of 8 waves (32 x 64 per wave) by the same
// rule, else 64 x 64 blocks of 4 waves (two workgroups per CU). Measured on the decoder's shapes: the 256 x 128
// blocks run the 8192-row gate_up (9216 x 1536) at 340 us against 480 us for 128 x 128 blocks of 4 waves; at 544
// rows gate_up takes 36 us on 256 x 128 blocks (180 workgroups) against 43 us on 128 x 128 (360); at 288 rows 23 us
// on 128 x 128 (216) against 28 us on 64 x 64; at 1056 rows qkv / o_proj / down_proj take 28 / 18 / 31 us on
// 128 x 128 against 32 / 23 / 40 us on 64 x 64, while qkv at 544 rows stays faster on 64 x 64 (360 workgroups) than
// on 128 x 128 (100): 19.6 against 28 us. p.ksplit / p.kps / the wave range ksw are gemm_kernel's for the same
// (N, Kd).
template <int EPI>
int launch_tiled(GemmParams& p, int ksw, hipStream_t st) {
  const int z = EPI == EPI_PARTS ? p.ksplit : 1;
  const bool multi = EPI != EPI_PARTS && p.ksplit > 1;
  auto blocks = [&](int bf, int bm) { return static_cast<int64_t>((p.N + bf - 1) / bf) * ((p.M + bm - 1) / bm) * z; };
  // the largest block that still gives about two thirds of the CUs a workgroup (bigger blocks reuse each LDS byte
  // for more MFMAs; below that, idle CUs cost more than the reuse gains)
  const int64_t enough = (2 * stream_wgs() + 2) / 3;
  if (!multi && blocks(256, 128) >= enough) return launch_tiled_k<EPI, 4, 2, 4, 4, 2, 3, false>(p, ksw, st);
  if (blocks(128, 128) >= enough) return launch_tiled_cfg<EPI, 4, 2, 2, 4, 4, 2>(p, ksw, st);
  return launch_tiled_cfg<EPI, 2, 2, 2, 2, 4, 2>(p, ksw, st);
}

template <int FT, int NT, int EPI, int PRO, bool POST>
int launch_ft_nt(GemmParams& p, void* ws, size_t ws_bytes, hipStream_t st) {
  const int ksteps = p.Kd / 32;
  const int n_tiles = (p.N + FT * 16 - 1) / (FT * 16);
  p.ksplit = EPI == EPI_PARTS ? gemm_parts_split(n_tiles, ksteps) : gemm_ksplit(n_tiles, ksteps);
  p.kps = (ksteps + p.ksplit - 1) / p.ksplit;
  const int Mw = p.M;  // rows of one workgroup (M <= 64 here)
  if ((p.ksplit > 1 && EPI != EPI_PARTS) || POST) {
    if (n_tiles > CTR_TILES) return GSS_ERR_UNSUPPORTED;
    const size_t need = CTR_BYTES + (p.ksplit > 1 ? static_cast<size_t>(p.ksplit) * p.M * p.N * sizeof(float) : 0);
    if (!ws || ws_bytes < need) return GSS_ERR_WORKSPACE;
    p.tile_ctr = static_cast<uint32_t*>(ws);
    p.done_ctr = p.tile_ctr + CTR_TILES;
    p.part = reinterpret_cast<float*>(static_cast<char*>(ws) + CTR_BYTES);
  }
  // k-steps per wave: the fewest that cover a split with at most MAX_NW waves (rounded to a multiple of 4)
  int ksw = (p.kps + MAX_NW - 1) / MAX_NW;
  ksw = (ksw + 3) / 4 * 4;
  const int nw = (p.kps + ksw - 1) / ksw;
  const dim3 grid(n_tiles, p.ksplit), block(64 * nw);
  size_t lds = static_cast<size_t>(nw) * FT * NT * 64 * sizeof(floatx4_t);
  if constexpr (PRO == PRO_ADDNORM) {
    lds += static_cast<size_t>(p.M) * (p.Kd + XPAD) * sizeof(uint16_t);
    if (ksw > 4) return GSS_ERR_UNSUPPORTED;  // one pass of 4 k-steps per wave: Kd <= 32 * 4 * MAX_NW
    if (lds > MAX_LDS) return GSS_ERR_UNSUPPORTED;
    const int G = stream_wgs();
    if (p.ksplit == 1 && n_tiles > G) {  // the persistent kernel (same rule as without the prologue)
      switch (p.Kd / 64) {
        case 4: hipLaunchKernelGGL((gemm_stream_kernel<FT, NT, 4, EPI, PRO, 4>), dim3(G), block, lds, st, p, ksw, n_tiles, 0); break;
        case 8: hipLaunchKernelGGL((gemm_stream_kernel<FT, NT, 4, EPI, PRO, 8>), dim3(G), block, lds, st, p, ksw, n_tiles, 0); break;
        case 16: hipLaunchKernelGGL((gemm_stream_kernel<FT, NT, 4, EPI, PRO, 16>), dim3(G), block, lds, st, p, ksw, n_tiles, 0); break;
        case 24: hipLaunchKernelGGL((gemm_stream_kernel<FT, NT, 4, EPI, PRO, 24>), dim3(G), block, lds, st, p, ksw, n_tiles, 0); break;
        default: return GSS_ERR_UNSUPPORTED;
      }
      return gss_launch_status();
    }
    switch (p.Kd / 64) {
      case 4: hipLaunchKernelGGL((gemm_kernel<FT, NT, 4, EPI, PRO, 4>), grid, block, lds, st, p, ksw); break;
      case 8: hipLaunchKernelGGL((gemm_kernel<FT, NT, 4, EPI, PRO, 8>), grid, block, lds, st, p, ksw); break;
      case 16: hipLaunchKernelGGL((gemm_kernel<FT, NT, 4, EPI, PRO, 16>), grid, block, lds, st, p, ksw); break;
      case 24: hipLaunchKernelGGL((gemm_kernel<FT, NT, 4, EPI, PRO, 24>), grid, block, lds, st, p, ksw); break;
      default: return GSS_ERR_UNSUPPORTED;
    }
    return gss_launch_status();
  } else {
    if constexpr (!POST) {
      // more column tiles than CUs and one load pass per tile (a function of N and Kd only, so every row count
      // takes the same kernel): the persistent kernel, one workgroup per CU walking the tiles
      const int G = stream_wgs();
      if (EPI != EPI_PARTS && p.ksplit == 1 && ksw <= 4 && n_tiles > G) {
        // every workgroup has at most FEW_TILES tiles: partials for all of them (FT = 1: up to 3 x 12 x 4 KB)
        const int few = FT == 1 && n_tiles <= FEW_TILES * G && lds * FEW_TILES <= MAX_DYN_LDS;
        constexpr auto k0 = gemm_stream_kernel<FT, NT, 4, EPI>;
        if (!allow_full_lds<k0>()) return GSS_ERR_LAUNCH;
        hipLaunchKernelGGL(k0, dim3(G), block, lds * (few ? FEW_TILES : 1), st, p, ksw, n_tiles, few);
        return gss_launch_status();
      }
    }
    // activations staged in LDS when a wave's k-range is one pass and the rows fit (same arithmetic either way)
    const size_t lds_xs = lds + static_cast<size_t>(nw) * Mw * ksw * 64;
    // (the staged rows are addressed by 32-bit byte offsets from the first)
    const bool xs = kStageX && lds_xs <= MAX_DYN_LDS && static_cast<int64_t>(p.M) * p.ldx * 2 < (int64_t{1} << 31);
    if constexpr (FT + NT <= 3) {
      if (ksw % 8 == 0) {
        constexpr auto kx = gemm_kernel<FT, NT, 8, EPI, PRO_NONE, 8, POST, true>;
        if (xs && ksw == 8) {
          if (!allow_full_lds<kx>()) return GSS_ERR_LAUNCH;
          hipLaunchKernelGGL(kx, grid, block, lds_xs, st, p, ksw);
        } else {
          hipLaunchKernelGGL((gemm_kernel<FT, NT, 8, EPI, PRO_NONE, 8, POST>), grid, block, lds, st, p, ksw);
        }
        return gss_launch_status();
      }
    }
    constexpr auto kx4 = gemm_kernel<FT, NT, 4, EPI, PRO_NONE, 8, POST, true>;
    if (xs && ksw == 4) {
      if (!allow_full_lds<kx4>()) return GSS_ERR_LAUNCH;
      hipLaunchKernelGGL(kx4, grid, block, lds_xs, st, p, ksw);
    } else {
      hipLaunchKernelGGL((gemm_kernel<FT, NT, 4, EPI, PRO_NONE, 8, POST>), grid, block, lds, st, p, ksw);
    }
    return gss_launch_status();
  }
}

template <int EPI, int PRO, bool POST>
int launch_epi(GemmParams& p, void* ws, size_t ws_bytes, hipStream_t st) {
  if (p.M > 64) {
    // batched windows: the tiled kernel with the same k partition (splits and wave ranges of gemm_kernel for this
    // (N, Kd)); the fused prologue and post-norm need every row in one workgroup, so they stay at M <= 64
    if constexpr (PRO != PRO_NONE || POST) {
      return GSS_ERR_UNSUPPORTED;
    } else {
      const int ft = gemm_ft(p.N), ksteps = p.Kd / 32;
      const int n_tiles = (p.N + ft * 16 - 1) / (ft * 16);
      p.ksplit = EPI == EPI_PARTS ? gemm_parts_split(n_tiles, ksteps) : gemm_ksplit(n_tiles, ksteps);
      p.kps = (ksteps + p.ksplit - 1) / p.ksplit;
      int ksw = (p.kps + MAX_NW - 1) / MAX_NW;
      ksw = (ksw + 3) / 4 * 4;
      // the kernel addresses rows by 32-bit byte offsets from the matrix bases
      if ((static_cast<int64_t>(p.N) - 1) * p.ldw * 2 + p.Kd * 2 >= (int64_t{1} << 32) ||
          (static_cast<int64_t>(p.M) - 1) * p.ldx * 2 + p.Kd * 2 >= (int64_t{1} << 32))
        return GSS_ERR_UNSUPPORTED;
      return launch_tiled<EPI>(p, ksw, st);
    }
  }
  const int NT = (p.M + 15) / 16;
  // 16 features per workgroup unless that makes more than ~8 workgroups per CU (the LM head)
  if (gemm_ft(p.N) == 1) {
    switch (NT) {
      case 1: return launch_ft_nt<1, 1, EPI, PRO, POST>(p, ws, ws_bytes, st);
      case 2: return launch_ft_nt<1, 2, EPI, PRO, POST>(p, ws, ws_bytes, st);
      case 3: return launch_ft_nt<1, 3, EPI, PRO, POST>(p, ws, ws_bytes, st);
      default: return launch_ft_nt<1, 4, EPI, PRO, POST>(p, ws, ws_bytes, st);
    }
  }
  if constexpr (POST) {
    return GSS_ERR_UNSUPPORTED;  // the post-norm runs on hidden-size outputs only
  } else {
    switch (NT) {
      case 1: return launch_ft_nt<2, 1, EPI, PRO, false>(p, ws, ws_bytes, st);
      case 2: return launch_ft_nt<2, 2, EPI, PRO, false>(p, ws, ws_bytes, st);
      case 3: return launch_ft_nt<2, 3, EPI, PRO, false>(p, ws, ws_bytes, st);
      default: return launch_ft_nt<2, 4, EPI, PRO, false>(p, ws, ws_bytes, st);
    }
  }
}

int gemm_entry(GemmParams& p, int epi, void* ws, size_t ws_bytes, hipStream_t st) {
  const bool pro = p.h_in != nullptr, post = p.post_h != nullptr;
  if ((!pro && !p.x) || !p.w || p.M <= 0 || p.N <= 0 || p.Kd <= 0) return GSS_ERR_ARG;
  if (p.M > MAX_ROWS || p.Kd % 32 != 0 || p.N % 16 != 0) return GSS_ERR_UNSUPPORTED;
  if (p.ldw < p.Kd || (p.ldw % 8) || (!pro && (p.ldx < p.Kd || (p.ldx % 8)))) return GSS_ERR_ARG;
  if ((reinterpret_cast<uintptr_t>(p.x) | reinterpret_cast<uintptr_t>(p.w)) & 15u) return GSS_ERR_ARG;
  if (post) {
    if (pro || epi != EPI_PLAIN || p.out_f32 || p.ldy != p.N) return GSS_ERR_ARG;
    if (!p.post_wp || !p.post_wn || !p.post_x || p.post_x == p.post_h) return GSS_ERR_ARG;
    if (p.N % 512 != 0 || p.N / 64 > POST_MAX_E) return GSS_ERR_UNSUPPORTED;  // 8-element chunks per lane
    if ((reinterpret_cast<uintptr_t>(p.y) | reinterpret_cast<uintptr_t>(p.post_h) |
         reinterpret_cast<uintptr_t>(p.post_x) | reinterpret_cast<uintptr_t>(p.post_wp) |
         reinterpret_cast<uintptr_t>(p.post_wn)) & 15u)
      return GSS_ERR_ARG;
    return launch_epi<EPI_PLAIN, PRO_NONE, true>(p, ws, ws_bytes, st);
  }
  if (pro) {
    if (!p.w_next || (p.pa && !p.w_post) || p.h_out == p.h_in) return GSS_ERR_ARG;
    if (p.pa_parts && (p.pa || !p.w_post || p.n_parts < 1 || (reinterpret_cast<uintptr_t>(p.pa_parts) & 15u)))
      return GSS_ERR_ARG;
    if (p.Kd % 512 != 0) return GSS_ERR_UNSUPPORTED;  // 8-element chunks per lane
    if ((reinterpret_cast<uintptr_t>(p.h_in) | reinterpret_cast<uintptr_t>(p.pa) |
         reinterpret_cast<uintptr_t>(p.h_out) | reinterpret_cast<uintptr_t>(p.w_next) |
         reinterpret_cast<uintptr_t>(p.w_post)) & 15u)
      return GSS_ERR_ARG;
    switch (epi) {
      case EPI_PLAIN: return launch_epi<EPI_PLAIN, PRO_ADDNORM, false>(p, ws, ws_bytes, st);
      case EPI_SWIGLU: return launch_epi<EPI_SWIGLU, PRO_ADDNORM, false>(p, ws, ws_bytes, st);
      default: return launch_epi<EPI_ROPE, PRO_ADDNORM, false>(p, ws, ws_bytes, st);
    }
  }
  switch (epi) {
    case EPI_PLAIN: return launch_epi<EPI_PLAIN, PRO_NONE, false>(p, ws, ws_bytes, st);
    case EPI_SWIGLU: return launch_epi<EPI_SWIGLU, PRO_NONE, false>(p, ws, ws_bytes, st);
    case EPI_PARTS: return launch_epi<EPI_PARTS, PRO_NONE, false>(p, ws, ws_bytes, st);
    default: return launch_epi<EPI_ROPE, PRO_NONE, false>(p, ws, ws_bytes, st);
  }
}

// Fill the prologue fields of a GemmParams from the C descriptor (x comes from the prologue when h_in is set).
void set_prologue(GemmParams& p, const gss_norm_prologue* pro) {
  if (pro == nullptr) return;
  p.pa = static_cast<const uint16_t*>(pro->a);
  p.h_in = static_cast<const uint16_t*>(pro->h_in);
  p.h_out = static_cast<uint16_t*>(pro->h_out);
  p.w_post = static_cast<const uint16_t*>(pro->w_post);
  p.w_next = static_cast<const uint16_t*>(pro->w_next);
  p.eps = pro->eps;
  p.pa_parts = pro->a_parts;
  p.n_parts = pro->n_parts;
}

}  // namespace

extern "C" int gss_gemm_workspace_size(int M, int N, int Kd, size_t* bytes) {
  if (!bytes || M <= 0 || N <= 0 || Kd <= 0) return GSS_ERR_ARG;
  *bytes = gemm_ws_bytes(M, N, Kd);
  return GSS_OK;
}

extern "C" int gss_gemm(const void* x, int64_t ldx, const gss_norm_prologue* pro, const void* w, int64_t ldw, void* y,
                        int64_t ldy, int M, int N, int Kd, int out_dtype, const gss_norm_epilogue* post,
                        void* workspace, size_t workspace_bytes, gss_stream_t stream) {
  if (!y || ldy < N || (out_dtype != GSS_BF16 && out_dtype != GSS_F32)) return GSS_ERR_ARG;
  if ((ldy % 4) || (reinterpret_cast<uintptr_t>(y) & 15u)) return GSS_ERR_ARG;
  GemmParams p = {};
  p.x = static_cast<const uint16_t*>(x);
  p.ldx = ldx;
  p.w = static_cast<const uint16_t*>(w);
  p.ldw = ldw;
  p.y = y;
  p.ldy = ldy;
  p.M = M;
  p.N = N;
  p.Kd = Kd;
  p.out_f32 = out_dtype == GSS_F32;
  set_prologue(p, pro);
  if (post != nullptr) {
    if (!post->h) return GSS_ERR_ARG;
    p.post_h = static_cast<uint16_t*>(post->h);
    p.post_wp = static_cast<const uint16_t*>(post->w_post);
    p.post_wn = static_cast<const uint16_t*>(post->w_next);
    p.post_x = static_cast<uint16_t*>(post->x);
    p.post_eps = post->eps;
  }
  return gemm_entry(p, EPI_PLAIN, workspace, workspace_bytes, static_cast<hipStream_t>(stream));
}

extern "C" int gss_gemm_parts_count(int N, int Kd, int* n_parts) {
  if (!n_parts || N <= 0 || Kd <= 0 || N % 16 != 0 || Kd % 32 != 0) return GSS_ERR_ARG;
  const int ft = gemm_ft(N);
  *n_parts = gemm_parts_split((N + ft * 16 - 1) / (ft * 16), Kd / 32);
  return GSS_OK;
}

extern "C" int gss_gemm_parts(const void* x, int64_t ldx, const void* w, int64_t ldw, float* parts, int M, int N,
                              int Kd, gss_stream_t stream) {
  if (!parts || (reinterpret_cast<uintptr_t>(parts) & 15u)) return GSS_ERR_ARG;
  GemmParams p = {};
  p.x = static_cast<const uint16_t*>(x);
  p.ldx = ldx;
  p.w = static_cast<const uint16_t*>(w);
  p.ldw = ldw;
  p.y = parts;
  p.ldy = N;
  p.M = M;
  p.N = N;
  p.Kd = Kd;
  p.out_f32 = 1;
  return gemm_entry(p, EPI_PARTS, nullptr, 0, static_cast<hipStream_t>(stream));
}

extern "C" int gss_gemm_swiglu(const void* x, int64_t ldx, const gss_norm_prologue* pro, const void* w_gu_interleaved,
                               int64_t ldw, void* act, int M, int F, int Kd, void* workspace, size_t workspace_bytes,
                               gss_stream_t stream) {
  if (!act || (reinterpret_cast<uintptr_t>(act) & 3u)) return GSS_ERR_ARG;
  GemmParams p = {};
  p.x = static_cast<const uint16_t*>(x);
  p.ldx = ldx;
  p.w = static_cast<const uint16_t*>(w_gu_interleaved);
  p.ldw = ldw;
  p.y = act;
  p.ldy = F;
  p.M = M;
  p.N = 2 * F;
  p.Kd = Kd;
  set_prologue(p, pro);
  return gemm_entry(p, EPI_SWIGLU, workspace, workspace_bytes, static_cast<hipStream_t>(stream));
}

extern "C" int gss_gemm_rope_stage(const void* x, int64_t ldx, const gss_norm_prologue* pro, const void* w_qkv,
                                   int64_t ldw, const int32_t* seq_lens, const int32_t* pos_delta,
                                   const float* inv_freq, int rot_dim, void* q, void* k_win, void* v_win, int bs,
                                   int W, int Hq, int Hkv, int D, int Kd, void* workspace, size_t workspace_bytes,
                                   gss_stream_t stream) {
  if (!seq_lens || !inv_freq || !q || !k_win || !v_win || bs <= 0 || W <= 0) return GSS_ERR_ARG;
  if (D % 16 != 0 || rot_dim < 0 || rot_dim > D || rot_dim % 2) return GSS_ERR_ARG;
  GemmParams p = {};
  p.x = static_cast<const uint16_t*>(x);
  p.ldx = ldx;
  p.w = static_cast<const uint16_t*>(w_qkv);
  p.ldw = ldw;
  p.y = nullptr;
  p.M = bs * W;
  p.N = (Hq + 2 * Hkv) * D;
  p.Kd = Kd;
  p.seq_lens = seq_lens;
  p.pos_delta = pos_delta;
  p.inv_freq = inv_freq;
  p.rot_dim = rot_dim;
  p.W = W;
  p.Hq = Hq;
  p.Hkv = Hkv;
  p.D = D;
  p.q_out = static_cast<uint16_t*>(q);
  p.k_out = static_cast<uint16_t*>(k_win);
  p.v_out = static_cast<uint16_t*>(v_win);
  set_prologue(p, pro);
  return gemm_entry(p, EPI_ROPE, workspace, workspace_bytes, static_cast<hipStream_t>(stream));
}
