// Fused elementwise pieces of the GLM text decoder layer (transformers GlmOcrTextDecoderLayer), bf16 in/out with
// the same bf16 rounding points as the reference's bf16 module: every torch op on bf16 tensors rounds its result.
#include "gss_common.h"

#include <math.h>

namespace {

// ---- RoPE + window staging ---------------------------------------------------------------------------------------
// One workgroup per (sequence, window row). Thread t owns pair i = t % (D/2) of heads t/(D/2), t/(D/2)+H/.. and
// computes sin/cos once. GLM applies interleaved pairs (2i, 2i+1) over the first rot_dim dims with cos/sin cast to
// bf16 (modeling_glm_ocr.py:129-173): out0 = x0*c - x1*s, out1 = x1*c + x0*s, each product and sum rounded to bf16.
__global__ void __launch_bounds__(256) rope_stage_kernel(const uint16_t* qkv, int64_t ld_qkv, const int32_t* seq_lens,
                                                         const int32_t* pos_delta, int pos_offset,
                                                         const int32_t* pos3, int sec0, int sec01,
                                                         const float* inv_freq, int rot_dim, uint16_t* q,
                                                         uint16_t* k_win, uint16_t* v_win, int W, int Hq, int Hkv,
                                                         int D) {
  const int row = blockIdx.x;  // b * W + w
  const int b = row / W, w = row % W;
  // M-RoPE: with an explicit (t, h, w) position table, frequency i takes component 0 below sec0, 1 below sec01, else 2
  const int* p3 = pos3 ? pos3 + static_cast<int64_t>(row) * 3 : nullptr;
  const int pos = p3 ? 0 : seq_lens[b] + (pos_delta ? pos_delta[b] : 0) + pos_offset + w;
  const uint16_t* src = qkv + static_cast<int64_t>(row) * ld_qkv;
  const int half = D / 2;
  const int n_rot_heads = Hq + Hkv;
  for (int t = threadIdx.x; t < (n_rot_heads + Hkv) * half; t += blockDim.x) {
    const int h = t / half, i = t % half;
    const int d0 = 2 * i;
    if (h >= n_rot_heads) {  // V: plain copy
      const int hv = h - n_rot_heads;
      const uint32_t v2 = *reinterpret_cast<const uint32_t*>(src + (Hq + Hkv + hv) * D + d0);
      *reinterpret_cast<uint32_t*>(v_win + (static_cast<int64_t>(row) * Hkv + hv) * D + d0) = v2;
      continue;
    }
    const uint32_t x2 = *reinterpret_cast<const uint32_t*>(src + h * D + d0);
    uint32_t y2 = x2;
    if (d0 < rot_dim) {
      const float x0 = __uint_as_float(x2 << 16), x1 = __uint_as_float(x2 & 0xffff0000u);
      const int pi = p3 ? p3[i < sec0 ? 0 : (i < sec01 ? 1 : 2)] : pos;
      const float f = static_cast<float>(pi) * inv_freq[i];
      const float c = round_bf16(cosf(f)), s = round_bf16(sinf(f));
      const float y0 = round_bf16(round_bf16(x0 * c) - round_bf16(x1 * s));
      const float y1 = round_bf16(round_bf16(x1 * c) + round_bf16(x0 * s));
      y2 = pack_bf16x2(y0, y1);
    }
    if (h < Hq)
      *reinterpret_cast<uint32_t*>(q + (static_cast<int64_t>(row) * Hq + h) * D + d0) = y2;
    else
      *reinterpret_cast<uint32_t*>(k_win + (static_cast<int64_t>(row) * Hkv + (h - Hq)) * D + d0) = y2;
  }
}

// ---- RMSNorm -------------------------------------------------------------------------------------------------------
// GlmOcrRMSNorm: y = x * 1/sqrt(mean(x^2) + eps) in fp32, rounded to bf16, then weight * y rounded to bf16.
// One wavefront per row: lane l owns the E = H/64 consecutive elements [l*E, (l+1)*E) (loaded 16 bytes at a time
// when E % 8 == 0), all loads are issued up front, and the row sums are xor-shuffle reductions (fixed order).
constexpr int NORM_ROWS_PER_BLOCK = 4;
constexpr int MAX_E = 32;  // H <= 2048

template <int E>
GSS_DEV void load_row(const uint16_t* src, float* v) {
  if constexpr (E % 8 == 0) {
#pragma unroll
    for (int c = 0; c < E / 8; ++c) {
      const u32x4_t q = *reinterpret_cast<const u32x4_t*>(src + c * 8);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        v[c * 8 + 2 * e] = __uint_as_float(q[e] << 16);
        v[c * 8 + 2 * e + 1] = __uint_as_float(q[e] & 0xffff0000u);
      }
    }
  } else {
#pragma unroll
    for (int e = 0; e < E; ++e) v[e] = bf16_to_f32(src[e]);
  }
}

template <int E>
GSS_DEV void store_row(uint16_t* dst, const float* v) {
  if constexpr (E % 8 == 0) {
#pragma unroll
    for (int c = 0; c < E / 8; ++c)
      *reinterpret_cast<u32x4_t*>(dst + c * 8) =
          u32x4_t{pack_bf16x2(v[c * 8], v[c * 8 + 1]), pack_bf16x2(v[c * 8 + 2], v[c * 8 + 3]),
                  pack_bf16x2(v[c * 8 + 4], v[c * 8 + 5]), pack_bf16x2(v[c * 8 + 6], v[c * 8 + 7])};
  } else {
#pragma unroll
    for (int e = 0; e < E; ++e) dst[e] = f32_to_bf16(v[e]);
  }
}

template <int E>
__global__ void __launch_bounds__(64 * NORM_ROWS_PER_BLOCK) rmsnorm_kernel(const uint16_t* x, const uint16_t* w,
                                                                           uint16_t* out, int rows, float eps) {
  constexpr int H = 64 * E;
  const int row = blockIdx.x * NORM_ROWS_PER_BLOCK + (threadIdx.x >> 6), lane = threadIdx.x & 63;
  if (row >= rows) return;
  float xv[E], wv[E];
  load_row<E>(x + static_cast<int64_t>(row) * H + lane * E, xv);
  load_row<E>(w + lane * E, wv);
  float ss = 0.f;
#pragma unroll
  for (int e = 0; e < E; ++e) ss += xv[e] * xv[e];
  const float r = 1.f / sqrtf(wave_sum(ss) / static_cast<float>(H) + eps);
#pragma unroll
  for (int e = 0; e < E; ++e) xv[e] = wv[e] * round_bf16(xv[e] * r);
  store_row<E>(out + static_cast<int64_t>(row) * H + lane * E, xv);
}

// Embedding lookup + the first input norm: h = table[ids[row]] (the residual stream), x = rmsnorm(h) * w. An id
// outside [0, V) reads nothing and gives a zero row.
template <int E>
__global__ void __launch_bounds__(64 * NORM_ROWS_PER_BLOCK) embed_rmsnorm_kernel(const uint16_t* table,
                                                                                 const int32_t* ids, int V,
                                                                                 const uint16_t* w, uint16_t* h,
                                                                                 uint16_t* x, int rows, float eps) {
  constexpr int H = 64 * E;
  const int row = blockIdx.x * NORM_ROWS_PER_BLOCK + (threadIdx.x >> 6), lane = threadIdx.x & 63;
  if (row >= rows) return;
  const int id = ids[row];
  float xv[E], wv[E];
  if (id >= 0 && id < V) {
    load_row<E>(table + static_cast<int64_t>(id) * H + lane * E, xv);
  } else {
#pragma unroll
    for (int e = 0; e < E; ++e) xv[e] = 0.f;
  }
  load_row<E>(w + lane * E, wv);
  const int64_t off = static_cast<int64_t>(row) * H + lane * E;
  store_row<E>(h + off, xv);
  float ss = 0.f;
#pragma unroll
  for (int e = 0; e < E; ++e) ss += xv[e] * xv[e];
  const float r = 1.f / sqrtf(wave_sum(ss) / static_cast<float>(H) + eps);
#pragma unroll
  for (int e = 0; e < E; ++e) xv[e] = wv[e] * round_bf16(xv[e] * r);
  store_row<E>(x + off, xv);
}

// h = h + rmsnorm(a) * w_post ; x = rmsnorm(h) * w_next (sandwich-norm residual, then the next norm)
template <int E>
__global__ void __launch_bounds__(64 * NORM_ROWS_PER_BLOCK) add_rmsnorm_kernel(const uint16_t* a,
                                                                               const uint16_t* w_post, uint16_t* h,
                                                                               const uint16_t* w_next, uint16_t* x,
                                                                               int rows, float eps) {
  constexpr int H = 64 * E;
  const int row = blockIdx.x * NORM_ROWS_PER_BLOCK + (threadIdx.x >> 6), lane = threadIdx.x & 63;
  if (row >= rows) return;
  const int64_t off = static_cast<int64_t>(row) * H + lane * E;
  float av[E], hv[E], wp[E], wn[E];
  load_row<E>(a + off, av);
  load_row<E>(h + off, hv);
  load_row<E>(w_post + lane * E, wp);
  load_row<E>(w_next + lane * E, wn);
  float ss = 0.f;
#pragma unroll
  for (int e = 0; e < E; ++e) ss += av[e] * av[e];
  const float ra = 1.f / sqrtf(wave_sum(ss) / static_cast<float>(H) + eps);
  float sh = 0.f;
#pragma unroll
  for (int e = 0; e < E; ++e) {
    hv[e] = round_bf16(hv[e] + round_bf16(wp[e] * round_bf16(av[e] * ra)));
    sh += hv[e] * hv[e];
  }
  const float rh = 1.f / sqrtf(wave_sum(sh) / static_cast<float>(H) + eps);
  store_row<E>(h + off, hv);
#pragma unroll
  for (int e = 0; e < E; ++e) av[e] = wn[e] * round_bf16(hv[e] * rh);
  store_row<E>(x + off, av);
}

// The same with a given as NP fp32 partial sums [NP][rows][H] (a skinny GEMM's k splits): a = bf16 of their sum,
// added in part order. One wavefront per row, one row per workgroup (the parts are the bulk of the reads). NP is a
// compile-time count so every part load of the row is issued before the first one is used: one memory round trip.
template <int E, int NP>
__global__ void __launch_bounds__(64) add_rmsnorm_parts_kernel(const float* parts, const uint16_t* w_post,
                                                               uint16_t* h, const uint16_t* w_next, uint16_t* x,
                                                               int rows, float eps) {
  constexpr int H = 64 * E;
  const int row = blockIdx.x, lane = threadIdx.x;
  const int64_t off = static_cast<int64_t>(row) * H + lane * E;
  float av[E], hv[E], wp[E], wn[E];
  const int64_t pstride = static_cast<int64_t>(rows) * H;
  floatx4_t pv[NP][E / 4];
#pragma unroll
  for (int k = 0; k < NP; ++k)
#pragma unroll
    for (int e = 0; e < E; e += 4) pv[k][e / 4] = *reinterpret_cast<const floatx4_t*>(parts + k * pstride + off + e);
  load_row<E>(h + off, hv);
  load_row<E>(w_post + lane * E, wp);
  load_row<E>(w_next + lane * E, wn);
#pragma unroll
  for (int e = 0; e < E; e += 4) {
    floatx4_t s = pv[0][e / 4];
#pragma unroll
    for (int k = 1; k < NP; ++k) s += pv[k][e / 4];
#pragma unroll
    for (int i = 0; i < 4; ++i) av[e + i] = round_bf16(s[i]);
  }
  float ss = 0.f;
#pragma unroll
  for (int e = 0; e < E; ++e) ss += av[e] * av[e];
  const float ra = 1.f / sqrtf(wave_sum(ss) / static_cast<float>(H) + eps);
  float sh = 0.f;
#pragma unroll
  for (int e = 0; e < E; ++e) {
    hv[e] = round_bf16(hv[e] + round_bf16(wp[e] * round_bf16(av[e] * ra)));
    sh += hv[e] * hv[e];
  }
  const float rh = 1.f / sqrtf(wave_sum(sh) / static_cast<float>(H) + eps);
  store_row<E>(h + off, hv);
#pragma unroll
  for (int e = 0; e < E; ++e) av[e] = wn[e] * round_bf16(hv[e] * rh);
  store_row<E>(x + off, av);
}

// up * silu(gate): silu rounded to bf16 (torch's bf16 silu), then the product rounded.
__global__ void __launch_bounds__(256) silu_mul_kernel(const uint16_t* gu, int64_t ld_gu, uint16_t* out, int F) {
  const uint16_t* r = gu + static_cast<int64_t>(blockIdx.y) * ld_gu;
  uint16_t* o = out + static_cast<int64_t>(blockIdx.y) * F;
  for (int j = blockIdx.x * blockDim.x + threadIdx.x; j < F; j += gridDim.x * blockDim.x) {
    const float g = bf16_to_f32(r[j]), u = bf16_to_f32(r[F + j]);
    const float sg = round_bf16(g / (1.f + expf(-g)));
    o[j] = f32_to_bf16(u * sg);
  }
}

}  // namespace

extern "C" int gss_rope_stage(const void* qkv, int64_t ld_qkv, const int32_t* seq_lens, const int32_t* pos_delta,
                              int pos_offset, const float* inv_freq, int rot_dim, void* q, void* k_win, void* v_win,
                              int bs, int W, int Hq, int Hkv, int D, gss_stream_t stream) {
  if (!qkv || !seq_lens || !inv_freq || !q || !k_win || !v_win) return GSS_ERR_ARG;
  if (bs <= 0 || W <= 0 || Hq <= 0 || Hkv <= 0 || D <= 0 || D % 2 != 0) return GSS_ERR_ARG;
  if (rot_dim < 0 || rot_dim > D || rot_dim % 2 != 0 || ld_qkv < static_cast<int64_t>(Hq + 2 * Hkv) * D)
    return GSS_ERR_ARG;
  hipLaunchKernelGGL(rope_stage_kernel, dim3(bs * W), dim3(256), 0, static_cast<hipStream_t>(stream),
                     static_cast<const uint16_t*>(qkv), ld_qkv, seq_lens, pos_delta, pos_offset, nullptr, 0, 0,
                     inv_freq, rot_dim, static_cast<uint16_t*>(q), static_cast<uint16_t*>(k_win),
                     static_cast<uint16_t*>(v_win), W, Hq, Hkv, D);
  return gss_launch_status();
}

extern "C" int gss_rope_stage_mrope(const void* qkv, int64_t ld_qkv, const int32_t* positions, int sec_t, int sec_h,
                                    const float* inv_freq, int rot_dim, void* q, void* k_win, void* v_win, int rows,
                                    int Hq, int Hkv, int D, gss_stream_t stream) {
  if (!qkv || !positions || !inv_freq || !q || !k_win || !v_win) return GSS_ERR_ARG;
  if (rows <= 0 || Hq <= 0 || Hkv <= 0 || D <= 0 || D % 2 != 0 || sec_t < 0 || sec_h < 0) return GSS_ERR_ARG;
  if (rot_dim < 0 || rot_dim > D || rot_dim % 2 != 0 || ld_qkv < static_cast<int64_t>(Hq + 2 * Hkv) * D)
    return GSS_ERR_ARG;
  // one sequence of `rows` window rows; seq_lens is not read when the position table is given
  hipLaunchKernelGGL(rope_stage_kernel, dim3(rows), dim3(256), 0, static_cast<hipStream_t>(stream),
                     static_cast<const uint16_t*>(qkv), ld_qkv, nullptr, nullptr, 0, positions, sec_t,
                     sec_t + sec_h, inv_freq, rot_dim, static_cast<uint16_t*>(q), static_cast<uint16_t*>(k_win),
                     static_cast<uint16_t*>(v_win), rows, Hq, Hkv, D);
  return gss_launch_status();
}

#define GSS_NORM_CASES(X) X(1) X(2) X(4) X(6) X(8) X(12) X(16) X(24) X(32)

extern "C" int gss_rmsnorm(const void* x, const void* w, void* out, int rows, int H, float eps,
                           gss_stream_t stream) {
  if (!x || !w || !out || rows <= 0 || H <= 0) return GSS_ERR_ARG;
  if (H % 64 != 0 || H / 64 > MAX_E) return GSS_ERR_UNSUPPORTED;
  const dim3 grid((rows + NORM_ROWS_PER_BLOCK - 1) / NORM_ROWS_PER_BLOCK), block(64 * NORM_ROWS_PER_BLOCK);
  hipStream_t st = static_cast<hipStream_t>(stream);
  const uint16_t *xs = static_cast<const uint16_t*>(x), *ws = static_cast<const uint16_t*>(w);
  uint16_t* os = static_cast<uint16_t*>(out);
  switch (H / 64) {
#define X(E) \
  case E: hipLaunchKernelGGL(rmsnorm_kernel<E>, grid, block, 0, st, xs, ws, os, rows, eps); break;
    GSS_NORM_CASES(X)
#undef X
    default: return GSS_ERR_UNSUPPORTED;
  }
  return gss_launch_status();
}

extern "C" int gss_embed_rmsnorm(const void* table, const int32_t* ids, int V, const void* w, void* h, void* x,
                                 int rows, int H, float eps, gss_stream_t stream) {
  if (!table || !ids || !w || !h || !x || rows <= 0 || H <= 0 || V <= 0) return GSS_ERR_ARG;
  if (H % 64 != 0 || H / 64 > MAX_E) return GSS_ERR_UNSUPPORTED;
  const dim3 grid((rows + NORM_ROWS_PER_BLOCK - 1) / NORM_ROWS_PER_BLOCK), block(64 * NORM_ROWS_PER_BLOCK);
  hipStream_t st = static_cast<hipStream_t>(stream);
  const uint16_t *ts = static_cast<const uint16_t*>(table), *ws = static_cast<const uint16_t*>(w);
  uint16_t *hs = static_cast<uint16_t*>(h), *xs = static_cast<uint16_t*>(x);
  switch (H / 64) {
#define X(E) \
  case E: hipLaunchKernelGGL(embed_rmsnorm_kernel<E>, grid, block, 0, st, ts, ids, V, ws, hs, xs, rows, eps); break;
    GSS_NORM_CASES(X)
#undef X
    default: return GSS_ERR_UNSUPPORTED;
  }
  return gss_launch_status();
}

extern "C" int gss_add_rmsnorm(const void* a, const void* w_post, void* h, const void* w_next, void* x, int rows,
                               int H, float eps, gss_stream_t stream) {
  if (!a || !w_post || !h || !w_next || !x || rows <= 0 || H <= 0) return GSS_ERR_ARG;
  if (H % 64 != 0 || H / 64 > MAX_E) return GSS_ERR_UNSUPPORTED;
  const dim3 grid((rows + NORM_ROWS_PER_BLOCK - 1) / NORM_ROWS_PER_BLOCK), block(64 * NORM_ROWS_PER_BLOCK);
  hipStream_t st = static_cast<hipStream_t>(stream);
  const uint16_t *as = static_cast<const uint16_t*>(a), *wp = static_cast<const uint16_t*>(w_post),
                 *wn = static_cast<const uint16_t*>(w_next);
  uint16_t *hs = static_cast<uint16_t*>(h), *xs = static_cast<uint16_t*>(x);
  switch (H / 64) {
#define X(E) \
  case E: hipLaunchKernelGGL(add_rmsnorm_kernel<E>, grid, block, 0, st, as, wp, hs, wn, xs, rows, eps); break;
    GSS_NORM_CASES(X)
#undef X
    default: return GSS_ERR_UNSUPPORTED;
  }
  return gss_launch_status();
}

extern "C" int gss_add_rmsnorm_parts(const float* parts, int n_parts, const void* w_post, void* h, const void* w_next,
                                     void* x, int rows, int H, float eps, gss_stream_t stream) {
  if (!parts || !w_post || !h || !w_next || !x || rows <= 0 || H <= 0 || n_parts < 1) return GSS_ERR_ARG;
  if (reinterpret_cast<uintptr_t>(parts) & 15u) return GSS_ERR_ARG;
  if (H % 64 != 0 || H / 64 > MAX_E || (H / 64) % 4 != 0 || n_parts > 4) return GSS_ERR_UNSUPPORTED;
  hipStream_t st = static_cast<hipStream_t>(stream);
  const uint16_t *wp = static_cast<const uint16_t*>(w_post), *wn = static_cast<const uint16_t*>(w_next);
  uint16_t *hs = static_cast<uint16_t*>(h), *xs = static_cast<uint16_t*>(x);
  switch (H / 64) {
#define NPX(E, NP)                                                                                          \
  case NP:                                                                                                  \
    hipLaunchKernelGGL((add_rmsnorm_parts_kernel<E, NP>), dim3(rows), dim3(64), 0, st, parts, wp, hs, wn, xs, rows, \
                       eps);                                                                                \
    break;
#define X(E)                                             \
  case E:                                                \
    switch (n_parts) { NPX(E, 1) NPX(E, 2) NPX(E, 3) NPX(E, 4) } \
    break;
    X(4) X(8) X(12) X(16) X(24) X(32)
#undef X
#undef NPX
    default: return GSS_ERR_UNSUPPORTED;
  }
  return gss_launch_status();
}

extern "C" int gss_silu_mul(const void* gu, int64_t ld_gu, void* out, int rows, int F, gss_stream_t stream) {
  if (!gu || !out || rows <= 0 || F <= 0 || ld_gu < 2 * static_cast<int64_t>(F)) return GSS_ERR_ARG;
  const int bx = (F + 255) / 256 < 8 ? (F + 255) / 256 : 8;
  hipLaunchKernelGGL(silu_mul_kernel, dim3(bx, rows), dim3(256), 0, static_cast<hipStream_t>(stream),
                     static_cast<const uint16_t*>(gu), ld_gu, static_cast<uint16_t*>(out), F);
  return gss_launch_status();
}

extern "C" const char* gss_version(void) { return "gss 0.1 gfx950"; }

extern "C" const char* gss_status_string(int status) {
  switch (status) {
    case GSS_OK: return "ok";
    case GSS_ERR_ARG: return "invalid argument";
    case GSS_ERR_UNSUPPORTED: return "unsupported shape";
    case GSS_ERR_WORKSPACE: return "workspace missing or too small";
    case GSS_ERR_LAUNCH: return "kernel launch failed";
    default: return "unknown status";
  }
}
