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
                                                         const float* inv_freq, int rot_dim, uint16_t* q,
                                                         uint16_t* k_win, uint16_t* v_win, int W, int Hq, int Hkv,
                                                         int D) {
  const int row = blockIdx.x;  // b * W + w
  const int b = row / W, w = row % W;
  const int pos = seq_lens[b] + (pos_delta ? pos_delta[b] : 0) + pos_offset + w;
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
      const float f = static_cast<float>(pos) * inv_freq[i];
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
GSS_DEV float sum_squares_row(const uint16_t* x, int H, float* red) {
  float ss = 0.f;
  for (int j = threadIdx.x; j < H; j += blockDim.x) {
    const float v = bf16_to_f32(x[j]);
    ss += v * v;
  }
  return block_sum(ss, red);
}

__global__ void __launch_bounds__(256) rmsnorm_kernel(const uint16_t* x, const uint16_t* w, uint16_t* out, int H,
                                                      float eps) {
  __shared__ float red[4];
  const uint16_t* xr = x + static_cast<int64_t>(blockIdx.x) * H;
  uint16_t* orow = out + static_cast<int64_t>(blockIdx.x) * H;
  const float r = 1.f / sqrtf(sum_squares_row(xr, H, red) / static_cast<float>(H) + eps);
  for (int j = threadIdx.x; j < H; j += blockDim.x)
    orow[j] = f32_to_bf16(bf16_to_f32(w[j]) * round_bf16(bf16_to_f32(xr[j]) * r));
}

// h = h + rmsnorm(a) * w_post ; x = rmsnorm(h) * w_next. One workgroup per row; the row of h stays in LDS.
__global__ void __launch_bounds__(256) add_rmsnorm_kernel(const uint16_t* a, const uint16_t* w_post, uint16_t* h,
                                                          const uint16_t* w_next, uint16_t* x, int H, float eps) {
  extern __shared__ float hrow[];
  __shared__ float red[4];
  const int64_t off = static_cast<int64_t>(blockIdx.x) * H;
  const float ra = 1.f / sqrtf(sum_squares_row(a + off, H, red) / static_cast<float>(H) + eps);
  float ss = 0.f;
  for (int j = threadIdx.x; j < H; j += blockDim.x) {
    const float na = round_bf16(bf16_to_f32(w_post[j]) * round_bf16(bf16_to_f32(a[off + j]) * ra));
    const float hn = round_bf16(bf16_to_f32(h[off + j]) + na);
    hrow[j] = hn;
    ss += hn * hn;
  }
  const float rh = 1.f / sqrtf(block_sum(ss, red) / static_cast<float>(H) + eps);
  for (int j = threadIdx.x; j < H; j += blockDim.x) {
    const float hn = hrow[j];
    h[off + j] = f32_to_bf16(hn);
    x[off + j] = f32_to_bf16(bf16_to_f32(w_next[j]) * round_bf16(hn * rh));
  }
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
                     static_cast<const uint16_t*>(qkv), ld_qkv, seq_lens, pos_delta, pos_offset, inv_freq, rot_dim,
                     static_cast<uint16_t*>(q), static_cast<uint16_t*>(k_win), static_cast<uint16_t*>(v_win), W, Hq,
                     Hkv, D);
  return gss_launch_status();
}

extern "C" int gss_rmsnorm(const void* x, const void* w, void* out, int rows, int H, float eps,
                           gss_stream_t stream) {
  if (!x || !w || !out || rows <= 0 || H <= 0) return GSS_ERR_ARG;
  hipLaunchKernelGGL(rmsnorm_kernel, dim3(rows), dim3(256), 0, static_cast<hipStream_t>(stream),
                     static_cast<const uint16_t*>(x), static_cast<const uint16_t*>(w), static_cast<uint16_t*>(out),
                     H, eps);
  return gss_launch_status();
}

extern "C" int gss_add_rmsnorm(const void* a, const void* w_post, void* h, const void* w_next, void* x, int rows,
                               int H, float eps, gss_stream_t stream) {
  if (!a || !w_post || !h || !w_next || !x || rows <= 0 || H <= 0) return GSS_ERR_ARG;
  if (H > 16384) return GSS_ERR_UNSUPPORTED;
  hipLaunchKernelGGL(add_rmsnorm_kernel, dim3(rows), dim3(256), H * sizeof(float),
                     static_cast<hipStream_t>(stream), static_cast<const uint16_t*>(a),
                     static_cast<const uint16_t*>(w_post), static_cast<uint16_t*>(h),
                     static_cast<const uint16_t*>(w_next), static_cast<uint16_t*>(x), H, eps);
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
