// (c) Fused LM-head argmax + accept-longest-prefix + bonus token, in one launch.
//
// Phase 1: workgroup (chunk, row) scans 4096 logits of one row (16 per thread, 16-byte loads), keeps the best
//   (value, index) under the greedy rule (max value, lowest index on ties, NaN as max), reduces across the
//   wavefront with xor-shuffles and across the workgroup through LDS, and stores the chunk's winner.
// Phase 2: the last workgroup to finish for a sequence (chunk winners handed over through the coherence point and an
//   atomic counter in the workspace) reduces the chunk winners of each of its W rows in chunk order, then runs the linear-chain accept:
//   acc = leading r with target[r] == window[r+1]; next_x0 = target[acc]; packed row as the reference's readback.
//   It then resets the counter, so the workspace needs zeroing only once and the launch is graph-replayable.
#include "gss_common.h"

namespace {

constexpr int ARG_THREADS = 256;
constexpr int PER_THREAD = 16;
constexpr int CHUNK = ARG_THREADS * PER_THREAD;  // logits per workgroup
constexpr int MAX_W = 64;

struct Best {
  float v;
  int i;
};

// a beats b: NaN first (lowest index among NaNs), then larger value, then lower index.
GSS_DEV bool beats(float av, int ai, float bv, int bi) {
  const bool an = av != av, bn = bv != bv;
  if (an || bn) return an && (!bn || ai < bi);
  return av > bv || (av == bv && ai < bi);
}

template <typename T>
GSS_DEV float load_logit(const T* p, int64_t i);
template <>
GSS_DEV float load_logit<uint16_t>(const uint16_t* p, int64_t i) { return bf16_to_f32(p[i]); }
template <>
GSS_DEV float load_logit<float>(const float* p, int64_t i) { return p[i]; }

template <typename T>
GSS_DEV void scan16(const T* row, int j0, int V, float& bv, int& bi) {
  // 16 consecutive logits starting at j0 (in index order, so ties keep the earlier index)
  float vals[PER_THREAD];
  const bool vec = (j0 + PER_THREAD <= V) && ((reinterpret_cast<uintptr_t>(row + j0) & 15u) == 0);
  if (vec) {
    if constexpr (sizeof(T) == 2) {
      const u32x4_t a = *reinterpret_cast<const u32x4_t*>(row + j0);
      const u32x4_t b = *reinterpret_cast<const u32x4_t*>(row + j0 + 8);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        vals[2 * e] = __uint_as_float(a[e] << 16);
        vals[2 * e + 1] = __uint_as_float(a[e] & 0xffff0000u);
        vals[8 + 2 * e] = __uint_as_float(b[e] << 16);
        vals[8 + 2 * e + 1] = __uint_as_float(b[e] & 0xffff0000u);
      }
    } else {
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const floatx4_t a = *reinterpret_cast<const floatx4_t*>(row + j0 + 4 * q);
#pragma unroll
        for (int e = 0; e < 4; ++e) vals[4 * q + e] = a[e];
      }
    }
#pragma unroll
    for (int e = 0; e < PER_THREAD; ++e)
      if (beats(vals[e], j0 + e, bv, bi)) { bv = vals[e]; bi = j0 + e; }
  } else {
    for (int e = 0; e < PER_THREAD && j0 + e < V; ++e) {
      const float x = load_logit<T>(row, j0 + e);
      if (beats(x, j0 + e, bv, bi)) { bv = x; bi = j0 + e; }
    }
  }
}

struct ArgParams {
  const void* logits;
  int64_t ld_row;
  int W, V, n_chunks;
  const int32_t* window;
  int32_t* target;
  int32_t* accept_len;
  int32_t* next_x0;
  int32_t* packed;
  float* part_v;       // [bs*W, n_chunks]
  int32_t* part_i;     // [bs*W, n_chunks]
  uint32_t* counters;  // [bs]
};

template <typename T>
__global__ void __launch_bounds__(ARG_THREADS) argmax_accept_kernel(ArgParams p) {
  const int chunk = blockIdx.x, row = blockIdx.y;  // row = b * W + r
  const int b = row / p.W;
  const T* lrow = static_cast<const T*>(p.logits) + static_cast<int64_t>(row) * p.ld_row;
  const int tid = threadIdx.x;

  float bv = -INFINITY;
  int bi = 0x7fffffff;
  const int j0 = chunk * CHUNK + tid * PER_THREAD;
  if (j0 < p.V) scan16<T>(lrow, j0, p.V, bv, bi);
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    const float ov = __shfl_xor(bv, o, 64);
    const int oi = __shfl_xor(bi, o, 64);
    if (beats(ov, oi, bv, bi)) { bv = ov; bi = oi; }
  }
  __shared__ float sv[ARG_THREADS / 64];
  __shared__ int si[ARG_THREADS / 64];
  __shared__ bool is_last;
  if ((tid & 63) == 0) { sv[tid >> 6] = bv; si[tid >> 6] = bi; }
  __syncthreads();
  if (tid == 0) {
    for (int w = 1; w < ARG_THREADS / 64; ++w)
      if (beats(sv[w], si[w], bv, bi)) { bv = sv[w]; bi = si[w]; }
    const int64_t slot = static_cast<int64_t>(row) * p.n_chunks + chunk;
    st_agent(reinterpret_cast<uint32_t*>(p.part_v + slot), __float_as_uint(bv));
    st_agent(reinterpret_cast<uint32_t*>(p.part_i + slot), static_cast<uint32_t>(bi));
    wait_stores();
    is_last = count_arrival(&p.counters[b]) == static_cast<uint32_t>(p.n_chunks * p.W - 1);
  }
  __syncthreads();
  if (!is_last) return;

  // ---- phase 2: this workgroup finishes sequence b ------------------------------------------------------------
  __shared__ int tgt[MAX_W];
  if (tid < p.W) {
    const int64_t base = (static_cast<int64_t>(b) * p.W + tid) * p.n_chunks;
    const uint32_t* pv = reinterpret_cast<const uint32_t*>(p.part_v) + base;
    const uint32_t* pi = reinterpret_cast<const uint32_t*>(p.part_i) + base;
    float v = __uint_as_float(ld_agent(pv));
    int i = static_cast<int>(ld_agent(pi));
    for (int c = 1; c < p.n_chunks; ++c) {
      const float cv = __uint_as_float(ld_agent(pv + c));
      const int ci = static_cast<int>(ld_agent(pi + c));
      if (beats(cv, ci, v, i)) { v = cv; i = ci; }
    }
    tgt[tid] = i;
    p.target[b * p.W + tid] = i;
  }
  __syncthreads();
  if (p.window != nullptr) {
    __shared__ int acc_s;
    if (tid == 0) {
      const int32_t* win = p.window + static_cast<int64_t>(b) * p.W;
      int a = 0;
      while (a < p.W - 1 && tgt[a] == win[a + 1]) ++a;
      acc_s = a;
      if (p.accept_len) p.accept_len[b] = a;
      if (p.next_x0) p.next_x0[b] = tgt[a];
      if (p.packed) {
        p.packed[static_cast<int64_t>(b) * (p.W + 2) + 0] = win[0];
        p.packed[static_cast<int64_t>(b) * (p.W + 2) + 1] = a;
      }
    }
    __syncthreads();
    if (p.packed && tid < p.W)
      p.packed[static_cast<int64_t>(b) * (p.W + 2) + 2 + tid] = tid <= acc_s ? tgt[tid] : 0;
  }
  if (tid == 0) reset_counter(&p.counters[b]);
}

// Workspace layout: the per-sequence counters first (a fixed offset, whatever W and V are, so calls with different
// window sizes can share one workspace), then the chunk winners' values and indices.
constexpr size_t COUNTER_BYTES = 4096;  // up to 1024 sequences

size_t ws_bytes(int bs, int W, int V) {
  const size_t nc = (static_cast<size_t>(V) + CHUNK - 1) / CHUNK;
  const size_t parts = static_cast<size_t>(bs) * W * nc;
  return COUNTER_BYTES + parts * (sizeof(float) + sizeof(int32_t));
}

}  // namespace

extern "C" int gss_argmax_workspace_size(int bs, int W, int V, size_t* bytes) {
  if (!bytes || bs <= 0 || W <= 0 || V <= 0) return GSS_ERR_ARG;
  if (W > MAX_W) return GSS_ERR_UNSUPPORTED;
  *bytes = ws_bytes(bs, W, V);
  return GSS_OK;
}

extern "C" int gss_argmax_accept(const void* logits, int dtype, int64_t ld_row, int bs, int W, int V,
                                 const int32_t* window, int32_t* target, int32_t* accept_len, int32_t* next_x0,
                                 int32_t* packed, void* workspace, size_t workspace_bytes, gss_stream_t stream) {
  if (!logits || !target || bs <= 0 || W <= 0 || V <= 0 || ld_row < V) return GSS_ERR_ARG;
  if (dtype != GSS_BF16 && dtype != GSS_F32) return GSS_ERR_ARG;
  if (W > MAX_W || bs > static_cast<int>(COUNTER_BYTES / sizeof(uint32_t))) return GSS_ERR_UNSUPPORTED;
  if (!workspace || workspace_bytes < ws_bytes(bs, W, V)) return GSS_ERR_WORKSPACE;
  ArgParams p;
  p.logits = logits;
  p.ld_row = ld_row;
  p.W = W;
  p.V = V;
  p.n_chunks = (V + CHUNK - 1) / CHUNK;
  p.window = window;
  p.target = target;
  p.accept_len = accept_len;
  p.next_x0 = next_x0;
  p.packed = packed;
  const size_t parts = static_cast<size_t>(bs) * W * p.n_chunks;
  p.counters = static_cast<uint32_t*>(workspace);
  p.part_v = reinterpret_cast<float*>(static_cast<char*>(workspace) + COUNTER_BYTES);
  p.part_i = reinterpret_cast<int32_t*>(p.part_v + parts);
  const dim3 grid(p.n_chunks, bs * W);
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (dtype == GSS_BF16)
    hipLaunchKernelGGL(argmax_accept_kernel<uint16_t>, grid, dim3(ARG_THREADS), 0, st, p);
  else
    hipLaunchKernelGGL(argmax_accept_kernel<float>, grid, dim3(ARG_THREADS), 0, st, p);
  return gss_launch_status();
}
