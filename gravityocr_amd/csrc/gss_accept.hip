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

// Up to 16 consecutive logits starting at j0 (j0 < V) into vals, in index order; returns how many are in range.
template <typename T>
GSS_DEV int load16(const T* row, int j0, int V, float (&vals)[PER_THREAD]) {
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
    return PER_THREAD;
  }
  const int n = V - j0 < PER_THREAD ? V - j0 : PER_THREAD;
  for (int e = 0; e < n; ++e) vals[e] = load_logit<T>(row, j0 + e);
  return n;
}

template <typename T>
GSS_DEV void scan16(const T* row, int j0, int V, float& bv, int& bi) {
  // 16 consecutive logits starting at j0 (in index order, so ties keep the earlier index)
  float vals[PER_THREAD];
  const int n = load16<T>(row, j0, V, vals);
  if (n == PER_THREAD) {
#pragma unroll
    for (int e = 0; e < PER_THREAD; ++e)
      if (beats(vals[e], j0 + e, bv, bi)) { bv = vals[e]; bi = j0 + e; }
  } else {
    for (int e = 0; e < n; ++e)
      if (beats(vals[e], j0 + e, bv, bi)) { bv = vals[e]; bi = j0 + e; }
  }
}

struct ArgParams {
  const void* logits;
  int64_t ld_row;
  int W, V, n_chunks, flags;
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
    // softmax rule: a NaN or +inf anywhere in the row makes every fp32 softmax probability NaN, whose argmax is 0
    const bool soft = (p.flags & GSS_ARGMAX_SOFTMAX) && !((p.flags & GSS_ARGMAX_LAST_RAW) && tid == p.W - 1);
    if (soft && (v != v || v == INFINITY)) i = 0;
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

extern "C" int gss_argmax_accept(const void* logits, int dtype, int64_t ld_row, int bs, int W, int V, int flags,
                                 const int32_t* window, int32_t* target, int32_t* accept_len, int32_t* next_x0,
                                 int32_t* packed, void* workspace, size_t workspace_bytes, gss_stream_t stream) {
  if (!logits || !target || bs <= 0 || W <= 0 || V <= 0 || ld_row < V) return GSS_ERR_ARG;
  if (dtype != GSS_BF16 && dtype != GSS_F32) return GSS_ERR_ARG;
  if (flags & ~(GSS_ARGMAX_SOFTMAX | GSS_ARGMAX_LAST_RAW)) return GSS_ERR_ARG;
  if (W > MAX_W || bs > static_cast<int>(COUNTER_BYTES / sizeof(uint32_t))) return GSS_ERR_UNSUPPORTED;
  if (!workspace || workspace_bytes < ws_bytes(bs, W, V)) return GSS_ERR_WORKSPACE;
  ArgParams p;
  p.logits = logits;
  p.ld_row = ld_row;
  p.W = W;
  p.V = V;
  p.flags = flags;
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

// ---------------------------------------------------------------- block-diffusion unmask step --------------------
// One threshold-unmask step of the cached block-diffusion decode on the logits of one block forward.
// Phase 1: workgroup (chunk, row) reduces 4096 logits of one row to (max, first index of the max, sum of
//   exp(x - max)) under the greedy rule (NaN as max), across the wavefront with xor-shuffles and across the
//   workgroup through LDS in wave order, and hands it over like the argmax kernel.
// Phase 2: the last workgroup of sequence b merges the chunks of each row in chunk order (x1 = argmax of the fp32
//   softmax, conf = its probability = 1 / sum), applies the in-block token shift (position j reads row max(j-1, 0)),
//   and runs the unmask rule serially over the W positions.

namespace {

struct UnmaskParams {
  const void* logits;
  int64_t ld_row;
  int W, V, n_chunks, mask_id;
  float threshold;
  int32_t* block;       // [bs, W] in/out
  int32_t* x1_out;      // [bs, W] or null
  float* conf_out;      // [bs, W] or null
  int32_t* n_unmasked;  // [bs] or null
  int32_t* n_left;      // [bs] or null
  int32_t* seed_out;    // [bs] or null
  float* part_m;        // [bs*W, n_chunks]
  int32_t* part_i;
  float* part_s;
  uint32_t* counters;   // [bs]
};

// merge (om, oi, os) into (m, i, s): the greedy winner, and the exp-sums rescaled to its value. A part whose max is
// -inf holds no probability mass. Both lanes of a shuffle pair compute the same result (a + b == b + a).
GSS_DEV void merge_softmax(float& m, int& i, float& s, float om, int oi, float os) {
  float M = m;
  int I = i;
  if (beats(om, oi, m, i)) { M = om; I = oi; }
  const float a = m == -INFINITY ? 0.f : s * expf(m - M);
  const float b = om == -INFINITY ? 0.f : os * expf(om - M);
  m = M;
  i = I;
  s = a + b;
}

template <typename T>
__global__ void __launch_bounds__(ARG_THREADS) unmask_step_kernel(UnmaskParams p) {
  const int chunk = blockIdx.x, row = blockIdx.y;  // row = b * W + r
  const int b = row / p.W;
  const T* lrow = static_cast<const T*>(p.logits) + static_cast<int64_t>(row) * p.ld_row;
  const int tid = threadIdx.x;

  float m = -INFINITY, s = 0.f;
  int mi = 0x7fffffff;
  const int j0 = chunk * CHUNK + tid * PER_THREAD;
  if (j0 < p.V) {
    float vals[PER_THREAD];
    const int n = load16<T>(lrow, j0, p.V, vals);
    for (int e = 0; e < n; ++e)
      if (beats(vals[e], j0 + e, m, mi)) { m = vals[e]; mi = j0 + e; }
    if (m != -INFINITY)
      for (int e = 0; e < n; ++e) s += expf(vals[e] - m);
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    const float om = __shfl_xor(m, o, 64);
    const int oi = __shfl_xor(mi, o, 64);
    const float os = __shfl_xor(s, o, 64);
    merge_softmax(m, mi, s, om, oi, os);
  }
  __shared__ float wm[ARG_THREADS / 64], ws[ARG_THREADS / 64];
  __shared__ int wi[ARG_THREADS / 64];
  __shared__ bool is_last;
  if ((tid & 63) == 0) { wm[tid >> 6] = m; wi[tid >> 6] = mi; ws[tid >> 6] = s; }
  __syncthreads();
  if (tid == 0) {
    for (int w = 1; w < ARG_THREADS / 64; ++w) merge_softmax(m, mi, s, wm[w], wi[w], ws[w]);
    const int64_t slot = static_cast<int64_t>(row) * p.n_chunks + chunk;
    st_agent(reinterpret_cast<uint32_t*>(p.part_m + slot), __float_as_uint(m));
    st_agent(reinterpret_cast<uint32_t*>(p.part_i + slot), static_cast<uint32_t>(mi));
    st_agent(reinterpret_cast<uint32_t*>(p.part_s + slot), __float_as_uint(s));
    wait_stores();
    is_last = count_arrival(&p.counters[b]) == static_cast<uint32_t>(p.n_chunks * p.W - 1);
  }
  __syncthreads();
  if (!is_last) return;

  // ---- phase 2: this workgroup finishes sequence b ------------------------------------------------------------
  __shared__ int rx[MAX_W];
  __shared__ float rc[MAX_W];
  if (tid < p.W) {
    const int64_t base = (static_cast<int64_t>(b) * p.W + tid) * p.n_chunks;
    const uint32_t* pm = reinterpret_cast<const uint32_t*>(p.part_m) + base;
    const uint32_t* pi = reinterpret_cast<const uint32_t*>(p.part_i) + base;
    const uint32_t* ps = reinterpret_cast<const uint32_t*>(p.part_s) + base;
    float M = __uint_as_float(ld_agent(pm)), S = __uint_as_float(ld_agent(ps));
    int I = static_cast<int>(ld_agent(pi));
    for (int c = 1; c < p.n_chunks; ++c)
      merge_softmax(M, I, S, __uint_as_float(ld_agent(pm + c)), static_cast<int>(ld_agent(pi + c)),
                    __uint_as_float(ld_agent(ps + c)));
    // a NaN or +inf in the row, or a row of -inf, makes the whole fp32 softmax NaN: argmax 0, probability NaN
    const bool finite_max = M == M && M != INFINITY && M != -INFINITY;
    rx[tid] = finite_max ? I : 0;
    rc[tid] = finite_max ? 1.f / S : __builtin_nanf("");
  }
  __syncthreads();
  int32_t* blk = p.block + static_cast<int64_t>(b) * p.W;
  if (tid < p.W) {
    const int src = tid > 0 ? tid - 1 : 0;
    if (p.x1_out) p.x1_out[static_cast<int64_t>(b) * p.W + tid] = rx[src];
    if (p.conf_out) p.conf_out[static_cast<int64_t>(b) * p.W + tid] = rc[src];
  }
  if (tid == 0) {
    // the forced position: first argmax of conf over masked positions (-inf elsewhere; NaN as max)
    float best = -INFINITY;
    int bj = 0x7fffffff;
    for (int j = 0; j < p.W; ++j) {
      const float c = blk[j] == p.mask_id ? rc[j > 0 ? j - 1 : 0] : -INFINITY;
      if (beats(c, j, best, bj)) { best = c; bj = j; }
    }
    int un = 0, left = 0;
    for (int j = 0; j < p.W; ++j) {
      if (blk[j] != p.mask_id) continue;
      const int src = j > 0 ? j - 1 : 0;
      if (rc[src] > p.threshold || j == bj) {
        blk[j] = rx[src];
        ++un;
      }
      left += blk[j] == p.mask_id;  // a position unmasked to the mask id itself stays masked, as in the reference
    }
    if (p.n_unmasked) p.n_unmasked[b] = un;
    if (p.n_left) p.n_left[b] = left;
    if (p.seed_out) p.seed_out[b] = rx[p.W - 1];
    reset_counter(&p.counters[b]);
  }
}

size_t unmask_ws_bytes(int bs, int W, int V) {
  const size_t nc = (static_cast<size_t>(V) + CHUNK - 1) / CHUNK;
  const size_t parts = static_cast<size_t>(bs) * W * nc;
  return COUNTER_BYTES + parts * (2 * sizeof(float) + sizeof(int32_t));
}

}  // namespace

extern "C" int gss_unmask_workspace_size(int bs, int W, int V, size_t* bytes) {
  if (!bytes || bs <= 0 || W <= 0 || V <= 0) return GSS_ERR_ARG;
  if (W > MAX_W) return GSS_ERR_UNSUPPORTED;
  *bytes = unmask_ws_bytes(bs, W, V);
  return GSS_OK;
}

extern "C" int gss_unmask_step(const void* logits, int dtype, int64_t ld_row, int bs, int W, int V, int32_t* block,
                               int mask_id, float threshold, int32_t* x1, float* conf, int32_t* n_unmasked,
                               int32_t* n_left, int32_t* seed, void* workspace, size_t workspace_bytes,
                               gss_stream_t stream) {
  if (!logits || !block || bs <= 0 || W <= 0 || V <= 0 || ld_row < V) return GSS_ERR_ARG;
  if (dtype != GSS_BF16 && dtype != GSS_F32) return GSS_ERR_ARG;
  if (W > MAX_W || bs > static_cast<int>(COUNTER_BYTES / sizeof(uint32_t))) return GSS_ERR_UNSUPPORTED;
  if (!workspace || workspace_bytes < unmask_ws_bytes(bs, W, V)) return GSS_ERR_WORKSPACE;
  UnmaskParams p;
  p.logits = logits;
  p.ld_row = ld_row;
  p.W = W;
  p.V = V;
  p.n_chunks = (V + CHUNK - 1) / CHUNK;
  p.mask_id = mask_id;
  p.threshold = threshold;
  p.block = block;
  p.x1_out = x1;
  p.conf_out = conf;
  p.n_unmasked = n_unmasked;
  p.n_left = n_left;
  p.seed_out = seed;
  const size_t parts = static_cast<size_t>(bs) * W * p.n_chunks;
  p.counters = static_cast<uint32_t*>(workspace);
  p.part_m = reinterpret_cast<float*>(static_cast<char*>(workspace) + COUNTER_BYTES);
  p.part_s = p.part_m + parts;
  p.part_i = reinterpret_cast<int32_t*>(p.part_s + parts);
  const dim3 grid(p.n_chunks, bs * W);
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (dtype == GSS_BF16)
    hipLaunchKernelGGL(unmask_step_kernel<uint16_t>, grid, dim3(ARG_THREADS), 0, st, p);
  else
    hipLaunchKernelGGL(unmask_step_kernel<float>, grid, dim3(ARG_THREADS), 0, st, p);
  return gss_launch_status();
}
