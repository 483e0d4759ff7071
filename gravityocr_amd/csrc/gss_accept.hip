// (c) Fused LM-head argmax + accept-longest-prefix + bonus token, in one launch.
//
// Phase 1: workgroup (chunk, row) scans 1, 2 or 4 pieces of 4096 logits of one row (16 per thread per piece,
//   16-byte loads; more pieces per workgroup for larger batches), keeps the best (value, index) under the greedy
//   rule (max value, lowest index on ties, NaN as max), reduces across the wavefront with xor-shuffles and across
//   the workgroup through LDS, and stores the chunk's winner.
// Phase 2: the last workgroup to finish for a sequence (chunk winners handed over through the coherence point and
//   two levels of atomic counters in the workspace) reduces the chunk winners of each of its W rows in chunk order, then runs the linear-chain accept:
//   acc = leading r with target[r] == window[r+1]; next_x0 = target[acc]; packed row as the reference's readback.
//   It then resets the counter, so the workspace needs zeroing only once and the launch is graph-replayable.
#include "gss_common.h"

#include <mutex>

namespace {

constexpr int ARG_THREADS = 256;
constexpr int PER_THREAD = 16;
constexpr int CHUNK = ARG_THREADS * PER_THREAD;  // logits per workgroup
constexpr int MAX_W = 64;
constexpr int MAX_CHUNKS = 32;  // V <= MAX_CHUNKS * CHUNK (131072)

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
#pragma unroll
  for (int e = 0; e < PER_THREAD; ++e) vals[e] = e < n ? load_logit<T>(row, j0 + e) : -INFINITY;  // static indices
  return n;
}


// Arrival counting of the (chunk, row) workgroups of one sequence, in two levels: workgroup g counts into sub-counter
// g % SUB, the last arrival of each sub-counter counts into the sequence counter, and the last of those finishes the
// sequence. Every counter sits on its own 128-byte line: atomics on one line serialize, and a single counter taking
// W * n_chunks arrivals costs several microseconds. The sub-counters reset themselves; the finishing workgroup resets
// the sequence counter when it is done.
constexpr int SUB = 8;
constexpr int LINE_U32 = 32;
constexpr int MAX_SEQ = 1024;
constexpr size_t COUNTER_BYTES = static_cast<size_t>(MAX_SEQ) * (SUB + 1) * LINE_U32 * sizeof(uint32_t);

GSS_DEV uint32_t* seq_counter(uint32_t* counters, int b) {
  return counters + static_cast<size_t>(b) * (SUB + 1) * LINE_U32;
}

GSS_DEV bool arrive_last(uint32_t* counters, int b, int g, int n_g) {
  uint32_t* base = seq_counter(counters, b);
  const int sub = g % SUB;
  const int in_sub = (n_g - 1 - sub) / SUB + 1;  // workgroups counting into this sub-counter
  uint32_t* c = base + (1 + sub) * LINE_U32;
  if (count_arrival(c) != static_cast<uint32_t>(in_sub - 1)) return false;
  reset_counter(c);
  return count_arrival(base) == static_cast<uint32_t>((n_g < SUB ? n_g : SUB) - 1);
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
  uint64_t* part;      // [bs*W, n_chunks] chunk winner (value bits | index << 32)
  uint32_t* counters;  // arrival counters (see arrive_last)
};


// SPC: CHUNK-logit pieces of the row per workgroup (chunk c covers pieces [c * SPC, (c + 1) * SPC)); the winner is
// the maximum of a strict total order, so it does not depend on how the row is cut. A thread loads all its pieces
// before comparing, so they are in flight together.
template <typename T, int SPC>
__global__ void __launch_bounds__(ARG_THREADS) argmax_accept_kernel(ArgParams p) {
  const int chunk = blockIdx.x, row = blockIdx.y;  // row = b * W + r
  const int b = row / p.W;
  const T* lrow = static_cast<const T*>(p.logits) + static_cast<int64_t>(row) * p.ld_row;
  const int tid = threadIdx.x;

  float bv = -INFINITY;
  int bi = 0x7fffffff;
  float vals[SPC][PER_THREAD];
  int n[SPC];
  bool full = true;
#pragma unroll
  for (int q = 0; q < SPC; ++q) {
    const int j0 = (chunk * SPC + q) * CHUNK + tid * PER_THREAD;
    if (j0 < p.V) {
      n[q] = load16<T>(lrow, j0, p.V, vals[q]);
    } else {
      n[q] = 0;
#pragma unroll
      for (int e = 0; e < PER_THREAD; ++e) vals[q][e] = -INFINITY;
    }
    full = full && n[q] == PER_THREAD;
  }
  // Fast path (every piece full, no NaN): the thread's maximum, then the lowest index holding it (ties between
  // +0 and -0 compare equal, as in the rule). Otherwise the rule's own comparison, element by element.
  float m = -INFINITY;
  bool nan = false;
#pragma unroll
  for (int q = 0; q < SPC; ++q)
#pragma unroll
    for (int e = 0; e < PER_THREAD; ++e) {
      nan = nan || vals[q][e] != vals[q][e];
      m = fmaxf(m, vals[q][e]);
    }
  if (full && !nan) {
    bv = m;
#pragma unroll
    for (int q = SPC - 1; q >= 0; --q)
#pragma unroll
      for (int e = PER_THREAD - 1; e >= 0; --e)
        if (vals[q][e] == m) bi = (chunk * SPC + q) * CHUNK + tid * PER_THREAD + e;
  } else {
#pragma unroll
    for (int q = 0; q < SPC; ++q) {  // pieces in index order, each in index order
      const int j0 = (chunk * SPC + q) * CHUNK + tid * PER_THREAD;
#pragma unroll
      for (int e = 0; e < PER_THREAD; ++e)
        if (e < n[q] && beats(vals[q][e], j0 + e, bv, bi)) { bv = vals[q][e]; bi = j0 + e; }
    }
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    const float ov = lane_xor(bv, o);
    const int oi = lane_xor(bi, o);
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
    st_agent(p.part + slot, static_cast<uint64_t>(__float_as_uint(bv)) | (static_cast<uint64_t>(bi) << 32));
    wait_stores();
    const int r = row - b * p.W;
    is_last = arrive_last(p.counters, b, r * p.n_chunks + chunk, p.W * p.n_chunks);
  }
  __syncthreads();
  if (!is_last) return;

  // ---- phase 2: this workgroup finishes sequence b ------------------------------------------------------------
  // the chunk winners of its W rows, one (row, chunk) per thread (coherent loads), then each row in chunk order
  __shared__ float cv_s[MAX_W * MAX_CHUNKS];
  __shared__ int ci_s[MAX_W * MAX_CHUNKS];
  __shared__ int tgt[MAX_W];
  __shared__ int win_s[MAX_W];
  if (p.window != nullptr && tid < p.W) win_s[tid] = p.window[static_cast<int64_t>(b) * p.W + tid];
  {
    const uint32_t* base = reinterpret_cast<const uint32_t*>(p.part + static_cast<int64_t>(b) * p.W * p.n_chunks);
    for (int t = tid; t < p.W * p.n_chunks; t += ARG_THREADS) {
      uint32_t v, i, unused;
      ld_agent_u32(2, base + 2 * t, base + 2 * t + 1, nullptr, v, i, unused);
      cv_s[t] = __uint_as_float(v);
      ci_s[t] = static_cast<int>(i);
    }
  }
  __syncthreads();
  if (tid < p.W) {
    const float* rv = cv_s + tid * p.n_chunks;
    const int* ri = ci_s + tid * p.n_chunks;
    float v = rv[0];
    int i = ri[0];
    for (int c = 1; c < p.n_chunks; ++c)
      if (beats(rv[c], ri[c], v, i)) { v = rv[c]; i = ri[c]; }
    // softmax rule: a NaN or +inf anywhere in the row makes every fp32 softmax probability NaN, whose argmax is 0
    const bool soft = (p.flags & GSS_ARGMAX_SOFTMAX) && !((p.flags & GSS_ARGMAX_LAST_RAW) && tid == p.W - 1);
    if (soft && (v != v || v == INFINITY)) i = 0;
    tgt[tid] = i;
    p.target[b * p.W + tid] = i;
  }
  __syncthreads();
  if (p.window != nullptr && tid < 64) {
    // accept length = the first r < W-1 with target[r] != window[r+1] (W-1 when every one matches): a ballot over
    // the lanes of wave 0 instead of a serial scan
    const bool miss = tid < p.W - 1 && tgt[tid] != win_s[tid + 1];
    const uint64_t m = __ballot(miss);
    const int a = m ? __builtin_ctzll(m) : p.W - 1;
    if (tid == 0) {
      if (p.accept_len) p.accept_len[b] = a;
      if (p.next_x0) p.next_x0[b] = tgt[a];
      if (p.packed) {
        p.packed[static_cast<int64_t>(b) * (p.W + 2) + 0] = win_s[0];
        p.packed[static_cast<int64_t>(b) * (p.W + 2) + 1] = a;
      }
    }
    if (p.packed && tid < p.W)
      p.packed[static_cast<int64_t>(b) * (p.W + 2) + 2 + tid] = tid <= a ? tgt[tid] : 0;
  }
  if (tid == 0) reset_counter(seq_counter(p.counters, b));
}

// Workspace layout: the arrival counters first (a fixed block, whatever bs, W and V are, so calls of different shapes
// can share one workspace), then the chunk winners.
constexpr size_t PARTS_OFFSET = COUNTER_BYTES;

size_t ws_bytes(int bs, int W, int V) {
  const size_t nc = (static_cast<size_t>(V) + CHUNK - 1) / CHUNK;
  const size_t parts = static_cast<size_t>(bs) * W * nc;
  return PARTS_OFFSET + parts * sizeof(uint64_t);
}

}  // namespace

// Pieces per workgroup: as many as keep about four workgroups per CU (one piece per workgroup for a single
// sequence's 17 rows, whose 255 workgroups already fill the chip once), at most 4.
static int pieces_per_chunk(int rows, int V) {
  const int pieces = (V + CHUNK - 1) / CHUNK;
  const int64_t units = static_cast<int64_t>(rows) * pieces;
  return units >= 4096 ? 4 : units >= 1024 ? 2 : 1;
}

static void launch_argmax(ArgParams& p, int dtype, int bs, int spc, hipStream_t st) {
  p.n_chunks = ((p.V + CHUNK - 1) / CHUNK + spc - 1) / spc;
  const dim3 grid(p.n_chunks, bs * p.W);
  const bool bf = dtype == GSS_BF16;
  switch (spc) {
    case 4:
      if (bf) hipLaunchKernelGGL((argmax_accept_kernel<uint16_t, 4>), grid, dim3(ARG_THREADS), 0, st, p);
      else hipLaunchKernelGGL((argmax_accept_kernel<float, 4>), grid, dim3(ARG_THREADS), 0, st, p);
      break;
    case 2:
      if (bf) hipLaunchKernelGGL((argmax_accept_kernel<uint16_t, 2>), grid, dim3(ARG_THREADS), 0, st, p);
      else hipLaunchKernelGGL((argmax_accept_kernel<float, 2>), grid, dim3(ARG_THREADS), 0, st, p);
      break;
    default:
      if (bf) hipLaunchKernelGGL((argmax_accept_kernel<uint16_t, 1>), grid, dim3(ARG_THREADS), 0, st, p);
      else hipLaunchKernelGGL((argmax_accept_kernel<float, 1>), grid, dim3(ARG_THREADS), 0, st, p);
  }
}

extern "C" int gss_argmax_workspace_size(int bs, int W, int V, size_t* bytes) {
  if (!bytes || bs <= 0 || W <= 0 || V <= 0) return GSS_ERR_ARG;
  if (W > MAX_W || V > MAX_CHUNKS * CHUNK) return GSS_ERR_UNSUPPORTED;
  *bytes = ws_bytes(bs, W, V);
  return GSS_OK;
}

extern "C" int gss_argmax_accept(const void* logits, int dtype, int64_t ld_row, int bs, int W, int V, int flags,
                                 const int32_t* window, int32_t* target, int32_t* accept_len, int32_t* next_x0,
                                 int32_t* packed, void* workspace, size_t workspace_bytes, gss_stream_t stream) {
  if (!logits || !target || bs <= 0 || W <= 0 || V <= 0 || ld_row < V) return GSS_ERR_ARG;
  if (dtype != GSS_BF16 && dtype != GSS_F32) return GSS_ERR_ARG;
  if (flags & ~(GSS_ARGMAX_SOFTMAX | GSS_ARGMAX_LAST_RAW)) return GSS_ERR_ARG;
  if (W > MAX_W || V > MAX_CHUNKS * CHUNK || bs > MAX_SEQ) return GSS_ERR_UNSUPPORTED;
  if (!workspace || workspace_bytes < ws_bytes(bs, W, V)) return GSS_ERR_WORKSPACE;
  ArgParams p;
  p.logits = logits;
  p.ld_row = ld_row;
  p.W = W;
  p.V = V;
  p.flags = flags;
  p.window = window;
  p.target = target;
  p.accept_len = accept_len;
  p.next_x0 = next_x0;
  p.packed = packed;
  p.counters = static_cast<uint32_t*>(workspace);
  p.part = reinterpret_cast<uint64_t*>(static_cast<char*>(workspace) + PARTS_OFFSET);
  launch_argmax(p, dtype, bs, pieces_per_chunk(bs * W, V), static_cast<hipStream_t>(stream));
  return gss_launch_status();
}

// ---------------------------------------------------------------- argmax + accept without allocation -----------
// gss_argmax_accept_noalloc: the same kernel on a scratch block compiled into the library, for callers that cannot
// allocate. `scratch` is a file-scope device array (each GPU holds its own copy for the life of the process); host
// code never passes its name to a kernel (in host code the name is a stand-in, not a device address): the device
// address comes from hipGetSymbolAddress, once per device, with that device current, and only that address is
// used. Layout: the arrival counters of NOALLOC_MAX_SEQ sequences, then the chunk winners of up to
// NOALLOC_MAX_SEQ * MAX_W rows of MAX_CHUNKS chunks (1,122,304 bytes in all).
namespace {
constexpr int NOALLOC_MAX_SEQ = 64;
constexpr size_t NOALLOC_COUNTER_BYTES = static_cast<size_t>(NOALLOC_MAX_SEQ) * (SUB + 1) * LINE_U32 * sizeof(uint32_t);
constexpr size_t NOALLOC_PART_BYTES = static_cast<size_t>(NOALLOC_MAX_SEQ) * MAX_W * MAX_CHUNKS * sizeof(uint64_t);
constexpr size_t NOALLOC_SCRATCH_BYTES = NOALLOC_COUNTER_BYTES + NOALLOC_PART_BYTES;
constexpr int NOALLOC_MAX_DEVICES = 64;
}  // namespace

static __device__ __align__(256) unsigned char scratch[NOALLOC_SCRATCH_BYTES];

namespace {

__global__ void __launch_bounds__(256) zero_words_kernel(uint32_t* p, size_t n) {
  for (size_t i = static_cast<size_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n;
       i += static_cast<size_t>(gridDim.x) * blockDim.x)
    p[i] = 0u;
}

std::mutex g_scratch_mu;
void* g_scratch_ptr[NOALLOC_MAX_DEVICES];  // device address of `scratch` on each device (null: not set up yet)

// The current device's scratch address. On the first call per device it is looked up and its arrival counters are
// cleared by a fill kernel on `st` (ordered before the caller's launch on the same stream; the kernels leave the
// counters at zero after every call, so this is the only clear).
int noalloc_scratch(hipStream_t st, void** out) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= NOALLOC_MAX_DEVICES) return GSS_ERR_LAUNCH;
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    void* ptr = nullptr;
    if (hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)) != hipSuccess || ptr == nullptr) return GSS_ERR_LAUNCH;
    hipLaunchKernelGGL(zero_words_kernel, dim3(16), dim3(256), 0, st, static_cast<uint32_t*>(ptr),
                       NOALLOC_COUNTER_BYTES / sizeof(uint32_t));
    if (gss_launch_status() != GSS_OK) return GSS_ERR_LAUNCH;
    g_scratch_ptr[dev] = ptr;
  }
  *out = g_scratch_ptr[dev];
  return GSS_OK;
}

}  // namespace

extern "C" int gss_argmax_accept_noalloc(const void* logits, int dtype, int64_t ld_row, int bs, int W, int V,
                                         int flags, const int32_t* window, int32_t* target, int32_t* accept_len,
                                         int32_t* next_x0, int32_t* packed, gss_stream_t stream) {
  if (!logits || !target || bs <= 0 || W <= 0 || V <= 0 || ld_row < V) return GSS_ERR_ARG;
  if (dtype != GSS_BF16 && dtype != GSS_F32) return GSS_ERR_ARG;
  if (flags & ~(GSS_ARGMAX_SOFTMAX | GSS_ARGMAX_LAST_RAW)) return GSS_ERR_ARG;
  if (W > MAX_W || V > MAX_CHUNKS * CHUNK || bs > NOALLOC_MAX_SEQ) return GSS_ERR_UNSUPPORTED;
  hipStream_t st = static_cast<hipStream_t>(stream);
  void* base = nullptr;
  const int rc = noalloc_scratch(st, &base);
  if (rc != GSS_OK) return rc;
  ArgParams p;
  p.logits = logits;
  p.ld_row = ld_row;
  p.W = W;
  p.V = V;
  p.flags = flags;
  p.window = window;
  p.target = target;
  p.accept_len = accept_len;
  p.next_x0 = next_x0;
  p.packed = packed;
  p.counters = static_cast<uint32_t*>(base);
  p.part = reinterpret_cast<uint64_t*>(static_cast<char*>(base) + NOALLOC_COUNTER_BYTES);
  launch_argmax(p, dtype, bs, pieces_per_chunk(bs * W, V), st);
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
  u32x4_t* part;        // [bs*W, n_chunks] (max bits, index, sum bits, 0)
  uint32_t* counters;   // arrival counters (see arrive_last)
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
    const float om = lane_xor(m, o);
    const int oi = lane_xor(mi, o);
    const float os = lane_xor(s, o);
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
    st_agent_x4(p.part + slot, u32x4_t{__float_as_uint(m), static_cast<uint32_t>(mi), __float_as_uint(s), 0u});
    wait_stores();
    const int r = row - b * p.W;
    is_last = arrive_last(p.counters, b, r * p.n_chunks + chunk, p.W * p.n_chunks);
  }
  __syncthreads();
  if (!is_last) return;

  // ---- phase 2: this workgroup finishes sequence b ------------------------------------------------------------
  // the chunk results of its W rows, one (row, chunk) per thread (coherent loads), then each row in chunk order
  __shared__ float cm_s[MAX_W * MAX_CHUNKS], cs_s[MAX_W * MAX_CHUNKS];
  __shared__ int ci_s[MAX_W * MAX_CHUNKS];
  __shared__ int rx[MAX_W];
  __shared__ float rc[MAX_W];
  __shared__ int blk_s[MAX_W];
  int32_t* blk = p.block + static_cast<int64_t>(b) * p.W;
  if (tid < p.W) blk_s[tid] = blk[tid];
  {
    const u32x4_t* base = p.part + static_cast<int64_t>(b) * p.W * p.n_chunks;
    const int n_items = p.W * p.n_chunks;
    for (int t0 = tid; t0 < n_items; t0 += 2 * ARG_THREADS) {  // two items per thread and memory round trip
      const int t1 = t0 + ARG_THREADS < n_items ? t0 + ARG_THREADS : t0;
      u32x4_t q0, q1, u2, u3;
      ld_agent_x4(2, base + t0, base + t1, nullptr, nullptr, q0, q1, u2, u3);
      cm_s[t0] = __uint_as_float(q0[0]);
      ci_s[t0] = static_cast<int>(q0[1]);
      cs_s[t0] = __uint_as_float(q0[2]);
      cm_s[t1] = __uint_as_float(q1[0]);
      ci_s[t1] = static_cast<int>(q1[1]);
      cs_s[t1] = __uint_as_float(q1[2]);
    }
  }
  __syncthreads();
  if (tid < p.W) {
    const int r0 = tid * p.n_chunks;
    float M = cm_s[r0], S = cs_s[r0];
    int I = ci_s[r0];
    for (int c = 1; c < p.n_chunks; ++c) merge_softmax(M, I, S, cm_s[r0 + c], ci_s[r0 + c], cs_s[r0 + c]);
    // a NaN or +inf in the row, or a row of -inf, makes the whole fp32 softmax NaN: argmax 0, probability NaN
    const bool finite_max = M == M && M != INFINITY && M != -INFINITY;
    rx[tid] = finite_max ? I : 0;
    rc[tid] = finite_max ? 1.f / S : __builtin_nanf("");
  }
  __syncthreads();
  if (tid < p.W) {
    const int src = tid > 0 ? tid - 1 : 0;
    if (p.x1_out) p.x1_out[static_cast<int64_t>(b) * p.W + tid] = rx[src];
    if (p.conf_out) p.conf_out[static_cast<int64_t>(b) * p.W + tid] = rc[src];
  }
  if (tid < 64) {
    // the unmask rule with one lane per position of wave 0: the forced position is the first argmax of conf over
    // the masked positions (-inf elsewhere; NaN as max), found by an xor-shuffle reduction under the same total
    // order; counts by ballot
    const int j = tid;
    const int src = j > 0 ? j - 1 : 0;
    const bool masked = j < p.W && blk_s[j] == p.mask_id;
    const float c = masked ? rc[src] : -INFINITY;
    float best = c;
    int bj = j < p.W ? j : 0x7fffffff;
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
      const float ob = lane_xor(best, o);
      const int oj = lane_xor(bj, o);
      if (beats(ob, oj, best, bj)) { best = ob; bj = oj; }
    }
    const bool un = masked && (c > p.threshold || j == bj);
    const int nv = un ? rx[src] : (j < p.W ? blk_s[j] : 0);
    if (un) blk[j] = nv;
    // a position unmasked to the mask id itself stays masked, as in the reference
    const uint64_t left = __ballot(j < p.W && nv == p.mask_id), unm = __ballot(un);
    if (j == 0) {
      if (p.n_unmasked) p.n_unmasked[b] = __popcll(unm);
      if (p.n_left) p.n_left[b] = __popcll(left);
      if (p.seed_out) p.seed_out[b] = rx[p.W - 1];
      reset_counter(seq_counter(p.counters, b));
    }
  }
}

size_t unmask_ws_bytes(int bs, int W, int V) {
  const size_t nc = (static_cast<size_t>(V) + CHUNK - 1) / CHUNK;
  const size_t parts = static_cast<size_t>(bs) * W * nc;
  return PARTS_OFFSET + parts * sizeof(u32x4_t);
}

}  // namespace

extern "C" int gss_unmask_workspace_size(int bs, int W, int V, size_t* bytes) {
  if (!bytes || bs <= 0 || W <= 0 || V <= 0) return GSS_ERR_ARG;
  if (W > MAX_W || V > MAX_CHUNKS * CHUNK) return GSS_ERR_UNSUPPORTED;
  *bytes = unmask_ws_bytes(bs, W, V);
  return GSS_OK;
}

extern "C" int gss_unmask_step(const void* logits, int dtype, int64_t ld_row, int bs, int W, int V, int32_t* block,
                               int mask_id, float threshold, int32_t* x1, float* conf, int32_t* n_unmasked,
                               int32_t* n_left, int32_t* seed, void* workspace, size_t workspace_bytes,
                               gss_stream_t stream) {
  if (!logits || !block || bs <= 0 || W <= 0 || V <= 0 || ld_row < V) return GSS_ERR_ARG;
  if (dtype != GSS_BF16 && dtype != GSS_F32) return GSS_ERR_ARG;
  if (W > MAX_W || V > MAX_CHUNKS * CHUNK || bs > MAX_SEQ) return GSS_ERR_UNSUPPORTED;
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
  p.counters = static_cast<uint32_t*>(workspace);
  p.part = reinterpret_cast<u32x4_t*>(static_cast<char*>(workspace) + PARTS_OFFSET);
  const dim3 grid(p.n_chunks, bs * W);
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (dtype == GSS_BF16)
    hipLaunchKernelGGL(unmask_step_kernel<uint16_t>, grid, dim3(ARG_THREADS), 0, st, p);
  else
    hipLaunchKernelGGL(unmask_step_kernel<float>, grid, dim3(ARG_THREADS), 0, st, p);
  return gss_launch_status();
}
