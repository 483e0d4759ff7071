// Integer bookkeeping at the serving boundary, in SGLang's buffer types: the round's commit (packed readback row,
// seed-pool update, seq_lens, compacted free list of rejected verify slots) and the flattened KV index list of a
// batch. Both are one wavefront per sequence; the per-sequence offsets are prefix sums each wavefront computes over
// the sequences before it (bs is small), so there is no second launch and no inter-workgroup communication.
#include "gss_common.h"

namespace {

// Sum of v over lanes (int64), fixed xor-shuffle order.
GSS_DEV int64_t wave_sum_i64(int64_t v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    const int lo = __shfl_xor(static_cast<int>(v & 0xffffffff), o, 64);
    const int hi = __shfl_xor(static_cast<int>(v >> 32), o, 64);
    v += (static_cast<int64_t>(hi) << 32) | static_cast<uint32_t>(lo);
  }
  return v;
}

struct CommitParams {
  const int32_t* predict;  // [bs*K (+1)]  verify argmax rows
  const int32_t* acc;      // [bs]
  const int64_t* a0;       // a0 of row i at a0[i * a0_stride]
  int64_t a0_stride;
  const int64_t* rpi;      // [bs] request pool index of each row
  int64_t* seeds;          // [pool] seed (next boundary token) of every request slot
  int64_t* seq_lens;       // [bs] += acc + 1
  const int64_t* loc;      // [bs*K] KV slots the verify rows were written to
  int32_t* packed;         // [bs, K+2]
  int64_t* free_slots;     // [bs*K] rejected slots, compacted in row order
  int64_t* out;            // [bs] next seeds
  int K;
  int64_t n_seeds;         // seed pool size (rows with rpi outside [0, n_seeds) do not write it)
};

__global__ void __launch_bounds__(64) ss_commit_kernel(CommitParams p) {
  const int i = blockIdx.x, j = threadIdx.x, K = p.K;
  // rejected slots of the rows before i
  int64_t prev = 0;
  // accept lengths are clamped into [0, K-1] wherever they are read, so every index below stays in its row
  for (int r = j; r < i; r += 64) prev += K - 1 - min(max(p.acc[r], 0), K - 1);
  prev = wave_sum_i64(prev);
  const int a = min(max(p.acc[i], 0), K - 1);
  int32_t* row = p.packed + static_cast<int64_t>(i) * (K + 2);
  if (j < K) row[2 + j] = j <= a ? p.predict[static_cast<int64_t>(i) * K + j] : 0;
  if (j == 0) {
    row[0] = static_cast<int32_t>(p.a0[static_cast<int64_t>(i) * p.a0_stride]);
    row[1] = a;
    const int64_t seed = p.predict[static_cast<int64_t>(i) * K + a];
    const int64_t r = p.rpi[i];
    if (r >= 0 && r < p.n_seeds) p.seeds[r] = seed;
    p.out[i] = seed;
    p.seq_lens[i] += a + 1;
  }
  if (j < K && j > a) p.free_slots[prev + (j - a - 1)] = p.loc[static_cast<int64_t>(i) * K + j];
}

struct MetaParams {
  const int32_t* req_to_token;  // [pool, r2t_stride] KV slot of every token of every request slot
  int64_t r2t_stride;
  const int64_t* rpi;           // [bs]
  const int64_t* seq_lens;      // [bs]
  int extra;                    // window rows appended after each sequence's committed tokens
  int32_t* kv_indptr;           // [bs + 1]
  int32_t* kv_indices;          // [sum(seq_lens + extra)]
  int64_t n_req;                // rows of req_to_token
  int64_t cap;                  // capacity of kv_indices (entries past it are not written)
};

__global__ void __launch_bounds__(256) kv_meta_kernel(MetaParams p) {
  const int i = blockIdx.x, t = threadIdx.x;
  // entries of row r: seq_lens[r] + extra, clamped into [0, r2t_stride] (a row holds at most r2t_stride tokens)
  auto row_len = [&](int r) { return min(max(p.seq_lens[r] + p.extra, int64_t{0}), p.r2t_stride); };
  __shared__ int64_t part[4];
  int64_t prev = 0;
  for (int r = t; r < i; r += blockDim.x) prev += row_len(r);
  prev = wave_sum_i64(prev);
  if ((t & 63) == 0) part[t >> 6] = prev;
  __syncthreads();
  prev = 0;
  for (int w = 0; w < static_cast<int>(blockDim.x >> 6); ++w) prev += part[w];
  const int64_t start = prev;
  const int64_t n = row_len(i);
  if (t == 0) {
    if (i == 0) p.kv_indptr[0] = 0;
    p.kv_indptr[i + 1] = static_cast<int32_t>(start + n);
  }
  const int64_t r = p.rpi[i];
  if (r < 0 || r >= p.n_req) return;
  const int32_t* src = p.req_to_token + r * p.r2t_stride;
  for (int64_t k = t; k < n && start + k < p.cap; k += blockDim.x) p.kv_indices[start + k] = src[k];
}

// Round history on the device: row min(*ctr, capacity - 1) of up to three logs receives the current contents of
// their source rows, then *ctr advances by one. One workgroup; every thread reads the counter before the barrier
// that precedes its update.
struct LogParams {
  int64_t* ctr;
  int capacity;
  const int32_t* src[3];
  int32_t* log[3];
  int len[3];
};

__global__ void __launch_bounds__(256) log_append_kernel(LogParams p) {
  const int64_t c = *p.ctr;
  const int64_t li = c < 0 ? 0 : (c < p.capacity ? c : p.capacity - 1);
#pragma unroll
  for (int s = 0; s < 3; ++s) {
    if (p.src[s] == nullptr) continue;
    int32_t* dst = p.log[s] + li * p.len[s];
    for (int i = threadIdx.x; i < p.len[s]; i += blockDim.x) dst[i] = p.src[s][i];
  }
  __syncthreads();
  if (threadIdx.x == 0) *p.ctr = c + 1;
}

}  // namespace

extern "C" int gss_ss_commit(const int32_t* predict, const int32_t* accept_len, const int64_t* a0, int64_t a0_stride,
                             const int64_t* req_pool_indices, int64_t* seeds, int64_t* seq_lens, const int64_t* loc,
                             int32_t* packed, int64_t* free_slots, int64_t* out, int64_t n_seeds, int bs, int K,
                             gss_stream_t stream) {
  if (!predict || !accept_len || !a0 || !req_pool_indices || !seeds || !seq_lens || !loc || !packed ||
      !free_slots || !out)
    return GSS_ERR_ARG;
  if (bs <= 0 || K <= 0 || a0_stride <= 0 || n_seeds <= 0) return GSS_ERR_ARG;
  if (K > 64) return GSS_ERR_UNSUPPORTED;
  CommitParams p{predict, accept_len, a0, a0_stride, req_pool_indices, seeds, seq_lens, loc, packed, free_slots, out, K,
                 n_seeds};
  hipLaunchKernelGGL(ss_commit_kernel, dim3(bs), dim3(64), 0, static_cast<hipStream_t>(stream), p);
  return gss_launch_status();
}

extern "C" int gss_kv_meta(const int32_t* req_to_token, int64_t r2t_stride, int64_t n_req,
                           const int64_t* req_pool_indices, const int64_t* seq_lens, int extra, int32_t* kv_indptr,
                           int32_t* kv_indices, int64_t kv_indices_cap, int bs, gss_stream_t stream) {
  if (!req_to_token || !req_pool_indices || !seq_lens || !kv_indptr || !kv_indices) return GSS_ERR_ARG;
  if (bs <= 0 || extra < 0 || r2t_stride <= 0 || n_req <= 0 || kv_indices_cap < 0) return GSS_ERR_ARG;
  MetaParams p{req_to_token, r2t_stride, req_pool_indices, seq_lens, extra, kv_indptr, kv_indices, n_req,
               kv_indices_cap};
  hipLaunchKernelGGL(kv_meta_kernel, dim3(bs), dim3(256), 0, static_cast<hipStream_t>(stream), p);
  return gss_launch_status();
}

extern "C" int gss_log_append(int64_t* ctr, int capacity, const int32_t* src0, int32_t* log0, int len0,
                              const int32_t* src1, int32_t* log1, int len1, const int32_t* src2, int32_t* log2,
                              int len2, gss_stream_t stream) {
  if (!ctr || capacity <= 0) return GSS_ERR_ARG;
  LogParams p{ctr, capacity, {src0, src1, src2}, {log0, log1, log2}, {len0, len1, len2}};
  for (int s = 0; s < 3; ++s) {
    if (p.src[s] == nullptr) continue;
    if (p.log[s] == nullptr || p.len[s] <= 0) return GSS_ERR_ARG;
  }
  hipLaunchKernelGGL(log_append_kernel, dim3(1), dim3(256), 0, static_cast<hipStream_t>(stream), p);
  return gss_launch_status();
}
