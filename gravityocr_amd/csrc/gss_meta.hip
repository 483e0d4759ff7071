// Integer bookkeeping at the serving boundary, in SGLang's buffer types: the round's commit (packed readback row,
// seed-pool update, the finish rule's cut index, seq_lens, compacted free list of the verify slots no kept token
// needs) and the flattened KV index list of a batch. Both are one wavefront per sequence; the per-sequence offsets are prefix sums each wavefront computes over
// the sequences before it (bs is small), so there is no second launch and no inter-workgroup communication.
#include "gss_common.h"

namespace {

// Sum of v over lanes (int64), fixed xor-shuffle order.
GSS_DEV int64_t wave_sum_i64(int64_t v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    const int lo = lane_xor(static_cast<int>(v & 0xffffffff), o);
    const int hi = lane_xor(static_cast<int>(v >> 32), o);
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
  int64_t* seq_lens;       // [bs] += j (j = acc + 1 without a finish rule)
  const int64_t* loc;      // [bs*K] KV slots the verify rows were written to
  int32_t* packed;         // [bs, K+2]
  int64_t* free_slots;     // [bs*K] slots of whole pages past every row's kept rows, compacted in row order
  int64_t* out;            // [bs] next seeds
  int K;
  int64_t n_seeds;         // seed pool size (rows with rpi outside [0, n_seeds) do not write it)
  int page;                // KV page size of the slots (1: every rejected slot is freed)
  // finish rule (budget == nullptr: none, every committed token is kept)
  const int32_t* budget;   // [bs] tokens the request may still emit; < 0: its finish needs the per-token path
  const int32_t* stop_ids; // [bs, n_stop] ids that stop each request (negative = padding)
  int n_stop;
  const int32_t* vocab;    // [bs] ids above it (or negative) end the request at the vocabulary boundary
  int32_t* cut;            // [bs] out (optional): j, the index of the last committed token of T
  int32_t* n_free;         // [1] out (optional): entries written to free_slots
};

// Cut index j of row r (T = [a0, t_0 .. t_a], a + 2 tokens: T[:j + 1] is committed, the KV of verify rows 0 .. j - 1
// is kept). The closed form of appending T one token at a time and stopping after the first token that exhausts
// the budget, is a stop id or lies outside [0, vocab]: j = the first such t, at most lim = min(a + 1,
// max(budget - 1, 0)). Without a rule (or for a request marked for the per-token path) j = a + 1. One lane.
GSS_DEV int row_cut(const CommitParams& p, int r, int a) {
  if (p.budget == nullptr || p.budget[r] < 0) return a + 1;
  const int lim = min(a + 1, max(p.budget[r] - 1, 0));
  const int32_t* stop = p.stop_ids + static_cast<int64_t>(r) * p.n_stop;
  const int vmax = p.vocab[r];
  for (int t = 0; t < lim; ++t) {
    const int32_t x = t == 0 ? static_cast<int32_t>(p.a0[static_cast<int64_t>(r) * p.a0_stride])
                             : p.predict[static_cast<int64_t>(r) * p.K + t - 1];
    bool ends = x < 0 || x > vmax;
    for (int k = 0; k < p.n_stop && !ends; ++k) ends = stop[k] == x;
    if (ends) return t;
  }
  return lim;
}

// Freed slots of row r: the verify rows j .. K-1 hold no kept token, but the ones that share a page with the kept
// rows stay allocated (the next round writes its rows into that page). Slots are page-aligned (slot % page ==
// position % page), so the rejected rows inside the last kept page are the (page - loc[j] % page) % page rows from
// row j on. The freed rows are the last c of the row.
GSS_DEV int row_freed(const CommitParams& p, int r, int j) {
  if (j >= p.K) return 0;
  const int64_t s = p.loc[static_cast<int64_t>(r) * p.K + j];
  const int in_page = static_cast<int>((p.page - s % p.page) % p.page);
  return max(0, p.K - j - in_page);
}

__global__ void __launch_bounds__(64) ss_commit_kernel(CommitParams p, int bs) {
  const int i = blockIdx.x, lane = threadIdx.x, K = p.K;
  // accept lengths are clamped into [0, K-1] wherever they are read, so every index below stays in its row
  auto acc_of = [&](int r) { return min(max(p.acc[r], 0), K - 1); };
  // freed slots of the rows before i (each lane takes rows lane, lane + 64, ...)
  int64_t prev = 0;
  for (int r = lane; r < i; r += 64) prev += row_freed(p, r, row_cut(p, r, acc_of(r)));
  prev = wave_sum_i64(prev);
  const int a = acc_of(i);
  const int j = row_cut(p, i, a);
  const int c = row_freed(p, i, j);
  int32_t* row = p.packed + static_cast<int64_t>(i) * (K + 2);
  if (lane < K) row[2 + lane] = lane <= a ? p.predict[static_cast<int64_t>(i) * K + lane] : 0;
  if (lane == 0) {
    row[0] = static_cast<int32_t>(p.a0[static_cast<int64_t>(i) * p.a0_stride]);
    row[1] = a;
    const int64_t seed = p.predict[static_cast<int64_t>(i) * K + a];
    const int64_t r = p.rpi[i];
    if (r >= 0 && r < p.n_seeds) p.seeds[r] = seed;
    p.out[i] = seed;
    p.seq_lens[i] += j;
    if (p.cut) p.cut[i] = j;
    if (p.n_free && i == bs - 1) *p.n_free = static_cast<int32_t>(prev + c);
  }
  if (lane < c) p.free_slots[prev + lane] = p.loc[static_cast<int64_t>(i) * K + (K - c) + lane];
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
                             int page, const gss_finish_rule* finish, int32_t* cut, int32_t* n_free,
                             gss_stream_t stream) {
  if (!predict || !accept_len || !a0 || !req_pool_indices || !seeds || !seq_lens || !loc || !packed ||
      !free_slots || !out)
    return GSS_ERR_ARG;
  if (bs <= 0 || K <= 0 || a0_stride <= 0 || n_seeds <= 0 || page <= 0) return GSS_ERR_ARG;
  if (finish && (!finish->budget || !finish->vocab || finish->n_stop < 0 || (finish->n_stop > 0 && !finish->stop_ids)))
    return GSS_ERR_ARG;
  if (K > 64) return GSS_ERR_UNSUPPORTED;
  CommitParams p{predict, accept_len, a0, a0_stride, req_pool_indices, seeds, seq_lens, loc, packed, free_slots, out, K,
                 n_seeds, page};
  if (finish) {
    p.budget = finish->budget;
    p.stop_ids = finish->stop_ids;
    p.n_stop = finish->n_stop;
    p.vocab = finish->vocab;
  }
  p.cut = cut;
  p.n_free = n_free;
  hipLaunchKernelGGL(ss_commit_kernel, dim3(bs), dim3(64), 0, static_cast<hipStream_t>(stream), p, bs);
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
