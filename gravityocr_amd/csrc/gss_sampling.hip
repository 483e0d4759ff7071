// Sampled (non-greedy) verify of the serving round: the logits processing AR decode applies to each verify row
// (penalties with the row's in-block tokens, logit_bias), AR's target distribution (temperature softmax, top-k /
// top-p / min-p) and speculative sampling of the deterministic draft chain, plus the plain draw a0 needs.
//
// penalize_kernel: grid (V chunks, bs * K rows); every element of row (b, r) gets the penalizers in the caller's
//   order with the state of the committed tokens plus the row's in-block tokens cand[b, 1..r] (read from LDS).
// sample_rows_kernel: one workgroup per row, the row's probabilities held in registers (thread t owns the EPT
//   consecutive tokens [t * EPT, (t + 1) * EPT)). Softmax of logits / T; the filters keep a prefix of the tokens
//   in descending probability, so the kept set is {p >= tau} for the smallest tau passing the filter's test,
//   found by a binary search over the fp32 bit patterns (about 30 block reductions of the count and mass of the tokens
//   above a candidate; flashinfer's min-p chain runs a second search for top-p above the top-k cut); renormalized. Verify mode: row j < K-1 tests its draft token cand[b, j + 1] against its coin
//   and draws its residual (the distribution without that token; the last row its full distribution) with the
//   sequence's uniform; the last of the K workgroups of a sequence resolves the chain (accept length, committed
//   targets, packed row, next seed). Sample mode (no cand): every row draws from its distribution with its own
//   uniform. A draw is the smallest index whose inclusive prefix sum exceeds u * total, prefix sums in index order
//   (per-thread chunks, then an ordered scan over the threads).
#include "gss_common.h"

namespace {

constexpr int PEN_THREADS = 256;
constexpr int PEN_PER_THREAD = 8;
constexpr int MAX_K = 64;
constexpr size_t COUNTER_STRIDE = 32;  // u32 per sequence counter (one 128-byte line each)
constexpr int SV_MAX_WAVES = 16;
constexpr uint32_t NARROW = 1u << 22;  // threshold search: full passes until [lo, hi] spans this many bit patterns
constexpr int CAND_MAX = 512;          // then up to this many candidate tokens, searched by one wave

enum { PEN_REPETITION = 1, PEN_PRESENCE = 2, PEN_FREQUENCY = 3, PEN_MIN_NEW_TOKENS = 4 };
enum { FILTER_NONE = 0, FILTER_JOINT = 1, FILTER_TORCH = 2, FILTER_FI_MIN_P = 3 };

struct PenParams {
  float* logits;
  int64_t ld_row;
  int K, V, n_order;
  int order[4];
  const int32_t* cand;
  const float *rep_cum, *rep_pen, *pres_cum, *pres_pen, *freq_cum, *freq_pen;
  const int32_t *len_out, *min_new;
  const float* stop_pen;
  const float* bias;
};

__global__ void __launch_bounds__(PEN_THREADS) penalize_kernel(PenParams p) {
  const int row = blockIdx.y, b = row / p.K, r = row % p.K;
  __shared__ int blk[MAX_K];
  if (threadIdx.x < r) blk[threadIdx.x] = p.cand[static_cast<int64_t>(b) * p.K + 1 + threadIdx.x];
  __syncthreads();
  // the output-length test only when min_new_tokens is one of the penalizers (then both arrays were checked)
  bool uses_min_new = false;
  for (int o = 0; o < p.n_order; ++o) uses_min_new |= p.order[o] == PEN_MIN_NEW_TOKENS;
  const bool min_new_on = uses_min_new && p.len_out[b] + r < p.min_new[b];
  float* lr = p.logits + static_cast<int64_t>(row) * p.ld_row;
  const int64_t sv = static_cast<int64_t>(b) * p.V;
  const int v0 = blockIdx.x * PEN_THREADS * PEN_PER_THREAD + threadIdx.x;
  for (int i = 0; i < PEN_PER_THREAD; ++i) {
    const int v = v0 + i * PEN_THREADS;
    if (v >= p.V) break;
    int cnt = 0;
    for (int t = 0; t < r; ++t) cnt += blk[t] == v;
    float x = lr[v];
    for (int o = 0; o < p.n_order; ++o) {
      switch (p.order[o]) {
        case PEN_REPETITION: {
          const float S = cnt ? p.rep_pen[b] : p.rep_cum[sv + v];
          x = x > 0.f ? x / S : x * S;
          break;
        }
        case PEN_PRESENCE: x -= cnt ? p.pres_pen[b] : p.pres_cum[sv + v]; break;
        case PEN_FREQUENCY: {
          float S = p.freq_cum[sv + v];
          for (int c = 0; c < cnt; ++c) S += p.freq_pen[b];  // one add per occurrence, in order
          x -= S;
          break;
        }
        default:
          if (min_new_on) x += p.stop_pen[sv + v];
          break;
      }
    }
    if (p.bias != nullptr) x += p.bias[sv + v];
    lr[v] = x;
  }
}

struct SvParams {
  const float* logits;
  int64_t ld_row;
  int K, V, mode;
  const float* temperature;  // [bs]
  const int32_t* top_k;      // [bs]
  const float* top_p;        // [bs]
  const float* min_p;        // [bs] or null
  const int32_t* cand;       // [bs, K] or null (sample mode)
  const float* coins;        // [bs, K] (verify)
  const float* u;            // [bs] (verify) or [bs, K] (sample)
  int32_t* sampled;          // [bs, K]
  int32_t* target;           // [bs, K] (verify) or null
  int32_t* accept_len;       // [bs] (verify) or null
  int32_t* next_x0;          // [bs] (verify) or null
  int32_t* packed;           // [bs, K + 2] (verify) or null
  uint32_t* part;            // [bs, K, 2] handoff (accept flag, draw)
  uint32_t* counters;        // [bs]
};

// Block sums in a fixed order (xor-shuffle within each wave, then the NW waves in order): every thread gets the
// result.
template <int NW>
GSS_DEV float block_sum_f(float v, float* red) {
  v = wave_sum(v);
  __syncthreads();
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
  __syncthreads();
  float s = red[0];
  for (int w = 1; w < NW; ++w) s += red[w];
  return s;
}

// Two block sums in one exchange (the count, exact below 2^24, and the mass of a threshold test).
template <int NW>
GSS_DEV float2 block_sum2(float a, float c, float2* red) {
  a = wave_sum(a);
  c = wave_sum(c);
  __syncthreads();
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = float2{a, c};
  __syncthreads();
  float2 s = red[0];
  for (int w = 1; w < NW; ++w) {
    s.x += red[w].x;
    s.y += red[w].y;
  }
  return s;
}

template <int NW>
GSS_DEV float block_max_f(float v, float* red) {
  v = wave_max(v);
  __syncthreads();
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
  __syncthreads();
  float m = red[0];
  for (int w = 1; w < NW; ++w) m = fmaxf(m, red[w]);
  return m;
}

// Inclusive-prefix draw over the weights q (thread t's EPT consecutive tokens): the smallest token whose prefix
// sum exceeds u * total; -1 when the weights are all zero.
template <int EPT, int NW>
GSS_DEV int draw(const float (&q)[EPT], float u, float* redf, float* scan) {
  const int tid = threadIdx.x;
  float c = 0.f;
#pragma unroll
  for (int e = 0; e < EPT; ++e) c += q[e];
  __syncthreads();
  scan[tid] = c;
  __syncthreads();
  // exclusive prefix of the thread sums in thread order (one pass by thread 0 of each wave over its 64, then waves)
  if ((tid & 63) == 0) {
    float s = 0.f;
    for (int i = 0; i < 64; ++i) {
      const float x = scan[tid + i];
      scan[tid + i] = s;
      s += x;
    }
    redf[tid >> 6] = s;
  }
  __syncthreads();
  float wave_base = 0.f, total = 0.f;
  for (int w = 0; w < NW; ++w) {
    if (w < (tid >> 6)) wave_base += redf[w];
    total += redf[w];
  }
  __shared__ int pick;
  if (tid == 0) pick = 0x7fffffff;
  __syncthreads();
  if (total > 0.f) {
    const float target = u * total;
    float run = wave_base + scan[tid];
    int hit = -1;
#pragma unroll
    for (int e = 0; e < EPT; ++e) {
      run += q[e];
      if (hit < 0 && q[e] > 0.f && run > target) hit = tid * EPT + e;
    }
    if (hit >= 0) atomicMin(&pick, hit);  // LDS atomic: the smallest index wins (order-independent)
  }
  __syncthreads();
  int r = pick == 0x7fffffff ? -1 : pick;
  if (r < 0 && total > 0.f) {
    // rounding left no prefix above the target: the last token with weight
    __shared__ int last;
    if (tid == 0) last = -1;
    __syncthreads();
    int mine = -1;
#pragma unroll
    for (int e = 0; e < EPT; ++e)
      if (q[e] > 0.f) mine = tid * EPT + e;
    if (mine >= 0) atomicMax(&last, mine);
    __syncthreads();
    r = last;
  }
  return r;
}

template <int EPT, int NTH>
__global__ void __launch_bounds__(NTH) sample_rows_kernel(SvParams p) {
  constexpr int NW = NTH / 64;
  const int row = blockIdx.x, b = row / p.K, j = row % p.K, tid = threadIdx.x;
  __shared__ float redf[NW];
  __shared__ float2 red2[NW];
  __shared__ float scan[NTH];
  __shared__ float pd_s;
  __shared__ float cand[CAND_MAX];  // threshold-search candidates
  __shared__ int cnt_w[NW];
  __shared__ uint32_t tau_s;
  const float* lr = p.logits + static_cast<int64_t>(row) * p.ld_row;
  const int v0 = tid * EPT;
  const float T = p.temperature[b];
  float pr[EPT];
  const bool vec = (p.ld_row & 3) == 0 && (reinterpret_cast<uintptr_t>(p.logits) & 15u) == 0;
#pragma unroll
  for (int e = 0; e < EPT; e += 4) {
    if (vec && v0 + e + 3 < p.V) {
      const floatx4_t q = *reinterpret_cast<const floatx4_t*>(lr + v0 + e);
#pragma unroll
      for (int i = 0; i < 4; ++i) pr[e + i] = q[i];
    } else {
#pragma unroll
      for (int i = 0; i < 4; ++i) pr[e + i] = v0 + e + i < p.V ? lr[v0 + e + i] : -INFINITY;
    }
  }

  if (!(T > 0.f)) {
    // temperature 0: a point mass at the row maximum (lowest index on ties)
    float m = -INFINITY;
    int mi = 0x7fffffff;
#pragma unroll
    for (int e = 0; e < EPT; ++e)
      if (pr[e] > m) { m = pr[e]; mi = v0 + e; }
    const float M = block_max_f<NW>(m, redf);
    __shared__ int am;
    if (tid == 0) am = 0x7fffffff;
    __syncthreads();
    if (m == M && mi < p.V) atomicMin(&am, mi);
    __syncthreads();
    const int a = am;
#pragma unroll
    for (int e = 0; e < EPT; ++e) pr[e] = v0 + e == a ? 1.f : 0.f;
  } else {
    // softmax of logits / T
    float m = -INFINITY;
#pragma unroll
    for (int e = 0; e < EPT; ++e) {
      pr[e] = pr[e] / T;
      m = fmaxf(m, pr[e]);
    }
    const float M = block_max_f<NW>(m, redf);
    float s = 0.f;
#pragma unroll
    for (int e = 0; e < EPT; ++e) {
      pr[e] = v0 + e < p.V ? expf(pr[e] - M) : 0.f;
      s += pr[e];
    }
    const float S = block_sum_f<NW>(s, redf);
    float pmax = 0.f;
#pragma unroll
    for (int e = 0; e < EPT; ++e) {
      pr[e] = pr[e] / S;
      pmax = fmaxf(pmax, pr[e]);
    }
    if (p.mode != FILTER_NONE) {
      const float PM = block_max_f<NW>(pmax, redf);
      const int k = p.top_k[b] <= 0 ? 0x7fffffff : p.top_k[b];  // top_k <= 0: no top-k cut
      const float tp = p.top_p[b];
      // smallest tau (fp32 bit pattern in [lo, bits(PM)]) whose strictly-greater count C and mass MS pass the
      // test; the tests are monotone in tau, so the kept tokens are exactly those with p >= tau. Full passes over
      // the row narrow [lo, hi] to at most NARROW bit patterns (half a binade). Past that, tokens above hi count
      // at every remaining tau (a constant count and mass, summed in the full passes' order) and tokens at or below
      // lo never do, so the tokens in (lo, hi] are compacted into LDS in token order and wave 0 finishes the search
      // over them alone (wave reductions, no workgroup barrier per step); more than CAND_MAX of them: more full
      // passes (and one more attempt). The candidate masses are added to the constant in a fixed order, so the test stays monotone and
      // the result deterministic.
      const uint32_t top = __float_as_uint(PM);
      auto search = [&](uint32_t lo, auto&& ok) {
        uint32_t hi = top;
        // the candidate compaction is attempted at NARROW and, when that leaves too many, once more at a 64 times
        // narrower range (the candidates shrink with the range: a flat row under top-p 0.95 leaves ~6000 at 2^22
        // and ~170 at 2^16 of its 59392 tokens)
        uint32_t narrow = NARROW;
        int attempts = 0;
#pragma unroll 1
        while (lo < hi) {
          if (attempts < 2 && hi - lo <= narrow) {
            ++attempts;
            narrow >>= 6;
            const float flo = __uint_as_float(lo), fhi = __uint_as_float(hi);
            float c = 0.f, ms = 0.f;
            int n = 0;
#pragma unroll
            for (int e = 0; e < EPT; ++e) {
              if (pr[e] > fhi) { c += 1.f; ms += pr[e]; }
              n += pr[e] > flo && !(pr[e] > fhi) ? 1 : 0;
            }
            const float2 cm = block_sum2<NW>(c, ms, red2);  // also orders the LDS reuse below after earlier reads
            // exclusive prefix of the candidate counts in thread order: within the wave, then the waves before it
            int incl = n;
#pragma unroll
            for (int o = 1; o < 64; o <<= 1) {
              const int t = __shfl_up(incl, o, 64);
              if ((tid & 63) >= o) incl += t;
            }
            if ((tid & 63) == 63) cnt_w[tid >> 6] = incl;
            __syncthreads();
            int off = incl - n, total = 0;
            for (int w = 0; w < NW; ++w) {
              const int t = cnt_w[w];
              off += w < (tid >> 6) ? t : 0;
              total += t;
            }
            if (total <= CAND_MAX) {  // workgroup-uniform
#pragma unroll
              for (int e = 0; e < EPT; ++e)
                if (pr[e] > flo && !(pr[e] > fhi)) cand[off++] = pr[e];
              __syncthreads();
              if (tid < 64) {
#pragma unroll 1
                while (lo < hi) {
                  const uint32_t mid = lo + (hi - lo) / 2;
                  const float tau = __uint_as_float(mid);
                  float cc = 0.f, mm = 0.f;
                  for (int q = tid; q < total; q += 64) {  // lane order, then the wave sum
                    const float x = cand[q];
                    if (x > tau) { cc += 1.f; mm += x; }
                  }
                  cc = wave_sum(cc);
                  mm = wave_sum(mm);
                  if (ok(static_cast<int>(cm.x + cc), cm.y + mm)) hi = mid; else lo = mid + 1;
                }
                if (tid == 0) tau_s = lo;
              }
              __syncthreads();
              lo = tau_s;
              __syncthreads();  // every thread has read tau_s (a later search writes it again)
              break;
            }
          }
          const uint32_t mid = lo + (hi - lo) / 2;
          const float tau = __uint_as_float(mid);
          float c = 0.f, ms = 0.f;
#pragma unroll
          for (int e = 0; e < EPT; ++e)
            if (pr[e] > tau) { c += 1.f; ms += pr[e]; }
          const float2 cm = block_sum2<NW>(c, ms, red2);
          if (ok(static_cast<int>(cm.x), cm.y)) hi = mid; else lo = mid + 1;
        }
        return lo;
      };
      float tau;
      if (p.mode == FILTER_FI_MIN_P) {
        // top-k renorm, then top-p on the renormalized mass: MS / Z1 < top_p with Z1 the mass the top-k cut keeps
        uint32_t t = search(0u, [&](int C, float) { return C < k; });
        if (tp < 1.f) {
          const float t1 = __uint_as_float(t);
          float z = 0.f;
#pragma unroll
          for (int e = 0; e < EPT; ++e) z += pr[e] >= t1 ? pr[e] : 0.f;
          const float Z1 = block_sum_f<NW>(z, redf);
          t = search(t, [&](int, float MS) { return MS / Z1 < tp; });
        }
        tau = __uint_as_float(t);
      } else if (p.mode == FILTER_JOINT) {
        tau = __uint_as_float(search(0u, [&](int C, float MS) { return C < k && (MS < tp || tp >= 1.f); }));
      } else {
        tau = __uint_as_float(search(0u, [&](int C, float MS) { return C < k && !(MS > tp); }));
      }
      // min-p: p >= min_p * max(p) (the ratio is the same on renormalized probabilities)
      if ((p.mode == FILTER_TORCH || p.mode == FILTER_FI_MIN_P) && p.min_p != nullptr && p.min_p[b] > 0.f)
        tau = fmaxf(tau, PM * p.min_p[b]);
      int keep_one = -1;
      if (p.mode == FILTER_TORCH && k == 1) {
        // rank-based top-1: only the lowest-index maximum (the tied maxima are ranked by index)
        __shared__ int am1;
        if (tid == 0) am1 = 0x7fffffff;
        __syncthreads();
#pragma unroll
        for (int e = EPT - 1; e >= 0; --e)
          if (pr[e] == PM && v0 + e < p.V) keep_one = v0 + e;
        if (keep_one >= 0) atomicMin(&am1, keep_one);
        __syncthreads();
        keep_one = am1;
      }
      float ks = 0.f;
#pragma unroll
      for (int e = 0; e < EPT; ++e) {
        const bool keep = keep_one >= 0 ? v0 + e == keep_one : pr[e] >= tau;
        pr[e] = keep ? pr[e] : 0.f;
        ks += pr[e];
      }
      const float KS = block_sum_f<NW>(ks, redf);
#pragma unroll
      for (int e = 0; e < EPT; ++e) pr[e] = pr[e] / KS;
    }
  }

  const bool verify = p.cand != nullptr;
  float u;
  if (verify) {
    u = p.u[b];
    if (j < p.K - 1) {
      const int d = p.cand[static_cast<int64_t>(b) * p.K + j + 1];
      if (tid == 0) pd_s = 0.f;
      __syncthreads();
#pragma unroll
      for (int e = 0; e < EPT; ++e)
        if (v0 + e == d) { pd_s = pr[e]; pr[e] = 0.f; }  // its target probability; removed from the residual
      __syncthreads();
    }
  } else {
    u = p.u[row];
  }
  const int tok = draw<EPT, NW>(pr, u, redf, scan);
  if (tid == 0) p.sampled[row] = tok;
  if (!verify) return;

  // hand the row's (accept, draw) to the last workgroup of the sequence
  __shared__ bool is_last;
  if (tid == 0) {
    const bool acc = j < p.K - 1 && p.coins[static_cast<int64_t>(b) * p.K + j] <= pd_s;
    st_agent(p.part + 2 * static_cast<int64_t>(row), acc ? 1u : 0u);
    st_agent(p.part + 2 * static_cast<int64_t>(row) + 1, static_cast<uint32_t>(tok));
    wait_stores();
    is_last = count_arrival(&p.counters[static_cast<int64_t>(b) * COUNTER_STRIDE]) == static_cast<uint32_t>(p.K - 1);
  }
  __syncthreads();
  if (!is_last) return;
  __shared__ uint32_t fl[MAX_K], tk[MAX_K];
  if (tid < p.K) {
    uint32_t a, t, unused;
    const uint32_t* base = p.part + 2 * (static_cast<int64_t>(b) * p.K + tid);
    ld_agent_u32(2, base, base + 1, nullptr, a, t, unused);
    fl[tid] = a;
    tk[tid] = t;
  }
  __syncthreads();
  if (tid < 64) {
    // accept length = the first row whose draft token was rejected (K-1 when none was)
    const bool miss = tid < p.K - 1 && fl[tid] == 0u;
    const uint64_t mk = __ballot(miss);
    const int acc = mk ? __builtin_ctzll(mk) : p.K - 1;
    const int64_t cb = static_cast<int64_t>(b) * p.K;
    const int t_r = tid < acc ? p.cand[cb + tid + 1] : static_cast<int>(tk[tid < p.K ? tid : 0]);
    if (tid < p.K && p.target) p.target[cb + tid] = t_r;
    if (tid == 0) {
      if (p.accept_len) p.accept_len[b] = acc;
      if (p.next_x0) p.next_x0[b] = static_cast<int>(tk[acc]);
      if (p.packed) {
        p.packed[static_cast<int64_t>(b) * (p.K + 2)] = p.cand[cb];
        p.packed[static_cast<int64_t>(b) * (p.K + 2) + 1] = acc;
      }
    }
    if (p.packed && tid < p.K) p.packed[static_cast<int64_t>(b) * (p.K + 2) + 2 + tid] = tid <= acc ? t_r : 0;
    if (tid == 0) reset_counter(&p.counters[static_cast<int64_t>(b) * COUNTER_STRIDE]);
  }
}

size_t sv_ws_bytes(int bs, int K) {
  return static_cast<size_t>(bs) * COUNTER_STRIDE * sizeof(uint32_t) + static_cast<size_t>(bs) * K * 2 * sizeof(uint32_t);
}

// Grammar vocabulary mask: logits[r, v] = -inf where bit v % 32 of word v / 32 of row r's mask is clear. One thread
// per mask word (32 tokens); rows in blockIdx.y.
constexpr int MASK_THREADS = 256;
__global__ void __launch_bounds__(MASK_THREADS) vocab_mask_kernel(float* logits, int64_t ld_row, int V,
                                                                  const int32_t* mask, int64_t ld_mask) {
  const int w = blockIdx.x * MASK_THREADS + threadIdx.x, r = blockIdx.y;
  if (w * 32 >= V) return;
  const uint32_t bits = static_cast<uint32_t>(mask[r * ld_mask + w]);
  if (bits == 0xffffffffu) return;
  float* row = logits + r * ld_row + w * 32;
  const int n = min(32, V - w * 32);
  for (int i = 0; i < n; ++i)
    if (!((bits >> i) & 1u)) row[i] = -INFINITY;
}

}  // namespace

extern "C" int gss_apply_vocab_mask(float* logits, int64_t ld_row, int rows, int V, const int32_t* mask,
                                    int64_t ld_mask, gss_stream_t stream) {
  if (!logits || !mask || rows <= 0 || V <= 0 || ld_row < V || ld_mask < (V + 31) / 32) return GSS_ERR_ARG;
  if (rows > 65535) return GSS_ERR_UNSUPPORTED;
  const dim3 grid(((V + 31) / 32 + MASK_THREADS - 1) / MASK_THREADS, rows);
  hipLaunchKernelGGL(vocab_mask_kernel, grid, dim3(MASK_THREADS), 0, static_cast<hipStream_t>(stream), logits, ld_row,
                     V, mask, ld_mask);
  return gss_launch_status();
}

extern "C" int gss_penalize_rows(float* logits, int64_t ld_row, int bs, int K, int V, const int32_t* cand,
                                 const gss_penalties* pen, gss_stream_t stream) {
  if (!logits || !cand || !pen || bs <= 0 || K <= 0 || V <= 0 || ld_row < V) return GSS_ERR_ARG;
  if (K > MAX_K || pen->n_order < 0 || pen->n_order > 4) return GSS_ERR_ARG;
  PenParams p;
  p.logits = logits;
  p.ld_row = ld_row;
  p.K = K;
  p.V = V;
  p.n_order = pen->n_order;
  p.cand = cand;
  for (int o = 0; o < 4; ++o) p.order[o] = o < pen->n_order ? pen->order[o] : 0;
  p.rep_cum = pen->rep_cum;
  p.rep_pen = pen->rep_pen;
  p.pres_cum = pen->pres_cum;
  p.pres_pen = pen->pres_pen;
  p.freq_cum = pen->freq_cum;
  p.freq_pen = pen->freq_pen;
  p.len_out = pen->len_out;
  p.min_new = pen->min_new;
  p.stop_pen = pen->stop_pen;
  p.bias = pen->logit_bias;
  for (int o = 0; o < p.n_order; ++o) {
    switch (p.order[o]) {
      case PEN_REPETITION: if (!p.rep_cum || !p.rep_pen) return GSS_ERR_ARG; break;
      case PEN_PRESENCE: if (!p.pres_cum || !p.pres_pen) return GSS_ERR_ARG; break;
      case PEN_FREQUENCY: if (!p.freq_cum || !p.freq_pen) return GSS_ERR_ARG; break;
      case PEN_MIN_NEW_TOKENS: if (!p.len_out || !p.min_new || !p.stop_pen) return GSS_ERR_ARG; break;
      default: return GSS_ERR_ARG;
    }
  }
  const dim3 grid((V + PEN_THREADS * PEN_PER_THREAD - 1) / (PEN_THREADS * PEN_PER_THREAD), bs * K);
  hipLaunchKernelGGL(penalize_kernel, grid, dim3(PEN_THREADS), 0, static_cast<hipStream_t>(stream), p);
  return gss_launch_status();
}

extern "C" int gss_sample_workspace_size(int bs, int K, size_t* bytes) {
  if (!bytes || bs <= 0 || K <= 0) return GSS_ERR_ARG;
  *bytes = sv_ws_bytes(bs, K);
  return GSS_OK;
}

extern "C" int gss_sample_rows(const float* logits, int64_t ld_row, int bs, int K, int V, int filter,
                               const float* temperature, const int32_t* top_k, const float* top_p, const float* min_p,
                               const int32_t* cand, const float* coins, const float* uniforms, int32_t* sampled,
                               int32_t* target, int32_t* accept_len, int32_t* next_x0, int32_t* packed,
                               void* workspace, size_t workspace_bytes, gss_stream_t stream) {
  if (!logits || !temperature || !uniforms || !sampled || bs <= 0 || K <= 0 || V <= 0 || ld_row < V)
    return GSS_ERR_ARG;
  if (filter < FILTER_NONE || filter > FILTER_FI_MIN_P) return GSS_ERR_ARG;
  if (filter != FILTER_NONE && (!top_k || !top_p)) return GSS_ERR_ARG;
  if (cand && !coins) return GSS_ERR_ARG;
  if (K > MAX_K) return GSS_ERR_UNSUPPORTED;
  if (cand && (!workspace || workspace_bytes < sv_ws_bytes(bs, K))) return GSS_ERR_WORKSPACE;
  SvParams p;
  p.logits = logits;
  p.ld_row = ld_row;
  p.K = K;
  p.V = V;
  p.mode = filter;
  p.temperature = temperature;
  p.top_k = top_k;
  p.top_p = top_p;
  p.min_p = min_p;
  p.cand = cand;
  p.coins = coins;
  p.u = uniforms;
  p.sampled = sampled;
  p.target = target;
  p.accept_len = accept_len;
  p.next_x0 = next_x0;
  p.packed = packed;
  p.counters = static_cast<uint32_t*>(workspace);
  p.part = p.counters ? p.counters + static_cast<size_t>(bs) * COUNTER_STRIDE : nullptr;
  hipStream_t st = static_cast<hipStream_t>(stream);
  const dim3 grid(bs * K);
  if (V <= 512 * 8)
    hipLaunchKernelGGL((sample_rows_kernel<8, 512>), grid, dim3(512), 0, st, p);
  else if (V <= 512 * 32)
    hipLaunchKernelGGL((sample_rows_kernel<32, 512>), grid, dim3(512), 0, st, p);
  else if (V <= 1024 * 64)
    hipLaunchKernelGGL((sample_rows_kernel<64, 1024>), grid, dim3(1024), 0, st, p);
  else
    return GSS_ERR_UNSUPPORTED;
  return gss_launch_status();
}
