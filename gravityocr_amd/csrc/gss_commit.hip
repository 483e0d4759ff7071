// (d) KV commit: write the accepted window rows' K/V of every layer into the paged cache, advance the committed
// length, report the slot of every committed row. Rejected rows are never written (discarded in place).
//
// Grid (n_layers * n_pb, bs): workgroup (layer, pb) of sequence b owns the pb-th 16-token page that the committed
// rows touch (pages base/16 + pb, n_pb = ceil((W + 15) / 16) covers every alignment of the window). It copies
// the rows of all Hkv heads that fall into that page: K pages are token-major ([page][head][token][D], one 16-byte
// store per 8 dims), V pages token-minor ([page][head][D][16]): the V rows go through LDS so that consecutive
// lanes store consecutive tokens of one dim. A workgroup's dependent chain is two memory round trips (the length,
// then the page id with the rows). The committed length of sequence b is read by every workgroup of b and advanced
// by the last of them to count itself in (agent-scope atomic counter in the workspace, reset afterwards).
#include "gss_common.h"

namespace {

constexpr int COMMIT_THREADS = 512;
constexpr int CPAGE = 16;         // tokens per page
constexpr int VROW_PAD = 2;       // bf16 elements of padding per staged V row (bank spread)
constexpr int MAX_LDS = 65536;  // dynamic LDS without an attribute

struct CommitParams {
  const uint16_t* k_win;
  const uint16_t* v_win;
  int64_t win_layer_stride;
  uint16_t* k_pages;
  uint16_t* v_pages;
  int64_t page_layer_stride;
  const int32_t* page_table;
  int pt_stride;
  int32_t* seq_lens;
  const int32_t* n_rows;
  int n_add;
  int32_t* slots;
  int W, n_layers, n_pb, Hkv, D;
  uint32_t* counters;
};

__global__ void __launch_bounds__(COMMIT_THREADS) kv_commit_kernel(CommitParams p) {
  extern __shared__ uint16_t vstage[];  // [Hkv][16][D + VROW_PAD]
  const int layer = blockIdx.x / p.n_pb, pb = blockIdx.x % p.n_pb, b = blockIdx.y, tid = threadIdx.x;
  const int base = p.seq_lens[b];
  int n = (p.n_rows ? p.n_rows[b] : 0) + p.n_add;
  n = min(max(n, 0), p.W);
  const int cap = p.pt_stride * CPAGE;  // positions the page-table row can address
  const int32_t* pt = p.page_table + static_cast<int64_t>(b) * p.pt_stride;
  // rows j in [jlo, jhi) land in page pg at token offsets t = base + j - p0
  const int pg = (base >= 0 ? base / CPAGE : 0) + pb, p0 = pg * CPAGE;
  const int jlo = max(0, p0 - base), jhi = min(min(n, p0 + CPAGE - base), cap - base);
  if (base >= 0 && jlo < jhi) {
    const int64_t page = pt[pg];
    const int parts = p.D / 8, DS = p.D + VROW_PAD;
    const int nr = jhi - jlo, t0 = base + jlo - p0;
    const int64_t row0 = static_cast<int64_t>(b) * p.W + jlo;
    const uint16_t* kw = p.k_win + layer * p.win_layer_stride;
    const uint16_t* vw = p.v_win + layer * p.win_layer_stride;
    uint16_t* kp = p.k_pages + layer * p.page_layer_stride + page * p.Hkv * CPAGE * p.D;
    uint16_t* vp = p.v_pages + layer * p.page_layer_stride + page * p.Hkv * CPAGE * p.D;
    // K: chunk c = (row i, head h, part) straight to its slot; V: the same chunk into LDS
    const int n_chunks = nr * p.Hkv * parts;
    for (int c = tid; c < n_chunks; c += COMMIT_THREADS) {
      const int i = c / (p.Hkv * parts), rem = c % (p.Hkv * parts);
      const int h = rem / parts, part = rem % parts;
      const int64_t src = ((row0 + i) * p.Hkv + h) * p.D + part * 8;
      const u32x4_t kv = *reinterpret_cast<const u32x4_t*>(kw + src);
      const u32x4_t vv = *reinterpret_cast<const u32x4_t*>(vw + src);
      *reinterpret_cast<u32x4_t*>(kp + (static_cast<int64_t>(h) * CPAGE + t0 + i) * p.D + part * 8) = kv;
      uint16_t* dst = vstage + (h * CPAGE + i) * DS + part * 8;
#pragma unroll
      for (int e = 0; e < 4; ++e) *reinterpret_cast<uint32_t*>(dst + 2 * e) = vv[e];
    }
    __syncthreads();
    // V: element (h, d, t) of the page at (h * D + d) * 16 + t; a thread keeps one token t (the stride is a multiple
    // of 16), so lanes t0 .. t0 + nr - 1 of every 16 store and consecutive lanes write consecutive tokens
    const int t = tid % CPAGE, i = t - t0;
    if (i >= 0 && i < nr) {
      for (int h = 0; h < p.Hkv; ++h) {
        const uint16_t* srow = vstage + (h * CPAGE + i) * DS;
        uint16_t* dcol = vp + static_cast<int64_t>(h) * p.D * CPAGE + t;
        for (int d = tid / CPAGE; d < p.D; d += COMMIT_THREADS / CPAGE) dcol[d * CPAGE] = srow[d];
      }
    }
  }
  if (blockIdx.x == 0 && p.slots != nullptr) {
    for (int j = tid; j < p.W; j += COMMIT_THREADS) {
      const int pos = base + j;
      p.slots[static_cast<int64_t>(b) * p.W + j] =
          (j < n && pos >= 0 && pos < cap) ? pt[pos / CPAGE] * CPAGE + pos % CPAGE : -1;
    }
  }
  // the last workgroup of sequence b advances its length: every workgroup has read `base` (its addresses depend on
  // it) before it counts itself, and the new length is read only by later kernels
  __syncthreads();
  if (tid == 0 && count_arrival(&p.counters[b]) == static_cast<uint32_t>(gridDim.x - 1)) {
    p.seq_lens[b] = base + n;
    reset_counter(&p.counters[b]);
  }
}

}  // namespace

extern "C" int gss_kv_commit_workspace_size(int bs, size_t* bytes) {
  if (!bytes || bs <= 0) return GSS_ERR_ARG;
  *bytes = static_cast<size_t>(bs) * sizeof(uint32_t);
  return GSS_OK;
}

extern "C" int gss_kv_commit(const void* k_win, const void* v_win, int64_t win_layer_stride, void* k_pages,
                             void* v_pages, int64_t page_layer_stride, const int32_t* page_table, int pt_stride,
                             int32_t* seq_lens, const int32_t* n_rows, int n_add, int32_t* slots, int bs, int W,
                             int n_layers, int Hkv, int D, int page, void* workspace, size_t workspace_bytes,
                             gss_stream_t stream) {
  if (!k_win || !v_win || !k_pages || !v_pages || !page_table || !seq_lens) return GSS_ERR_ARG;
  if (bs <= 0 || W <= 0 || n_layers <= 0 || Hkv <= 0 || pt_stride <= 0) return GSS_ERR_ARG;
  if (D % 8 != 0 || page != CPAGE) return GSS_ERR_UNSUPPORTED;
  const size_t lds = static_cast<size_t>(Hkv) * CPAGE * (D + VROW_PAD) * sizeof(uint16_t);
  if (lds > MAX_LDS) return GSS_ERR_UNSUPPORTED;
  if (win_layer_stride < static_cast<int64_t>(bs) * W * Hkv * D && n_layers > 1) return GSS_ERR_ARG;
  if (!workspace || workspace_bytes < static_cast<size_t>(bs) * sizeof(uint32_t)) return GSS_ERR_WORKSPACE;
  CommitParams p;
  p.k_win = static_cast<const uint16_t*>(k_win);
  p.v_win = static_cast<const uint16_t*>(v_win);
  p.win_layer_stride = win_layer_stride;
  p.k_pages = static_cast<uint16_t*>(k_pages);
  p.v_pages = static_cast<uint16_t*>(v_pages);
  p.page_layer_stride = page_layer_stride;
  p.page_table = page_table;
  p.pt_stride = pt_stride;
  p.seq_lens = seq_lens;
  p.n_rows = n_rows;
  p.n_add = n_add;
  p.slots = slots;
  p.W = W;
  p.n_layers = n_layers;
  p.n_pb = (W + 2 * CPAGE - 2) / CPAGE;  // pages W rows can touch at any alignment
  p.Hkv = Hkv;
  p.D = D;
  p.counters = static_cast<uint32_t*>(workspace);
  hipLaunchKernelGGL(kv_commit_kernel, dim3(n_layers * p.n_pb, bs), dim3(COMMIT_THREADS), lds,
                     static_cast<hipStream_t>(stream), p);
  return gss_launch_status();
}
