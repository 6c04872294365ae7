// Dynamic W-way set-associative HBM row cache for the offload tiers: per decode step, the selected host rows are
// looked up in the cache, the distinct missing ones get a line (or a spill row) and every selected entry is resolved
// to the HBM row that will hold it. The row copies themselves run in spmla_wcache_fill (spmla_gather.hip), so the
// bookkeeping here never waits on PCIe.
//
// Reference: the W-way cache of LayerOffload (dotsnote/engine/arcstats_pkg/arcstats/sparse_offload.py:677-789:
// _sa_scan_kernel, _sa_fill_kernel, _sa_advance_kernel, _sa_resolve_kernel, _sa_invalidate_kernel; composition
// _sa_prefill :1595-1622) and its epoch-tagged miss bookkeeping (offload_fill.py:1-45, ARC_OFFLOAD_HT_EPOCH).
//   * host row h lives in set h % S (S = C / W), in any of the set's W lines (tag[line] = h, -1 empty);
//   * scan: a hit pins its line for this step; each distinct missing row is appended once to the miss list;
//   * alloc: each miss takes a ticket in its set and replaces the ticket-th unpinned way counted round-robin from
//     rr[set]; misses beyond the set's unpinned ways go to spill rows (C + k, k < cap), past cap to the host (-2);
//   * advance (in the resolve launch): rr[set] += min(tickets, W) (mod W);
//   * resolve: res[t][k] = the line (tag hit) or the miss's spill row / -2; invalid entries -1.
//   * two-choice placement (option `two`; offload_fill.py:16-23, _set2 :136-138, P2 paths :158-165 and :269-279,
//     _invalidate2_kernel :296-303): row h may also live in a second set ((h * 2654435761) >> 12) % S. Lookups check
//     it for entries that miss the first set (a hit there pins that line); a miss that finds no unpinned way for its
//     ticket in the first set takes a ticket in the second before it spills; invalidation clears both sets. Tickets of
//     both kinds share the set's counter, so the ways one step hands out in a set stay distinct and rr advances by
//     min(tickets, W) as before. A row is cached in at most one of its sets (only a miss in both places it).
// Which ways the misses of one set take, and which misses of an overfull set spill, follow the order of the atomics;
// the rows an entry resolves to always hold that entry's host row.
//
// MI355X choices: the reference deduplicates the misses in a hashed table to save memory; with 288 GB of HBM this
// build keeps two ints per host row instead (8 bytes per row: 16 MB for 2M rows). claim[h] holds the last step that
// saw row h miss (atomicMax with the step's epoch: the entry that raises it owns the row's miss), rdst[h] the pool row
// the miss was given. One atomic per missing entry, no probing. The per-step state needs no clearing
// (graph-capturable without memsets): claims and pins compare against the epoch, which one 1-thread launch advances
// (with the step counters) at the start of every step.
#include "spmla_common.h"

namespace spmla {
namespace wc {

// state[0] epoch, [1] distinct misses this step, [2] spill rows used, [3] hits (entries whose row was cached)
enum { ST_EPOCH = 0, ST_MISS = 1, ST_SPILL = 2, ST_HITS = 3 };

struct Cache {
  int* tag; int C, W, S;
  int* rr; int* cnt; int* pin;
  int* claim; int* rdst;                              // per host row: last epoch it missed, its pool row then
  long long* ml; long long* mdst;                     // miss list: row, its destination row
  int* state; int cap;
  int two;                                            // two-choice placement
};

// the second candidate set of host row h (0 <= h < 2^31, so the product fits 63 bits)
__device__ inline int set2_of(long long h, int S) {
  return (int)((((unsigned long long)h * 2654435761ull) >> 12) % (unsigned long long)S);
}

__global__ void begin_kernel(int* state) {
  state[ST_EPOCH] = state[ST_EPOCH] + 1;
  state[ST_MISS] = 0;
  state[ST_SPILL] = 0;
  state[ST_HITS] = 0;
}

__device__ inline int find_way(const Cache& c, long long h, int st) {
  const int* tg = c.tag + (long long)st * c.W;
  for (int w = 0; w < c.W; ++w)
    if (tg[w] == (int)h) return st * c.W + w;
  return -1;
}

// one thread per entry (t, k), 1024 per workgroup. The hit and miss counters are advanced once per workgroup
// (per-wave ballot counts summed in LDS): same-address atomics serialize at the L2, and one per wave (4096 per
// config-3 step on two counters) measured 40 us of this kernel's 52.
constexpr int SCAN_TPB = 1024;
__global__ void __launch_bounds__(SCAN_TPB) scan_kernel(const int* __restrict__ idx, long long idx_st, int T, int K,
                                                        long long R, Cache c) {
  __shared__ int wh[SCAN_TPB / 64], wm[SCAN_TPB / 64];
  __shared__ int mbase;
  const long long g = (long long)blockIdx.x * SCAN_TPB + threadIdx.x;
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const int epoch = c.state[ST_EPOCH];
  long long h = -1;
  if (g < (long long)T * K) h = idx[(g / K) * idx_st + g % K];
  const bool valid = h >= 0 && h < R;
  int line = -1;
  if (valid) {
    line = find_way(c, h, (int)(h % c.S));
    if (line < 0 && c.two) line = find_way(c, h, set2_of(h, c.S));
    if (line >= 0) c.pin[line] = epoch;
  }
  // distinct misses: the entry that raises claim[h] to this epoch owns the row's miss
  const bool claimed = valid && line < 0 && atomicMax(c.claim + h, epoch) < epoch;
  const unsigned long long hb = __ballot(line >= 0), cb = __ballot(claimed);
  if (lane == 0) { wh[wv] = (int)__popcll(hb); wm[wv] = (int)__popcll(cb); }
  __syncthreads();
  if (threadIdx.x == 0) {
    int th = 0, tm = 0;
    for (int w = 0; w < SCAN_TPB / 64; ++w) {
      th += wh[w];
      const int x = wm[w];
      wm[w] = tm;                                     // exclusive prefix: this wave's first slot in the block
      tm += x;
    }
    if (th) atomicAdd(c.state + ST_HITS, th);
    mbase = tm ? atomicAdd(c.state + ST_MISS, tm) : 0;
  }
  __syncthreads();
  if (claimed) c.ml[mbase + wm[wv] + (int)__popcll(cb & ((1ull << lane) - 1ull))] = h;
}

// a ticket in set st: the ticket-th unpinned way counted round-robin from rr[st], or -2 past the set's unpinned ways
__device__ inline long long take_way(const Cache& c, int st, int epoch) {
  int ticket = atomicAdd(c.cnt + st, 1);
  const int r0 = c.rr[st];
  for (int j = 0; j < c.W; ++j) {
    const int w = r0 + j < c.W ? r0 + j : r0 + j - c.W;
    const int line = st * c.W + w;
    if (c.pin[line] != epoch) {
      if (ticket == 0) return line;
      --ticket;
    }
  }
  return -2;
}

// one thread per miss m < state[ST_MISS] (the launch covers every entry of the step)
__global__ void __launch_bounds__(256) alloc_kernel(long long n, Cache c) {
  const long long m = (long long)blockIdx.x * 256 + threadIdx.x;
  if (m >= n || m >= c.state[ST_MISS]) return;
  const int epoch = c.state[ST_EPOCH];
  const long long h = c.ml[m];
  long long dst = take_way(c, (int)(h % c.S), epoch);
  if (dst < 0 && c.two) dst = take_way(c, set2_of(h, c.S), epoch);
  if (dst >= 0) {
    c.tag[dst] = (int)h;
  } else {
    const int sp = atomicAdd(c.state + ST_SPILL, 1);
    dst = sp < c.cap ? (long long)c.C + sp : -2;
  }
  c.rdst[h] = (int)dst;
  c.mdst[m] = dst >= 0 ? dst : -1;                   // -1: no copy (stays on the host)
}

// also advances the round-robin pointers (threads g < S; alloc has finished with rr and cnt)
__global__ void __launch_bounds__(256) resolve_kernel(const int* __restrict__ idx, long long idx_st, int T, int K,
                                                      long long R, Cache c, int* __restrict__ res, long long res_st) {
  const long long g = (long long)blockIdx.x * 256 + threadIdx.x;
  if (g < c.S) {
    const int n = c.cnt[g];
    c.rr[g] = (c.rr[g] + (n < c.W ? n : c.W)) % c.W;
    c.cnt[g] = 0;
  }
  if (g >= (long long)T * K) return;
  const int t = (int)(g / K), k = (int)(g % K);
  const long long h = idx[(long long)t * idx_st + k];
  int r = -1;
  if (h >= 0 && h < R) {
    r = find_way(c, h, (int)(h % c.S));
    if (r < 0 && c.two) r = find_way(c, h, set2_of(h, c.S));
    if (r < 0) r = c.rdst[h];                        // this step's miss: its line (tag found above) or spill / host
  }
  res[(long long)t * res_st + k] = r;
}

// a rewritten host row must not be served from a stale line (sparse_offload.py:782-789)
__global__ void __launch_bounds__(256) invalidate_kernel(const long long* __restrict__ slots, int n, long long R,
                                                         int* tag, int W, int S, int two) {
  const int i = blockIdx.x * 256 + threadIdx.x;
  if (i >= n) return;
  const long long h = slots[i];
  if (h < 0 || h >= R) return;
  int* tg = tag + (h % S) * W;
  for (int w = 0; w < W; ++w)
    if (tg[w] == (int)h) tg[w] = -1;
  if (two) {
    tg = tag + (long long)set2_of(h, S) * W;
    for (int w = 0; w < W; ++w)
      if (tg[w] == (int)h) tg[w] = -1;
  }
}

// per token, two lists compacted in order and padded with -1, with counts per token:
//   pin == nullptr: entries with res >= 0 -> list A (pool rows), res == -2 -> list B (the entry's host row): the
//                    tier split of a cache with a bounded spill area;
//   pin != nullptr: entries whose line was a hit of this step (pin[line] == epoch) -> A, the other entries with
//                    res >= 0 (rows the step's fill brings in) -> B, both as pool rows: the split that lets the
//                    attention over the hits run while the misses are copied in.
__global__ void __launch_bounds__(256) split_res_kernel(const int* __restrict__ idx, long long idx_st,
                                                        const int* __restrict__ res, long long res_st, int K,
                                                        int* __restrict__ hbm, long long hbm_st, int* __restrict__ hcnt,
                                                        int* __restrict__ host, long long host_st,
                                                        int* __restrict__ scnt, const int* __restrict__ pin, int C,
                                                        const int* __restrict__ state) {
  __shared__ uint32_t wsum[4];
  const int t = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const bool by_hit = pin != nullptr;
  const int epoch = by_hit ? state[ST_EPOCH] : 0;
  uint32_t nh = 0, ns = 0;
  for (int k0 = 0; k0 < K; k0 += 2048) {
    int r[8], h[8];
    uint32_t cc = 0;
    bool a[8], b[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int k = k0 + 8 * tid + u;
      r[u] = k < K ? res[(long long)t * res_st + k] : -1;
      h[u] = (k < K && !by_hit) ? idx[(long long)t * idx_st + k] : r[u];
    }
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      if (by_hit) {
        a[u] = r[u] >= 0 && r[u] < C && pin[r[u]] == epoch;
        b[u] = r[u] >= 0 && !a[u];
      } else {
        a[u] = r[u] >= 0;
        b[u] = r[u] == -2;
      }
      cc += a[u] ? 1u : (b[u] ? 0x10000u : 0u);
    }
    uint32_t inc = cc;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
      const uint32_t y = __shfl_up(inc, o, 64);
      if (lane >= o) inc += y;
    }
    if (lane == 63) wsum[wv] = inc;
    __syncthreads();
    uint32_t base = 0, tot = 0;
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      base += w < wv ? wsum[w] : 0u;
      tot += wsum[w];
    }
    const uint32_t ex = base + inc - cc;
    uint32_t oh = nh + (ex & 0xffffu), os = ns + (ex >> 16);
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      if (a[u]) hbm[(long long)t * hbm_st + oh++] = r[u];
      else if (b[u]) host[(long long)t * host_st + os++] = h[u];
    }
    nh += tot & 0xffffu;
    ns += tot >> 16;
    __syncthreads();
  }
  for (int k = nh + tid; k < K; k += 256) hbm[(long long)t * hbm_st + k] = -1;
  for (int k = ns + tid; k < K; k += 256) host[(long long)t * host_st + k] = -1;
  if (tid == 0) { hcnt[t] = (int)nh; scnt[t] = (int)ns; }
}

}  // namespace wc
}  // namespace spmla

using namespace spmla;

extern "C" {

static int wcache_setup(wc::Cache& c, const int* idx, int T, int K, long long R, int* tag, int C, int W, int* rr,
                        int* cnt, int* pin, int* claim, int* rdst, long long* miss_rows, long long* miss_dst,
                        int* state, int cap, int two) {
  if (T < 0 || K < 0 || R < 0 || C <= 0 || W <= 0 || C % W || cap < 0 || (two != 0 && two != 1)) return SPMLA_EARG;
  if (R > 0x7fffffffll) return SPMLA_ELIMIT;
  const long long n = (long long)T * K;
  if (!tag || !rr || !cnt || !pin || !claim || !rdst || !miss_rows || !miss_dst || !state || (n > 0 && !idx))
    return SPMLA_EARG;
  c.tag = tag; c.C = C; c.W = W; c.S = C / W; c.rr = rr; c.cnt = cnt; c.pin = pin;
  c.claim = claim; c.rdst = rdst; c.ml = miss_rows; c.mdst = miss_dst;
  c.state = state; c.cap = cap; c.two = two;
  return SPMLA_OK;
}

int spmla_wcache_place(const int* idx, long long idx_st, int T, int K, long long R, int* tag, int C, int W, int* rr,
                       int* cnt, int* pin, int* claim, int* rdst, long long* miss_rows, long long* miss_dst, int* state,
                       int cap, int two, void* stream) {
  wc::Cache c;
  const int e =
      wcache_setup(c, idx, T, K, R, tag, C, W, rr, cnt, pin, claim, rdst, miss_rows, miss_dst, state, cap, two);
  if (e) return e;
  hipStream_t s = (hipStream_t)stream;
  const long long n = (long long)T * K;
  hipLaunchKernelGGL(wc::begin_kernel, dim3(1), dim3(1), 0, s, state);
  if (n > 0) {
    hipLaunchKernelGGL(wc::scan_kernel, dim3((unsigned)((n + wc::SCAN_TPB - 1) / wc::SCAN_TPB)), dim3(wc::SCAN_TPB), 0,
                       s, idx, idx_st, T, K, R, c);
    hipLaunchKernelGGL(wc::alloc_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, n, c);
  }
  return (int)hipGetLastError();
}

int spmla_wcache_resolve(const int* idx, long long idx_st, int T, int K, long long R, int* tag, int C, int W, int* rr,
                         int* cnt, int* pin, int* claim, int* rdst, long long* miss_rows, long long* miss_dst,
                         int* state, int cap, int two, int* res, long long res_st, void* stream) {
  wc::Cache c;
  const int e =
      wcache_setup(c, idx, T, K, R, tag, C, W, rr, cnt, pin, claim, rdst, miss_rows, miss_dst, state, cap, two);
  if (e) return e;
  if (!res) return SPMLA_EARG;
  const long long n = (long long)T * K;
  const long long nr = n > c.S ? n : c.S;
  hipLaunchKernelGGL(wc::resolve_kernel, dim3((unsigned)((nr + 255) / 256)), dim3(256), 0, (hipStream_t)stream, idx,
                     idx_st, T, K, R, c, res, res_st);
  return (int)hipGetLastError();
}

int spmla_wcache_step(const int* idx, long long idx_st, int T, int K, long long R, int* tag, int C, int W, int* rr,
                      int* cnt, int* pin, int* claim, int* rdst, long long* miss_rows, long long* miss_dst, int* state,
                      int cap, int two, int* res, long long res_st, void* stream) {
  wc::Cache c;                                        // validate everything before anything is launched
  int e =
      wcache_setup(c, idx, T, K, R, tag, C, W, rr, cnt, pin, claim, rdst, miss_rows, miss_dst, state, cap, two);
  if (e) return e;
  if (!res) return SPMLA_EARG;
  e = spmla_wcache_place(idx, idx_st, T, K, R, tag, C, W, rr, cnt, pin, claim, rdst, miss_rows, miss_dst, state,
                         cap, two, stream);
  if (e) return e;
  return spmla_wcache_resolve(idx, idx_st, T, K, R, tag, C, W, rr, cnt, pin, claim, rdst, miss_rows, miss_dst, state,
                              cap, two, res, res_st, stream);
}

int spmla_wcache_invalidate(const long long* slots, int n, long long R, int* tag, int C, int W, int two,
                            void* stream) {
  if (n < 0 || R < 0 || C <= 0 || W <= 0 || C % W || (two != 0 && two != 1)) return SPMLA_EARG;
  if (n == 0) return SPMLA_OK;
  if (!slots || !tag) return SPMLA_EARG;
  hipLaunchKernelGGL(wc::invalidate_kernel, dim3((n + 255) / 256), dim3(256), 0, (hipStream_t)stream, slots, n, R,
                     tag, W, C / W, two);
  return (int)hipGetLastError();
}

int spmla_split_res(const int* idx, long long idx_st, const int* res, long long res_st, int T, int K, int* hbm_idx,
                    long long hbm_st, int* hbm_cnt, int* host_idx, long long host_st, int* host_cnt, void* stream) {
  if (T < 0 || K < 0) return SPMLA_EARG;
  if (T == 0) return SPMLA_OK;
  if (!idx || !res || !hbm_idx || !hbm_cnt || !host_idx || !host_cnt) return SPMLA_EARG;
  hipLaunchKernelGGL(wc::split_res_kernel, dim3(T), dim3(256), 0, (hipStream_t)stream, idx, idx_st, res, res_st, K,
                     hbm_idx, hbm_st, hbm_cnt, host_idx, host_st, host_cnt, (const int*)nullptr, 0,
                     (const int*)nullptr);
  return (int)hipGetLastError();
}

int spmla_wcache_split(const int* res, long long res_st, int T, int K, const int* pin, int C, const int* state,
                       int* hit_idx, long long hit_st, int* hit_cnt, int* fresh_idx, long long fresh_st, int* fresh_cnt,
                       void* stream) {
  if (T < 0 || K < 0 || C <= 0) return SPMLA_EARG;
  if (T == 0) return SPMLA_OK;
  if (!res || !pin || !state || !hit_idx || !hit_cnt || !fresh_idx || !fresh_cnt) return SPMLA_EARG;
  hipLaunchKernelGGL(wc::split_res_kernel, dim3(T), dim3(256), 0, (hipStream_t)stream, res, res_st, res, res_st, K,
                     hit_idx, hit_st, hit_cnt, fresh_idx, fresh_st, fresh_cnt, pin, C, state);
  return (int)hipGetLastError();
}

}  // extern "C"
