// Dynamic W-way set-associative HBM row cache for the offload tiers: per decode step, the selected host rows are
// looked up in the cache, the distinct missing ones get a line (or a spill row) and every selected entry is resolved
// to the HBM row that will hold it. The row copies themselves run in spmla_wcache_fill (spmla_gather.hip), so the
// bookkeeping here never waits on PCIe.
//
// Reference: the W-way cache of LayerOffload (dotsnote/engine/arcstats_pkg/arcstats/sparse_offload.py:677-789:
// _sa_scan_kernel, _sa_fill_kernel, _sa_advance_kernel, _sa_resolve_kernel, _sa_invalidate_kernel; composition
// _sa_prefill :1595-1622) with its epoch-tagged miss table (offload_fill.py:1-45, ARC_OFFLOAD_HT_EPOCH).
//   * host row h lives in set h % S (S = C / W), in any of the set's W lines (tag[line] = h, -1 empty);
//   * scan: a hit pins its line for this step; each distinct missing row is appended once to the miss list;
//   * alloc: each miss takes a ticket in its set and replaces the ticket-th unpinned way counted round-robin from
//     rr[set]; misses beyond the set's unpinned ways go to spill rows (C + k, k < cap), past cap to the host (-2);
//   * advance: rr[set] += min(tickets, W) (mod W);
//   * resolve: res[t][k] = the line (tag hit) or the miss's spill row / -2; invalid entries -1.
// Which ways the misses of one set take, and which misses of an overfull set spill, follow the order of the atomics;
// the rows an entry resolves to always hold that entry's host row.
//
// MI355X choices: the per-step state needs no clearing (graph-capturable without memsets): the miss table's entries
// carry the step's epoch in their upper 32 bits (an entry of an older epoch is empty) and a line is pinned when
// pin[line] equals the epoch. One 1-thread launch advances the epoch and zeroes the step counters.
#include "spmla_common.h"

namespace spmla {
namespace wc {

// state[0] epoch, [1] distinct misses this step, [2] spill rows used, [3] hits (entries whose row was cached)
enum { ST_EPOCH = 0, ST_MISS = 1, ST_SPILL = 2, ST_HITS = 3 };

struct Cache {
  int* tag; int C, W, S;
  int* rr; int* cnt; int* pin;
  unsigned long long* ht; int* htv; unsigned hbits;   // miss table: 2^hbits entries (> the step's entries)
  long long* ml; int* mslot; long long* mdst;        // miss list: row, its table slot, its destination row
  int* state; int cap;
};

__device__ inline unsigned hslot(long long h, unsigned hbits) {   // multiplicative hash, top bits
  return (unsigned)(((unsigned long long)(uint32_t)h * 0x9E3779B97F4A7C15ull) >> (64 - hbits));
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

// one thread per entry (t, k)
__global__ void __launch_bounds__(256) scan_kernel(const int* __restrict__ idx, long long idx_st, int T, int K,
                                                   long long R, Cache c) {
  const long long g = (long long)blockIdx.x * 256 + threadIdx.x;
  if (g >= (long long)T * K) return;
  const int t = (int)(g / K), k = (int)(g % K);
  const long long h = idx[(long long)t * idx_st + k];
  if (h < 0 || h >= R) return;
  const unsigned epoch = (unsigned)c.state[ST_EPOCH];
  const int st = (int)(h % c.S);
  const int line = find_way(c, h, st);
  if (line >= 0) {
    c.pin[line] = (int)epoch;
    atomicAdd(c.state + ST_HITS, 1);
    return;
  }
  // distinct misses: insert (epoch, h) into the table; the table holds more slots than the step has entries, so
  // linear probing finds the key or a free slot within 2^hbits probes
  const unsigned long long key = ((unsigned long long)epoch << 32) | (uint32_t)h;
  const unsigned mask = (1u << c.hbits) - 1u;
  unsigned s = hslot(h, c.hbits);
  for (unsigned p = 0; p <= mask; ++p) {
    unsigned long long cur = __atomic_load_n(c.ht + s, __ATOMIC_RELAXED);
    while ((unsigned)(cur >> 32) != epoch) {          // free in this epoch: try to claim it
      const unsigned long long prev = atomicCAS(c.ht + s, cur, key);
      if (prev == cur) {
        const int m = atomicAdd(c.state + ST_MISS, 1);
        c.ml[m] = h;
        c.mslot[m] = (int)s;
        return;
      }
      cur = prev;
    }
    if (cur == key) return;                           // another entry of the same row claimed it
    s = (s + 1u) & mask;
  }
}

// one thread per miss m < state[ST_MISS] (the launch covers every entry of the step)
__global__ void __launch_bounds__(256) alloc_kernel(long long n, Cache c) {
  const long long m = (long long)blockIdx.x * 256 + threadIdx.x;
  if (m >= n || m >= c.state[ST_MISS]) return;
  const int epoch = c.state[ST_EPOCH];
  const long long h = c.ml[m];
  const int st = (int)(h % c.S);
  int ticket = atomicAdd(c.cnt + st, 1);
  const int r0 = c.rr[st];
  long long dst = -2;
  for (int j = 0; j < c.W; ++j) {
    const int w = r0 + j < c.W ? r0 + j : r0 + j - c.W;
    const int line = st * c.W + w;
    if (c.pin[line] != epoch) {
      if (ticket == 0) { dst = line; break; }
      --ticket;
    }
  }
  if (dst >= 0) {
    c.tag[dst] = (int)h;
  } else {
    const int sp = atomicAdd(c.state + ST_SPILL, 1);
    dst = sp < c.cap ? (long long)c.C + sp : -2;
  }
  c.htv[c.mslot[m]] = (int)dst;
  c.mdst[m] = dst >= 0 ? dst : -1;                   // -1: no copy (stays on the host)
}

__global__ void __launch_bounds__(256) advance_kernel(Cache c) {
  const int s = blockIdx.x * 256 + threadIdx.x;
  if (s >= c.S) return;
  const int n = c.cnt[s];
  c.rr[s] = (c.rr[s] + (n < c.W ? n : c.W)) % c.W;
  c.cnt[s] = 0;
}

__global__ void __launch_bounds__(256) resolve_kernel(const int* __restrict__ idx, long long idx_st, int T, int K,
                                                      long long R, Cache c, int* __restrict__ res, long long res_st) {
  const long long g = (long long)blockIdx.x * 256 + threadIdx.x;
  if (g >= (long long)T * K) return;
  const int t = (int)(g / K), k = (int)(g % K);
  const long long h = idx[(long long)t * idx_st + k];
  int r = -1;
  if (h >= 0 && h < R) {
    r = find_way(c, h, (int)(h % c.S));
    if (r < 0) {
      const unsigned epoch = (unsigned)c.state[ST_EPOCH];
      const unsigned long long key = ((unsigned long long)epoch << 32) | (uint32_t)h;
      const unsigned mask = (1u << c.hbits) - 1u;
      unsigned s = hslot(h, c.hbits);
      r = -2;
      for (unsigned p = 0; p <= mask; ++p) {
        const unsigned long long cur = c.ht[s];
        if (cur == key) { r = c.htv[s]; break; }
        if ((unsigned)(cur >> 32) != epoch) break;     // not in the table (cannot happen for a row of this step)
        s = (s + 1u) & mask;
      }
    }
  }
  res[(long long)t * res_st + k] = r;
}

// a rewritten host row must not be served from a stale line (sparse_offload.py:782-789)
__global__ void __launch_bounds__(256) invalidate_kernel(const long long* __restrict__ slots, int n, long long R,
                                                         int* tag, int W, int S) {
  const int i = blockIdx.x * 256 + threadIdx.x;
  if (i >= n) return;
  const long long h = slots[i];
  if (h < 0 || h >= R) return;
  int* tg = tag + (h % S) * W;
  for (int w = 0; w < W; ++w)
    if (tg[w] == (int)h) tg[w] = -1;
}

// per token: entries with res >= 0 -> hbm list (pool rows), res == -2 -> host list (the entry's host row); both
// compacted in order and padded with -1; counts per token (the tier split of a cache with a bounded spill area)
__global__ void __launch_bounds__(256) split_res_kernel(const int* __restrict__ idx, long long idx_st,
                                                        const int* __restrict__ res, long long res_st, int K,
                                                        int* __restrict__ hbm, long long hbm_st, int* __restrict__ hcnt,
                                                        int* __restrict__ host, long long host_st,
                                                        int* __restrict__ scnt) {
  __shared__ uint32_t wsum[4];
  const int t = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  uint32_t nh = 0, ns = 0;
  for (int k0 = 0; k0 < K; k0 += 2048) {
    int r[8], h[8];
    uint32_t cc = 0;
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int k = k0 + 8 * tid + u;
      r[u] = k < K ? res[(long long)t * res_st + k] : -1;
      h[u] = k < K ? idx[(long long)t * idx_st + k] : -1;
      cc += r[u] >= 0 ? 1u : (r[u] == -2 ? 0x10000u : 0u);
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
      if (r[u] >= 0) hbm[(long long)t * hbm_st + oh++] = r[u];
      else if (r[u] == -2) host[(long long)t * host_st + os++] = h[u];
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

int spmla_wcache_step(const int* idx, long long idx_st, int T, int K, long long R, int* tag, int C, int W, int* rr,
                      int* cnt, int* pin, unsigned long long* ht, int ht_log2, int* htv, long long* miss_rows,
                      int* miss_slots, long long* miss_dst, int* state, int cap, int* res, long long res_st,
                      void* stream) {
  if (T < 0 || K < 0 || R < 0 || C <= 0 || W <= 0 || C % W || cap < 0 || ht_log2 < 1 || ht_log2 > 30)
    return SPMLA_EARG;
  if (R > 0x7fffffffll) return SPMLA_ELIMIT;
  const long long n = (long long)T * K;
  if ((1ll << ht_log2) <= n) return SPMLA_ELIMIT;   // the miss table needs more slots than entries
  if (!tag || !rr || !cnt || !pin || !ht || !htv || !miss_rows || !miss_slots || !miss_dst || !state || !res ||
      (n > 0 && !idx))
    return SPMLA_EARG;
  hipStream_t s = (hipStream_t)stream;
  wc::Cache c;
  c.tag = tag; c.C = C; c.W = W; c.S = C / W; c.rr = rr; c.cnt = cnt; c.pin = pin;
  c.ht = ht; c.htv = htv; c.hbits = (unsigned)ht_log2; c.ml = miss_rows; c.mslot = miss_slots; c.mdst = miss_dst;
  c.state = state; c.cap = cap;
  hipLaunchKernelGGL(wc::begin_kernel, dim3(1), dim3(1), 0, s, state);
  if (n > 0) {
    const unsigned gb = (unsigned)((n + 255) / 256);
    hipLaunchKernelGGL(wc::scan_kernel, dim3(gb), dim3(256), 0, s, idx, idx_st, T, K, R, c);
    hipLaunchKernelGGL(wc::alloc_kernel, dim3(gb), dim3(256), 0, s, n, c);
    hipLaunchKernelGGL(wc::advance_kernel, dim3((c.S + 255) / 256), dim3(256), 0, s, c);
    hipLaunchKernelGGL(wc::resolve_kernel, dim3(gb), dim3(256), 0, s, idx, idx_st, T, K, R, c, res, res_st);
  }
  return (int)hipGetLastError();
}

int spmla_wcache_invalidate(const long long* slots, int n, long long R, int* tag, int C, int W, void* stream) {
  if (n < 0 || R < 0 || C <= 0 || W <= 0 || C % W) return SPMLA_EARG;
  if (n == 0) return SPMLA_OK;
  if (!slots || !tag) return SPMLA_EARG;
  hipLaunchKernelGGL(wc::invalidate_kernel, dim3((n + 255) / 256), dim3(256), 0, (hipStream_t)stream, slots, n, R,
                     tag, W, C / W);
  return (int)hipGetLastError();
}

int spmla_split_res(const int* idx, long long idx_st, const int* res, long long res_st, int T, int K, int* hbm_idx,
                    long long hbm_st, int* hbm_cnt, int* host_idx, long long host_st, int* host_cnt, void* stream) {
  if (T < 0 || K < 0) return SPMLA_EARG;
  if (T == 0) return SPMLA_OK;
  if (!idx || !res || !hbm_idx || !hbm_cnt || !host_idx || !host_cnt) return SPMLA_EARG;
  hipLaunchKernelGGL(wc::split_res_kernel, dim3(T), dim3(256), 0, (hipStream_t)stream, idx, idx_st, res, res_st, K,
                     hbm_idx, hbm_st, hbm_cnt, host_idx, host_st, host_cnt);
  return (int)hipGetLastError();
}

}  // extern "C"
