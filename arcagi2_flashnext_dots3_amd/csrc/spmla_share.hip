// Top-k overlap between the DSA layers of one step: for every query row and layer pair (a, b), the number of valid
// entries of b's top-k that are also in a's. This is the statistic the reference gathers to choose which layers may
// skip their indexer and reuse an earlier layer's top-k (cross-layer top-k sharing).
// Reference: dotsnote/engine/arcstats_pkg/arcstats/index_share.py:95-130 (TopkOverlap._accumulate: per row,
// hit = #{x in sorted(b) : x >= 0 and x in a} by searchsorted; recall = hit / |b|, jaccard = hit / (|a| + |b| - hit)).
//
// gfx950 mapping: one workgroup per query row. Layer a's set goes into an LDS hash table (4096 slots, linear probing,
// inserted with LDS compare-and-swap); every later layer's entries probe it, and the counts are summed in LDS. Each
// entry is read once per pair from global memory (L2-resident: a row's L sets are 8 KB each at K = 2048). Integer
// work, bound by LDS latency; exact, so results do not depend on the order of the atomics.
#include "spmla_common.h"

namespace spmla {
namespace share {

constexpr int TB = 4096;                 // hash slots (load factor <= 0.5 for K <= 2048)
constexpr int EMPTY = (int)0x80000000;   // entries >= 0 are row ids
constexpr int NT = 256;

struct Params {
  const int* sets; long long s_l, s_r;   // entry k of layer l, row i at sets[l * s_l + i * s_r + k]
  int L, n, K;
  int* hits;                             // [L][L][n]: hits[(a * L + b) * n + i], a != b (symmetric)
  int* nvalid;                           // [L][n]: valid entries (>= 0) of each set
};

__device__ inline unsigned slot_of(int x) { return ((unsigned)x * 2654435761u) >> (32 - 12); }

__global__ void __launch_bounds__(NT) overlap_kernel(Params p) {
  __shared__ int tbl[TB];
  __shared__ int red[NT / 64];
  const int i = blockIdx.x, tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  auto block_sum = [&](int v) -> int {   // all threads get the sum
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    __syncthreads();
    if (lane == 0) red[w] = v;
    __syncthreads();
    int s = 0;
#pragma unroll
    for (int k = 0; k < NT / 64; ++k) s += red[k];
    return s;
  };
  for (int a = 0; a < p.L; ++a) {
    for (int s = tid; s < TB; s += NT) tbl[s] = EMPTY;
    __syncthreads();
    const int* sa = p.sets + (long long)a * p.s_l + (long long)i * p.s_r;
    int na = 0;
    for (int k = tid; k < p.K; k += NT) {
      const int x = sa[k];
      if (x < 0) continue;
      ++na;
      unsigned s = slot_of(x);
      while (true) {                     // at most K of TB slots are ever used: a free or equal slot exists
        const int cur = atomicCAS(&tbl[s], EMPTY, x);
        if (cur == EMPTY || cur == x) break;
        s = (s + 1) & (TB - 1);
      }
    }
    na = block_sum(na);
    if (tid == 0) p.nvalid[(long long)a * p.n + i] = na;
    for (int b = a + 1; b < p.L; ++b) {
      const int* sb = p.sets + (long long)b * p.s_l + (long long)i * p.s_r;
      int h = 0;
      for (int k = tid; k < p.K; k += NT) {
        const int x = sb[k];
        if (x < 0) continue;
        unsigned s = slot_of(x);
        while (true) {                   // ends at the first empty slot (the table is never full)
          const int cur = tbl[s];
          if (cur == x) { ++h; break; }
          if (cur == EMPTY) break;
          s = (s + 1) & (TB - 1);
        }
      }
      h = block_sum(h);
      if (tid == 0) {
        p.hits[((long long)a * p.L + b) * p.n + i] = h;
        p.hits[((long long)b * p.L + a) * p.n + i] = h;
      }
    }
    __syncthreads();                     // every probe of table a is done before it is cleared
  }
}

}  // namespace share
}  // namespace spmla

using namespace spmla;

extern "C" {

int spmla_topk_overlap(const int* sets, long long s_l, long long s_r, int L, int n, int K, int* hits, int* nvalid,
                       void* stream) {
  if (L <= 0 || n < 0 || K < 0) return SPMLA_EARG;
  if (n == 0) return SPMLA_OK;
  if (!sets || !hits || !nvalid) return SPMLA_EARG;
  if (K > share::TB / 2) return SPMLA_ELIMIT;
  if ((long long)L * L * n > 0x7fffffffLL) return SPMLA_ELIMIT;
  share::Params p;
  p.sets = sets; p.s_l = s_l; p.s_r = s_r; p.L = L; p.n = n; p.K = K; p.hits = hits; p.nvalid = nvalid;
  hipLaunchKernelGGL(share::overlap_kernel, dim3((unsigned)n), dim3(share::NT), 0, (hipStream_t)stream, p);
  return (int)hipGetLastError();
}

}  // extern "C"
