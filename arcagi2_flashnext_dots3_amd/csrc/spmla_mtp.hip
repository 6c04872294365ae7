// Request-packed MTP decode, step 1: the union of the rows the G MTP tokens of a request selected, each with the
// bitmask of the tokens that selected it. The tokens of one request share most of their top-k rows (about 2400
// distinct of 4 x 2048 on real traffic), so the attention that follows loads and converts each union row once for
// all G tokens (the per-(token, row) mask keeps every token's softmax to its own rows).
// Reference: dotsnote/engine/arcstats_pkg/arcstats/csrc/offload_attn.cu:586-698 (pk_union_kernel).
//   u[r][0 .. cnt[r]) = the distinct valid rows (0 <= row < R) of tokens t0 .. t0 + G - 1 (G <= 6), ordered by
//   token mask descending (rows of every token first), then by the position j * topk + k of the row's first
//   occurrence (token j = the lowest token that selected it); mk = the masks; u[r][cnt .. nmax) = -1.
//
// gfx950 mapping: one 1024-thread workgroup per request. An LDS hash set of 16384 words ((row + 1) << 6 | token
// bits, inserted with compare-and-swap, bits merged with atomic or) collects the union; a histogram over the 64
// mask buckets gives each bucket's start; a stable placement then walks the entries in position order, 1024 per
// round: a wave ranks its lanes within their bucket by ballots over the distinct buckets it holds, and one thread
// per bucket turns the 16 waves' counts into offsets.
#include "spmla_common.h"

namespace spmla {
namespace mtp {

constexpr int NT = 1024, LOG = 14, TBL = 1 << LOG, GB = 6, NB = 1 << GB, PPT = 12;   // PPT x NT >= 6 x 2048

struct UnionParams {
  const int* idx; long long sit; int T, ql; const int* cu; long long R; int topk, nmax;
  int* u; uint8_t* mk; int* cnt;
};

__global__ void __launch_bounds__(NT) union_kernel(UnionParams p) {
  __shared__ uint32_t tbl[TBL];
  __shared__ int wcnt[NT / 64][NB];
  __shared__ int bcur[NB];
  __shared__ int tot;
  const int r = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int t0 = p.cu ? p.cu[r] : min(r * p.ql, p.T);
  const int t1 = p.cu ? p.cu[r + 1] : min(t0 + p.ql, p.T);
  const int G = min(max(t1 - t0, 0), GB);
  const int n = min(G * p.topk, PPT * NT);
  for (int i = tid; i < TBL; i += NT) tbl[i] = 0u;
  if (tid < NB) bcur[tid] = 0;
  __syncthreads();
  int ids[PPT], sl[PPT];
#pragma unroll
  for (int i = 0; i < PPT; ++i) {
    const int q = tid + i * NT;
    ids[i] = -1;
    sl[i] = -1;
    if (q < n) {
      const int j = q / p.topk, k = q - j * p.topk;
      const int h = p.idx[(long long)(t0 + j) * p.sit + k];
      if (h >= 0 && (long long)h < p.R) {
        const uint32_t key = (uint32_t)h + 1u, bit = 1u << j;
        uint32_t s = ((uint32_t)h * 2654435761u) >> (32 - LOG);
        while (true) {                   // at most 12288 of 16384 slots are used: the probe ends
          uint32_t cur = tbl[s];
          if (cur == 0u) {
            cur = atomicCAS(&tbl[s], 0u, (key << GB) | bit);
            if (cur == 0u) break;
          }
          if ((cur >> GB) == key) {
            atomicOr(&tbl[s], bit);
            break;
          }
          s = (s + 1) & (TBL - 1);
        }
        ids[i] = h;
        sl[i] = (int)s;
      }
    }
  }
  __syncthreads();
  for (int s = tid; s < TBL; s += NT) {   // bucket sizes: bucket (NB - 1) - mask (full masks first)
    const uint32_t w = tbl[s];
    if (w) atomicAdd(&bcur[(NB - 1) - (int)(w & (NB - 1))], 1);
  }
  __syncthreads();
  if (tid == 0) {
    int run = 0;
    for (int b = 0; b < NB; ++b) {
      const int c = bcur[b];
      bcur[b] = run;
      run += c;
    }
    tot = run;
    p.cnt[r] = run;
  }
  __syncthreads();
  const long long ub = (long long)r * p.nmax;
  const int nround = (n + NT - 1) / NT;
#pragma unroll
  for (int i = 0; i < PPT; ++i) {
    if (i < nround) {                    // workgroup-uniform
      for (int e = lane; e < NB; e += 64) wcnt[wv][e] = 0;
      int b = -1;
      uint32_t m = 0;
      if (sl[i] >= 0) {
        const int j = (tid + i * NT) / p.topk;
        m = tbl[sl[i]] & (NB - 1);
        if ((m & ((1u << j) - 1u)) == 0u) b = (NB - 1) - (int)m;   // the first occurrence: lowest selecting token
      }
      // rank among the lanes of this wave with the same bucket, and the wave's count per bucket
      int rank = 0;
      unsigned long long todo = __ballot(b >= 0);
      while (todo) {
        const int leader = __builtin_ctzll(todo);
        const int bb = __shfl(b, leader, 64);
        const unsigned long long peers = __ballot(b == bb);
        if (b == bb) rank = __popcll(peers & ((1ull << lane) - 1ull));
        if (lane == leader) wcnt[wv][bb] = __popcll(peers);
        todo &= ~peers;
      }
      __syncthreads();
      if (tid < NB) {                    // bucket tid: offsets of the 16 waves, in wave order
        int run = bcur[tid];
        for (int w = 0; w < NT / 64; ++w) {
          const int c = wcnt[w][tid];
          wcnt[w][tid] = run;
          run += c;
        }
        bcur[tid] = run;
      }
      __syncthreads();
      if (b >= 0) {
        const int d = wcnt[wv][b] + rank;
        p.u[ub + d] = ids[i];
        p.mk[ub + d] = (uint8_t)m;
      }
      __syncthreads();                   // wcnt reused by the next round
    }
  }
  for (int d = tot + tid; d < p.nmax; d += NT) p.u[ub + d] = -1;
}

}  // namespace mtp
}  // namespace spmla

using namespace spmla;

extern "C" {

int spmla_mtp_union(const int* idx, long long idx_st, int T, int ql, const int* cu, int nreq, long long R, int topk,
                    int nmax, int* u, unsigned char* mk, int* cnt, void* stream) {
  if (T < 0 || nreq < 0 || topk < 0 || nmax < 0 || R < 0 || (!cu && ql <= 0)) return SPMLA_EARG;
  if (!cu && ql > mtp::GB) return SPMLA_EARG;                          // at most 6 tokens per request
  if (nreq == 0) return SPMLA_OK;
  if (!idx || !u || !mk || !cnt) return SPMLA_EARG;
  if (R >= (1ll << (32 - mtp::GB)) - 1) return SPMLA_ELIMIT;          // (row + 1) << 6 fits 32 bits
  if ((long long)mtp::GB * topk > (long long)mtp::PPT * mtp::NT) return SPMLA_ELIMIT;
  const int gmax = cu ? mtp::GB : (ql < mtp::GB ? ql : mtp::GB);       // tokens per request used
  if ((long long)nmax < (long long)gmax * topk) return SPMLA_EARG;     // the union of the lists always fits
  mtp::UnionParams p;
  p.idx = idx; p.sit = idx_st; p.T = T; p.ql = ql; p.cu = cu; p.R = R; p.topk = topk; p.nmax = nmax;
  p.u = u; p.mk = mk; p.cnt = cnt;
  hipLaunchKernelGGL(mtp::union_kernel, dim3((unsigned)nreq), dim3(mtp::NT), 0, (hipStream_t)stream, p);
  return (int)hipGetLastError();
}

}  // extern "C"
