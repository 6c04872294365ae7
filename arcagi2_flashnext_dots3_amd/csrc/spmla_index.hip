// Indexer logits and exact top-k selection.
//
// Logits (dotsnote/engine/arcstats_pkg/arcstats/shard_logits_v2.py:49-123, shard_indexer.py:63-91; torch statement
// dotsnote/training/finetune/student.py:219-222):
//   logit[row][j] = min(sum_h w[row][h] * relu(q[row][h] . kcode[j]) * ks[j], 60000) for positions j < ctx[row]
//   (column j holds position j * P + rank of this rank's key store), -inf for j >= ctx (unless noinf).
//   gfx950: one wave per 32-key tile; S = Q K^T on bf16 MFMA (32x32x16; e4m3 key codes convert exactly to bf16,
//   two per instruction), 64 heads = 2 M blocks, keys as the B operand; the head reduction is in-lane plus one
//   cross-half exchange. (The fp8 MFMA would take the codes directly, but its internal accumulation keeps only
//   ~2^-12 of the largest product on gfx950, too coarse for the selection.)
//
// Top-k (dotsnote/engine/arcstats_pkg/arcstats/fast_topk.py:1-15, csrc/topk_select.cu:1-30 semantics):
//   per row, the K largest values among columns j < n = min(ctx, Lc) by torch's order-preserving key
//   (-0 < +0, NaN largest); equal keys -> lower column first; output positions sorted by (value desc, column asc),
//   -1 where the value is +-inf and in slots >= n.
//   gfx950: one 1024-thread workgroup per row: 11/11/10-bit radix passes with an LDS histogram; once the boundary
//   bin is small it is resolved exactly in LDS (candidate sort), else narrowed further; ties on the final key take
//   the lowest columns through an ordered block scan. The K winners are bitonic-sorted in LDS.
#include "spmla_common.h"

namespace spmla {
namespace idx {

// ------------------------------------------------------------------------------------------------ logits
constexpr int LG_TPW = 4;   // 32-key tiles per wave
constexpr int LG_KPB = 4 * LG_TPW * 32;   // keys per 256-thread block

struct LogitParams {
  const uint16_t* q; long long q_st, q_sh;   // q[row][64][128] bf16
  const float* w; long long w_st;            // w[row][64]
  const uint8_t* store; long long R_local; int rpb; long long blk_stride;
  const int* bt; long long bt_st; int bs;    // block table [req][...], block size (positions per block)
  const int* req; const int* ctx;            // per row
  int rows, Lc, P, rank, noinf;
  float* out; long long out_st;
};

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
__device__ inline uint32_t fp8lo_bf16x2(uint32_t w) {
  return __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w, 1.0f, false));
}
__device__ inline uint32_t fp8hi_bf16x2(uint32_t w) {
  return __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w, 1.0f, true));
}

__global__ void __launch_bounds__(256) logits_kernel(LogitParams p) {
  const int row = blockIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
  const int lane = threadIdx.x & 63;
  const int half = lane >> 5, l32 = lane & 31;
  const int ctx = p.ctx[row];
  const int j_blk = blockIdx.y * LG_KPB;
  float* orow = p.out + (long long)row * p.out_st;
  if ((long long)j_blk * p.P + p.rank >= ctx) {   // whole block beyond the context
    if (!p.noinf)
      for (int j = j_blk + threadIdx.x; j < j_blk + LG_KPB && j < p.Lc; j += 256) orow[j] = -__builtin_inff();
    return;
  }
  // query fragments (bf16 A operand): M block m = heads 32m..32m+31 (lane head 32m + l32); k-pair kp covers dims
  // 32kp + 16half + 0..15, MFMA 2kp taking the first 8 and 2kp+1 the next 8 (same permutation as the key operand)
  const uint16_t* qr = p.q + (long long)row * p.q_st;
  bf16x8 qf[2][8];
  float wl[2][16];
#pragma unroll
  for (int m = 0; m < 2; ++m) {
    const uint16_t* src = qr + (long long)(32 * m + l32) * p.q_sh + 16 * half;
#pragma unroll
    for (int kp = 0; kp < 4; ++kp) {
      qf[m][2 * kp] = __builtin_bit_cast(bf16x8, *(const u32x4*)(src + 32 * kp));
      qf[m][2 * kp + 1] = __builtin_bit_cast(bf16x8, *(const u32x4*)(src + 32 * kp + 8));
    }
    // weights of this lane's C-layout heads (8(i/4) + 4half + i%4 in block m)
    const float myw = p.w[(long long)row * p.w_st + 32 * m + l32];
#pragma unroll
    for (int i = 0; i < 16; ++i) wl[m][i] = __shfl(myw, 8 * (i >> 2) + 4 * half + (i & 3), 64);
  }
  const int* btr = p.bt + (long long)p.req[row] * p.bt_st;
#pragma unroll 1
  for (int tt = 0; tt < LG_TPW; ++tt) {
    const int j0 = j_blk + (wave * LG_TPW + tt) * 32;
    if (j0 >= p.Lc) break;
    const int j = j0 + l32;
    const long long pos = (long long)j * p.P + p.rank;
    bool ok = j < p.Lc && pos < ctx;
    long long lrow = 0;
    if (ok) {
      const int blk = btr[pos / p.bs];
      lrow = ((long long)blk * p.bs + pos % p.bs) / p.P;
      ok = blk >= 0 && lrow < p.R_local;
    }
    const uint8_t* kr = p.store + (ok ? (lrow / p.rpb) * p.blk_stride + (lrow % p.rpb) * 132 : 0);
    uint32_t kw[4][4];
    float ksc = 0.f;
    if (ok) {
#pragma unroll
      for (int kp = 0; kp < 4; ++kp)
#pragma unroll
        for (int i = 0; i < 4; ++i) kw[kp][i] = *(const uint32_t*)(kr + 32 * kp + 16 * half + 4 * i);
      ksc = *(const float*)(kr + 128);
    } else {
#pragma unroll
      for (int kp = 0; kp < 4; ++kp)
#pragma unroll
        for (int i = 0; i < 4; ++i) kw[kp][i] = 0u;
    }
    bf16x8 kb[8];
#pragma unroll
    for (int kp = 0; kp < 4; ++kp) {
      i32x4 a0, a1;
      a0[0] = (int)fp8lo_bf16x2(kw[kp][0]); a0[1] = (int)fp8hi_bf16x2(kw[kp][0]);
      a0[2] = (int)fp8lo_bf16x2(kw[kp][1]); a0[3] = (int)fp8hi_bf16x2(kw[kp][1]);
      a1[0] = (int)fp8lo_bf16x2(kw[kp][2]); a1[1] = (int)fp8hi_bf16x2(kw[kp][2]);
      a1[2] = (int)fp8lo_bf16x2(kw[kp][3]); a1[3] = (int)fp8hi_bf16x2(kw[kp][3]);
      kb[2 * kp] = __builtin_bit_cast(bf16x8, a0);
      kb[2 * kp + 1] = __builtin_bit_cast(bf16x8, a1);
    }
    float part = 0.f;
#pragma unroll
    for (int m = 0; m < 2; ++m) {
      f32x16 acc = f32x16{};
#pragma unroll
      for (int ks = 0; ks < 8; ++ks) acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(qf[m][ks], kb[ks], acc, 0, 0, 0);
#pragma unroll
      for (int i = 0; i < 16; ++i) part = __builtin_fmaf(wl[m][i], fmaxf(acc[i], 0.f), part);
    }
    part += __shfl_xor(part, 32, 64);
    if (half == 0 && j < p.Lc) {
      const float lg = fminf(part * ksc, 60000.f);
      if (ok) orow[j] = lg;
      else if (!p.noinf) orow[j] = -__builtin_inff();
    }
  }
}

// ------------------------------------------------------------------------------------------------ top-k
constexpr int TK_NT = 1024;
constexpr int TK_KMAX = 2048;
constexpr int TK_CAP = 4096;

__device__ inline uint32_t okey(float v) {
  const uint32_t x = f2u(v);
  if (v != v) return 0xffffffffu;
  return (x & 0x80000000u) ? ~x : (x | 0x80000000u);
}

// block-wide exclusive scan of a per-thread count (1024 threads = 16 waves)
__device__ inline uint32_t block_excl_scan(uint32_t v, uint32_t* wsum, uint32_t* total) {
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  uint32_t inc = v;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const uint32_t t = __shfl_up(inc, o, 64);
    if (lane >= o) inc += t;
  }
  if (lane == 63) wsum[wv] = inc;
  __syncthreads();
  if (wv == 0) {
    const uint32_t w = lane < TK_NT / 64 ? wsum[lane] : 0u;
    uint32_t wi = w;
#pragma unroll
    for (int o = 1; o < 16; o <<= 1) {
      const uint32_t t = __shfl_up(wi, o, 64);
      if (lane >= o) wi += t;
    }
    if (lane < TK_NT / 64) wsum[lane] = wi - w;
    if (lane == TK_NT / 64 - 1) wsum[16] = wi;
  }
  __syncthreads();
  const uint32_t r = wsum[wv] + inc - v;
  *total = wsum[16];
  __syncthreads();
  return r;
}

// bitonic sort of n (power of two) uint64 in LDS, descending
__device__ inline void bitonic_desc(unsigned long long* a, int n) {
  for (int size = 2; size <= n; size <<= 1) {
    for (int stride = size >> 1; stride > 0; stride >>= 1) {
      for (int t = threadIdx.x; t < n / 2; t += TK_NT) {
        const int lo = 2 * t - (t & (stride - 1));
        const int hi = lo + stride;
        const bool desc = (lo & size) == 0;
        const unsigned long long x = a[lo], y = a[hi];
        if ((x < y) == desc) { a[lo] = y; a[hi] = x; }
      }
      __syncthreads();
    }
  }
}

// Candidate sources of one row. n = number of candidates; val(j) = the value of candidate j; id(j) = what the
// output reports for it. Ties on the key go to the lower candidate number j.
struct RowSrc {     // a logits row: candidate j = column j
  const float* x; int n;
  __device__ float val(int j) const { return x[j]; }
  __device__ int id(int j) const { return j; }
};
struct MergeSrc {   // all-gathered payloads [P][nrows][2 * kl] = [values | positions]: candidate c = (c / kl, c % kl)
  const float* allp; long long nrows; int row, kl, n;
  __device__ const float* seg(int c, int& i) const {
    const int r = c / kl;
    i = c - r * kl;
    return allp + ((long long)r * nrows + row) * 2 * kl;
  }
  __device__ float val(int c) const { int i; const float* b = seg(c, i); return b[i]; }
  __device__ int id(int c) const { int i; const float* b = seg(c, i); return (int)f2u(b[kl + i]); }
};

struct TopkLds {
  uint32_t hist[2048];
  unsigned long long sel[TK_KMAX];
  unsigned long long cand[TK_CAP];
  uint32_t wsum[17];
  uint32_t sh[8];
};

__device__ inline unsigned long long tk_pack(uint32_t key, int j) {
  return ((unsigned long long)key << 32) | (uint32_t)(~(uint32_t)j);
}

// Selects the K largest candidates (key desc, j asc) of src into L.sel (unordered); returns their number min(n, K).
template <class Src>
__device__ int tk_select(const Src& src, int K, TopkLds& L) {
  const int tid = threadIdx.x, n = src.n;
  uint32_t* hist = L.hist;
  unsigned long long* sel = L.sel;
  unsigned long long* cand = L.cand;
  uint32_t* sh = L.sh;
  if (n <= K) {
    for (int j = tid; j < n; j += TK_NT) sel[j] = tk_pack(okey(src.val(j)), j);
    __syncthreads();
    return n;
  }
  if (tid == 0) sh[0] = 0;   // sel fill counter
  uint32_t prefix = 0, mask = 0;
  uint32_t need = (uint32_t)K;
  bool done = false;
  for (int pass = 0; pass < 3 && !done; ++pass) {
    const int shift = pass == 0 ? 21 : (pass == 1 ? 10 : 0);
    const uint32_t dm = pass == 2 ? 0x3ffu : 0x7ffu;
    for (int i = tid; i < 2048; i += TK_NT) hist[i] = 0;
    __syncthreads();
    for (int j = tid; j < n; j += TK_NT) {
      const uint32_t k = okey(src.val(j));
      if ((k & mask) == prefix) atomicAdd(&hist[(k >> shift) & dm], 1u);
    }
    __syncthreads();
    // thread t owns the two bins 2047 - 2t, 2046 - 2t (descending); suffix counts by a block scan
    const int b0 = 2047 - 2 * tid, b1 = b0 - 1;
    const uint32_t h0 = hist[b0], h1 = hist[b1];
    uint32_t tot;
    const uint32_t before = block_excl_scan(h0 + h1, L.wsum, &tot);
    if (before < need && before + h0 >= need) { sh[1] = (uint32_t)b0; sh[2] = before; sh[3] = h0; }
    if (before + h0 < need && before + h0 + h1 >= need) { sh[1] = (uint32_t)b1; sh[2] = before + h0; sh[3] = h1; }
    __syncthreads();
    const uint32_t b = sh[1], above = sh[2], binc = sh[3];
    const uint32_t pmask = mask, pprefix = prefix;
    const uint32_t np = prefix | (b << shift), nm = mask | (dm << shift);
    // elements under the current prefix whose digit is above b are selected
    const bool whole = above + binc == need;
    const bool fits = binc <= TK_CAP;
    const bool last = pass == 2;
    if (whole || fits || last) {
      if (tid == 0) sh[4] = 0;   // cand counter
      __syncthreads();
      for (int j = tid; j < n; j += TK_NT) {
        const uint32_t k = okey(src.val(j));
        if ((k & pmask) != pprefix) continue;
        const uint32_t d = (k >> shift) & dm;
        if (d > b || (whole && d == b)) {
          const uint32_t s = atomicAdd(&sh[0], 1u);
          sel[s] = tk_pack(k, j);
        } else if (d == b && fits && !whole) {
          const uint32_t s = atomicAdd(&sh[4], 1u);
          cand[s] = tk_pack(k, j);
        }
      }
      __syncthreads();
      if (whole) {
        done = true;
      } else if (fits) {
        // resolve inside the boundary bin: sort candidates, keep the first need - above
        const int nc = (int)sh[4];
        int np2 = 1;
        while (np2 < nc) np2 <<= 1;
        for (int i = nc + tid; i < np2; i += TK_NT) cand[i] = 0ull;
        __syncthreads();
        bitonic_desc(cand, np2);
        const uint32_t take = need - above;
        const uint32_t base = sh[0];
        for (uint32_t i = tid; i < take; i += TK_NT) sel[base + i] = cand[i];
        __syncthreads();
        if (tid == 0) sh[0] = base + take;
        done = true;
      } else {
        // last pass, boundary key fully known: take the lowest candidates equal to it (ordered scan)
        const uint32_t T = np;
        const uint32_t take = need - above;
        uint32_t got = 0;
        const uint32_t base = sh[0];
        __syncthreads();
        for (int j0 = 0; j0 < n && got < take; j0 += TK_NT) {
          const int j = j0 + tid;
          const bool eq = j < n && okey(src.val(j)) == T;
          uint32_t tot2;
          const uint32_t r = block_excl_scan(eq ? 1u : 0u, L.wsum, &tot2);
          if (eq && got + r < take) sel[base + got + r] = tk_pack(T, j);
          got += tot2;
        }
        __syncthreads();
        if (tid == 0) sh[0] = base + take;
        done = true;
      }
    } else {
      // narrow: everything above the bin is selected now, continue inside the bin
      for (int j = tid; j < n; j += TK_NT) {
        const uint32_t k = okey(src.val(j));
        if ((k & pmask) != pprefix) continue;
        if (((k >> shift) & dm) > b) {
          const uint32_t s = atomicAdd(&sh[0], 1u);
          sel[s] = tk_pack(k, j);
        }
      }
      prefix = np;
      mask = nm;
      need -= above;
    }
    __syncthreads();
  }
  return K;
}

// Sorts the nsel selected entries by (key desc, j asc) and writes src.id of the first kout slots to o
// (-1 where the value is +-inf and for slots >= nsel).
template <class Src>
__device__ void tk_emit_sorted(const Src& src, int nsel, int kout, int* o, TopkLds& L) {
  const int tid = threadIdx.x;
  int np2 = 1;
  while (np2 < nsel) np2 <<= 1;
  for (int i = nsel + tid; i < np2; i += TK_NT) L.sel[i] = 0ull;
  __syncthreads();
  if (np2 > 1) bitonic_desc(L.sel, np2);
  for (int s = tid; s < kout; s += TK_NT) {
    int r = -1;
    if (s < nsel) {
      const unsigned long long e = L.sel[s];
      const uint32_t key = (uint32_t)(e >> 32);
      const int j = (int)(~(uint32_t)e);
      const bool isinf = key == 0xff800000u || key == 0x007fffffu;   // +inf / -inf keys
      if (!isinf) r = src.id(j);
    }
    o[s] = r;
  }
}

struct TopkParams {
  const float* lg; long long lg_st;
  const int* ctx; int rows, Lc, K;
  int* out; long long out_st;
};

__global__ void __launch_bounds__(TK_NT) topk_kernel(TopkParams p) {
  __shared__ TopkLds L;
  const int row = blockIdx.x;
  int n = p.ctx[row];
  n = n < 0 ? 0 : (n > p.Lc ? p.Lc : n);
  const RowSrc src{p.lg + (long long)row * p.lg_st, n};
  const int nsel = tk_select(src, p.K, L);
  tk_emit_sorted(src, nsel, p.K, p.out + (long long)row * p.out_st, L);
}

// fast_topk.local (dotsnote/engine/arcstats_pkg/arcstats/fast_topk.py:52-66, csrc/topk_select.cu:1-13, :75-201):
// the row's valid columns are j < ceil((ctx - rank) / P) (clipped to Lc); the top kl of them go to the payload
// pk[row] = [values fp32 | positions j * P + rank as int32 bits] in ascending column order; fewer than kl valid
// columns: the rest is padded with -inf values and positions s * P + rank.
struct LocalParams {
  const float* lg; long long lg_st;
  const int* ctx; int rows, rank, P, Lc, kl;
  float* pk;
};

__global__ void __launch_bounds__(TK_NT) topk_local_kernel(LocalParams p) {
  __shared__ TopkLds L;
  const int row = blockIdx.x, tid = threadIdx.x;
  const int c = p.ctx[row];
  int n = c > p.rank ? (int)(((long long)c - p.rank + p.P - 1) / p.P) : 0;
  if (n > p.Lc) n = p.Lc;
  const RowSrc src{p.lg + (long long)row * p.lg_st, n};
  const int nsel = tk_select(src, p.kl, L);
  // ascending column order: sort descending on ~j
  int np2 = 1;
  while (np2 < nsel) np2 <<= 1;
  for (int i = tid; i < np2; i += TK_NT) {
    unsigned long long e = 0ull;
    if (i < nsel) e = (unsigned long long)(uint32_t)L.sel[i] << 32;   // low word of a selected entry is ~j
    L.sel[i] = e;
  }
  __syncthreads();
  if (np2 > 1) bitonic_desc(L.sel, np2);
  float* pv = p.pk + (long long)row * 2 * p.kl;
  int* pp = reinterpret_cast<int*>(pv + p.kl);
  for (int s = tid; s < p.kl; s += TK_NT) {
    if (s < nsel) {
      const int j = (int)(~(uint32_t)(L.sel[s] >> 32));
      pv[s] = src.val(j);
      pp[s] = j * p.P + p.rank;
    } else {
      pv[s] = u2f(0xff800000u);
      pp[s] = s * p.P + p.rank;
    }
  }
}

// fast_topk.merge (dotsnote/engine/arcstats_pkg/arcstats/fast_topk.py:69-78, csrc/topk_select.cu:203-244): per row,
// the top kk of the P * kl all-gathered candidates by (value key desc, concatenation index asc) -> their positions,
// -1 where the value is +-inf, slots [kk, topk_tokens) = -1.
struct MergeParams {
  const float* allp; int n, P, kl, kk, topk_tokens;
  int* out; long long out_st;
};

__global__ void __launch_bounds__(TK_NT) topk_merge_kernel(MergeParams p) {
  __shared__ TopkLds L;
  const int row = blockIdx.x;
  const MergeSrc src{p.allp, p.n, row, p.kl, p.P * p.kl};
  const int nsel = tk_select(src, p.kk, L);
  tk_emit_sorted(src, nsel, p.topk_tokens, p.out + (long long)row * p.out_st, L);
}

// ------------------------------------------------------------------------------------------------ rows
// rows[t][k] = block_table[req[t]][p / bs] * stride_rows + p % bs for p = topk[t][k] >= 0 (and a valid block),
// else -1. vLLM triton_convert_req_index_to_global_index semantics (call sites dsa_sm89.py:314-315, :467-469).
__global__ void rows_kernel(const int* topk, long long tk_st, const int* req, const int* bt, long long bt_st,
                            int bt_cols, int bs, long long stride_rows, int T, int K, int* rows, long long r_st,
                            int* counts) {
  const int t = blockIdx.y;
  const int k = blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= T) return;
  int r = -1;
  if (k < K) {
    const int pp = topk[(long long)t * tk_st + k];
    if (pp >= 0 && pp / bs < bt_cols) {
      const int blk = bt[(long long)req[t] * bt_st + pp / bs];
      if (blk >= 0) r = (int)((long long)blk * stride_rows + pp % bs);
    }
    rows[(long long)t * r_st + k] = r;
  }
  if (counts) {
    const unsigned long long b = __ballot(k < K && r >= 0);
    if ((threadIdx.x & 63) == 0 && b) atomicAdd(&counts[t], __popcll(b));
  }
}

__global__ void zero_i32(int* p, int n) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) p[i] = 0;
}

}  // namespace idx
}  // namespace spmla

using namespace spmla;

extern "C" {

int spmla_index_logits(const void* q, long long q_st, long long q_sh, const float* w, long long w_st,
                       const void* store, long long R_local, int rows_per_block, long long block_stride,
                       const int* block_table, long long bt_st, int block_size, const int* req, const int* ctx,
                       int rows, int H, int D, int Lc, int P, int rank, int noinf, float* out, long long out_st,
                       void* stream) {
  if (rows < 0 || Lc < 0 || P <= 0 || rank < 0 || rank >= P || block_size <= 0 || rows_per_block <= 0) return SPMLA_EARG;
  if (rows == 0 || Lc == 0) return SPMLA_OK;
  if (H != 64 || D != 128) return SPMLA_ELIMIT;
  if (!q || !w || !store || !block_table || !req || !ctx || !out) return SPMLA_EARG;
  if (((uintptr_t)q & 15) || (q_st & 7) || (q_sh & 7) || ((uintptr_t)store & 3) || (block_stride & 3))
    return SPMLA_EALIGN;
  idx::LogitParams p;
  p.q = (const uint16_t*)q; p.q_st = q_st; p.q_sh = q_sh; p.w = w; p.w_st = w_st;
  p.store = (const uint8_t*)store; p.R_local = R_local; p.rpb = rows_per_block; p.blk_stride = block_stride;
  p.bt = block_table; p.bt_st = bt_st; p.bs = block_size; p.req = req; p.ctx = ctx;
  p.rows = rows; p.Lc = Lc; p.P = P; p.rank = rank; p.noinf = noinf; p.out = out; p.out_st = out_st;
  dim3 grid(rows, (Lc + idx::LG_KPB - 1) / idx::LG_KPB);
  hipLaunchKernelGGL(idx::logits_kernel, grid, dim3(256), 0, (hipStream_t)stream, p);
  return (int)hipGetLastError();
}

int spmla_topk(const float* logits, long long lg_st, const int* ctx, int rows, int Lc, int K, int* out,
               long long out_st, void* stream) {
  if (rows < 0 || Lc < 0 || K <= 0) return SPMLA_EARG;
  if (K > idx::TK_KMAX) return SPMLA_ELIMIT;
  if (rows == 0) return SPMLA_OK;
  if (!logits || !ctx || !out) return SPMLA_EARG;
  idx::TopkParams p;
  p.lg = logits; p.lg_st = lg_st; p.ctx = ctx; p.rows = rows; p.Lc = Lc; p.K = K; p.out = out; p.out_st = out_st;
  hipLaunchKernelGGL(idx::topk_kernel, dim3(rows), dim3(idx::TK_NT), 0, (hipStream_t)stream, p);
  return (int)hipGetLastError();
}

int spmla_topk_local(const float* logits, long long lg_st, const int* ctx, int rows, int rank, int P, int Lc, int kl,
                     float* pk, void* stream) {
  if (rows < 0 || Lc < 0 || kl <= 0 || P <= 0 || rank < 0 || rank >= P) return SPMLA_EARG;
  if (kl > idx::TK_KMAX) return SPMLA_ELIMIT;
  if (rows == 0) return SPMLA_OK;
  if (!logits || !ctx || !pk) return SPMLA_EARG;
  idx::LocalParams p;
  p.lg = logits; p.lg_st = lg_st; p.ctx = ctx; p.rows = rows; p.rank = rank; p.P = P; p.Lc = Lc; p.kl = kl; p.pk = pk;
  hipLaunchKernelGGL(idx::topk_local_kernel, dim3(rows), dim3(idx::TK_NT), 0, (hipStream_t)stream, p);
  return (int)hipGetLastError();
}

int spmla_topk_merge(const float* allp, int n, int P, int kl, int kk, int topk_tokens, int* out, long long out_st,
                     void* stream) {
  if (n < 0 || P <= 0 || kl <= 0 || kk < 0 || kk > P * kl || topk_tokens < kk) return SPMLA_EARG;
  if (kk > idx::TK_KMAX) return SPMLA_ELIMIT;
  if (n == 0 || topk_tokens == 0) return SPMLA_OK;
  if (!allp || !out) return SPMLA_EARG;
  idx::MergeParams p;
  p.allp = allp; p.n = n; p.P = P; p.kl = kl; p.kk = kk; p.topk_tokens = topk_tokens; p.out = out; p.out_st = out_st;
  hipLaunchKernelGGL(idx::topk_merge_kernel, dim3(n), dim3(idx::TK_NT), 0, (hipStream_t)stream, p);
  return (int)hipGetLastError();
}

int spmla_rows_from_topk(const int* topk, long long tk_st, const int* req, const int* block_table, long long bt_st,
                         int bt_cols, int block_size, long long stride_rows, int T, int K, int* rows, long long r_st,
                         int* counts, void* stream) {
  if (T < 0 || K < 0 || block_size <= 0 || bt_cols < 0) return SPMLA_EARG;
  if (T == 0 || K == 0) return SPMLA_OK;
  if (!topk || !req || !block_table || !rows) return SPMLA_EARG;
  if (T > 65535) return SPMLA_ELIMIT;
  if (counts)   // a fill kernel, not hipMemsetAsync: safe inside captured graphs
    hipLaunchKernelGGL(idx::zero_i32, dim3((T + 255) / 256), dim3(256), 0, (hipStream_t)stream, counts, T);
  dim3 grid((K + 255) / 256, T);
  hipLaunchKernelGGL(idx::rows_kernel, grid, dim3(256), 0, (hipStream_t)stream, topk, tk_st, req, block_table, bt_st,
                     bt_cols, block_size, stride_rows, T, K, rows, r_st, counts);
  return (int)hipGetLastError();
}

}  // extern "C"
