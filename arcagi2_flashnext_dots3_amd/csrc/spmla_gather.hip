// Row movement for the offload tiers: gather / copy of KV rows with 16-byte coalesced loads, the per-token split
// of selected rows into the HBM hot-row tier and the host tier, and the prefill compact stage.
//
// References: LayerOffload.gather / _gather_rows_kernel (dotsnote/engine/arcstats_pkg/arcstats/sparse_offload.py:
// 293-306, 1157-1163: invalid row -> zero row); the hit / miss resolution of the row cache (offload_fill.py:204-248,
// sparse_offload.py:454-456: a row lives in an HBM line or is read from host memory); compact_stage
// (dsa_sm89.py:27-35: distinct selected positions, sorted, and the selection remapped into them).
//
// Rows are moved in 16-byte chunks, a wave per row for the gather: the same code serves HBM sources and pinned host
// memory mapped into the device address space (reads then cross PCIe). The gathers also read the reference's compact
// Row400 host rows (offload_rowfmt.py: _rows_kernel / _put_rows / _copy_kernel, :163-275) and write them out in the
// GPU row formats, decoded on the way.
#include "spmla_common.h"

namespace spmla {
namespace gth {

// Row reads: one 16-byte chunk per lane through a buffer resource that spans exactly the row (none for a zero row),
// so the load has no branch: lanes past the row's end, and every lane of an absent row, read zeros. A branch-free
// load keeps the compiler's vmcnt accounting exact, which the two-rows-in-flight loops below depend on (a load
// under a branch makes every later wait drain all loads). The row address is wave-uniform (readfirstlane).
__device__ inline u32x4 load_row(const uint8_t* s, int bytes, int lane) {
  const uint64_t a = (uint64_t)(uintptr_t)s;
  const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)a), hi = __builtin_amdgcn_readfirstlane((uint32_t)(a >> 32));
  const int nb = __builtin_amdgcn_readfirstlane(s ? bytes : 0);
  const __amdgpu_buffer_rsrc_t r =
      __builtin_amdgcn_make_buffer_rsrc((void*)(uintptr_t)(((uint64_t)hi << 32) | lo), (short)0, nb, 0x00020000);
  return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, lane * 16, 0, 0));
}

// Row operations of the wave-per-row kernels. load() issues the reads of one source row (nullptr: a zero row) into
// registers, one 16-byte chunk per lane (rows of at most 64 chunks); emit() writes the destination row from them.
// The kernels keep two rows in flight per wave: the next row's load is issued before the current row is emitted,
// and its row id one step earlier still, so a wave waits on one memory round trip per row, not two.
struct CopyRow {                 // byte copy
  int chunks;                    // <= 64
  static constexpr int LDS = 0;  // LDS bytes per wave
  __device__ u32x4 load(const uint8_t* s, int lane) const { return load_row(s, chunks * 16, lane); }
  __device__ void emit(u32x4 v, bool, uint8_t* d, int lane, SPMLA_LDS uint8_t*) const {
    if (lane < chunks) *(u32x4*)(d + lane * 16) = v;
  }
};

// e2m2 code -> e4m3 code for a block exponent k >= -4, where every nonzero magnitude lands in e4m3's normal range
// (or above 448, clamped to 0x7e): the value's exponent and its 2 mantissa bits move over as they are. Equal to
// e2m2_to_e4m3 on that range.
__device__ inline uint32_t e2m2_to_e4m3_normal(uint32_t code, int k) {
  const uint32_t mag = code & 15u, e2 = mag >> 2, m = mag & 3u;
  int E;
  uint32_t mt;
  if (e2) { E = (int)e2 + k + 6; mt = m << 1; }              // (4 + m) 2^(e2 - 3 + k) = (1 + m / 4) 2^(e2 - 1 + k)
  else { E = k + 5 + (m > 1u); mt = m == 3u ? 4u : 0u; }     // m 2^(k - 2): 2^(k - 2), 2^(k - 1), 1.5 * 2^(k - 1)
  uint32_t c = mag == 0u ? 0u : (E > 15 ? 0x7eu : ((uint32_t)E << 3) | mt);
  return c | ((code & 16u) << 3);
}

// Row400 -> Row656 (fmt 0: the e4m3 codes, scales 1.0, the rope widened to bf16, which holds every e4m3 value
// exactly; the two NaN codes widen to the canonical bf16 NaN 0x7fc0, as torch's float8_e4m3fn -> bfloat16 does)
// or Row576 (fmt 1: the reference's GPU row, offload_rowfmt.py:163-171). The row arrives as 25 chunks in lanes
// 0..24 and is spread through the wave's LDS slot: lane l then decodes latent values 8l .. 8l + 7 (nibble dword l,
// sign byte l, block exponent l / 4) and lanes 0..15 move 4 rope codes each. An invalid source gives a zero row
// (scales 0, like the byte gather).
struct DecodeRow400 {
  int fmt;
  static constexpr int LDS = 416;
  __device__ u32x4 load(const uint8_t* s, int lane) const { return load_row(s, ROW400, lane); }
  __device__ void emit(u32x4 v, bool valid, uint8_t* d, int lane, SPMLA_LDS uint8_t* w) const {
    if (lane < ROW400 / 16) *(SPMLA_LDS u32x4*)(w + 16 * lane) = v;
    // LDS instructions of one wave complete in order: the reads below see every lane's write above
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    const uint32_t lo = *(const SPMLA_LDS uint32_t*)(w + 4 * lane);
    const uint32_t sg = w[R4_SIGN + lane];
    const int k = (int)(int8_t)w[R4_K + (lane >> 2)];
    const uint32_t rp = lane < 16 ? *(const SPMLA_LDS uint32_t*)(w + R4_ROPE + 4 * lane) : 0u;
    uint32_t c[2] = {0u, 0u};
    if (k >= -4) {
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const uint32_t code = ((lo >> (4 * i)) & 15u) | (((sg >> i) & 1u) << 4);
        c[i >> 2] |= e2m2_to_e4m3_normal(code, k) << (8 * (i & 3));
      }
    } else {
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const uint32_t code = ((lo >> (4 * i)) & 15u) | (((sg >> i) & 1u) << 4);
        c[i >> 2] |= (uint32_t)e2m2_to_e4m3(code, k) << (8 * (i & 3));
      }
    }
    *(uint2*)(d + 8 * lane) = make_uint2(c[0], c[1]);
    if (fmt == 0) {
      if (lane < 4) *(float*)(d + SC_OFF + 4 * lane) = valid ? 1.0f : 0.0f;
      if (lane < 16) {
        uint32_t b[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const uint8_t x = (uint8_t)(rp >> (8 * e));
          b[e] = (x & 0x7fu) == 0x7fu ? 0x7fc0u : f2u(e4m3_to_f32(x)) >> 16;
        }
        *(uint2*)(d + ROPE_OFF + 8 * lane) = make_uint2(b[0] | (b[1] << 16), b[2] | (b[3] << 16));
      }
    } else if (lane < 16) {
      *(uint32_t*)(d + D_LAT + 4 * lane) = rp;
    }
  }
};

// Row576 (the reference's per-tensor rows: 512 + 64 e4m3 codes) -> Row656 staging for the attention: the codes as
// they are, scales 1.0 (0 for an absent row, which is all zeros), the rope widened to bf16 (exact for every e4m3
// value; the NaN codes widen to 0x7fc0 as above). Lanes 0..35 hold the row's chunks: lanes 0..31 write the codes,
// lanes 32..35 widen 16 rope codes each, lanes 0..3 write the scales.
struct DecodeRow576 {
  static constexpr int LDS = 0;
  __device__ u32x4 load(const uint8_t* s, int lane) const { return load_row(s, ROW576, lane); }
  __device__ void emit(u32x4 v, bool valid, uint8_t* d, int lane, SPMLA_LDS uint8_t*) const {
    if (lane < 32) *(u32x4*)(d + 16 * lane) = v;
    if (lane < 4) *(float*)(d + SC_OFF + 4 * lane) = valid ? 1.0f : 0.0f;
    if (lane >= 32 && lane < 36) {
      uint32_t b[8];
#pragma unroll
      for (int w = 0; w < 4; ++w)
#pragma unroll
        for (int e = 0; e < 4; e += 2) {
          uint32_t h[2];
#pragma unroll
          for (int i = 0; i < 2; ++i) {
            const uint8_t x = (uint8_t)(v[w] >> (8 * (e + i)));
            h[i] = (x & 0x7fu) == 0x7fu ? 0x7fc0u : f2u(e4m3_to_f32(x)) >> 16;
          }
          b[2 * w + e / 2] = h[0] | (h[1] << 16);
        }
      uint8_t* r = d + ROPE_OFF + 32 * (lane - 32);
      *(u32x4*)r = u32x4{b[0], b[1], b[2], b[3]};
      *(u32x4*)(r + 16) = u32x4{b[4], b[5], b[6], b[7]};
    }
  }
};

__device__ inline long long readlane64(long long x, int j) {
  const uint32_t lo = __builtin_amdgcn_readlane((uint32_t)x, j), hi = __builtin_amdgcn_readlane((uint32_t)(x >> 32), j);
  return (long long)(((uint64_t)hi << 32) | lo);
}

// The rows of one wave are processed in batches of up to 64: lane j of the wave first reads the ids of the batch's
// row j (one vector load for the whole batch, one memory round trip per 64 rows), then the rows are streamed with
// the next row's data load issued before the current row is emitted (two rows in flight per wave).
template <class Op>
__device__ inline void stream_batch(const Op& op, const uint8_t* src, long long R, int src_bytes, long long r_l,
                                    long long d_l, bool skip_invalid, long long R_dst, int nb, uint8_t* dst,
                                    long long dst_stride, int lane, SPMLA_LDS uint8_t* wl) {
  auto src_of = [&](long long r) -> const uint8_t* { return (r >= 0 && r < R) ? src + r * src_bytes : nullptr; };
  long long r = readlane64(r_l, 0);
  u32x4 cur = op.load(src_of(r), lane);
  for (int j = 0; j < nb; ++j) {
    const long long rn = j + 1 < nb ? readlane64(r_l, j + 1) : -1;
    const u32x4 nxt = op.load(src_of(rn), lane);
    const long long d = readlane64(d_l, j);
    const bool ok = r >= 0 && r < R;
    if (!skip_invalid || (ok && d >= 0 && d < R_dst)) op.emit(cur, ok, dst + d * dst_stride, lane, wl);
    cur = nxt;
    r = rn;
  }
}

// dst row i (or dst_rows[i]) = src row rows[i] (0 <= rows[i] < R), zero row otherwise. One wave per row, lane c
// moving 16-byte chunk c: each row is read as one contiguous run per instruction, which measured 45.5 GB/s from
// pinned host memory over PCIe for 656-byte rows against 42.2 GB/s with consecutive threads taking consecutive chunks
// across row boundaries (the rows' start addresses then split more requests). With dst_rows, pairs whose
// destination is outside [0, R_dst) or whose source is invalid are skipped instead.
template <class Op>
__global__ void __launch_bounds__(256) gather_kernel(const uint8_t* __restrict__ src, long long R, int src_bytes,
                                                     const long long* __restrict__ rows, int n,
                                                     uint8_t* __restrict__ dst, long long dst_stride,
                                                     const long long* __restrict__ dst_rows, long long R_dst, Op op,
                                                     const int* __restrict__ n_dev = nullptr) {
  __shared__ __attribute__((aligned(16))) uint8_t wl_all[4 * Op::LDS + 16];
  if (n_dev) n = min(n, *n_dev);                      // a count produced on the device (the cache's miss list)
  const int lane = threadIdx.x & 63, wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  SPMLA_LDS uint8_t* wl = (SPMLA_LDS uint8_t*)wl_all + wv * Op::LDS;
  const int step = gridDim.x * 4;
  for (int i0 = blockIdx.x * 4 + wv; i0 < n; i0 += 64 * step) {
    const int il = i0 + lane * step;                  // this lane's row of the batch
    long long r_l = -1, d_l = il;
    if (il < n) {
      r_l = rows[il];
      if (dst_rows) d_l = dst_rows[il];
    }
    const int nb = min(64, (n - i0 + step - 1) / step);
    stream_batch(op, src, R, src_bytes, r_l, d_l, dst_rows != nullptr, R_dst, nb, dst, dst_stride, lane, wl);
  }
}

// Host-tier staging: dst row t * K + k = src row rows[t][k] for k < counts[t] (zero row if rows[t][k] is outside
// [0, R)); other rows untouched, except that row 0 is zeroed when token 0 has no rows (the attention reads row 0 of
// its pool for masked entries, which must then be finite). Persistent grid: tokens are taken 1024 at a time, the
// counts' prefix sum goes to LDS and every wave copies entries v = wave, wave + waves, ... of the chunk, each lane
// locating its batch entry's token by binary search in the prefix.
template <class Op>
__global__ void __launch_bounds__(256) gather_tiers_kernel(const uint8_t* __restrict__ src, long long R, int src_bytes,
                                                           const int* __restrict__ rows, long long r_st,
                                                           const int* __restrict__ counts, int T, int K,
                                                           uint8_t* __restrict__ dst, long long dst_stride, Op op) {
  __shared__ int pre[1025];
  __shared__ int wsum[4];
  __shared__ __attribute__((aligned(16))) uint8_t wl_all[4 * Op::LDS + 16];
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int wu = __builtin_amdgcn_readfirstlane(wv);
  SPMLA_LDS uint8_t* wl = (SPMLA_LDS uint8_t*)wl_all + wu * Op::LDS;
  const int nw = gridDim.x * 4, gw = blockIdx.x * 4 + wu;
  if (gw == 0 && counts[0] <= 0) op.emit(op.load(nullptr, lane), false, dst, lane, wl);
  for (int t0 = 0; t0 < T; t0 += 1024) {
    const int nt = min(1024, T - t0);
    // inclusive prefix of clamp(counts[t0 + t], 0, K): thread tid sums tokens 4 tid .. 4 tid + 3
    int c4[4], s = 0;
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int t = 4 * tid + u;
      c4[u] = t < nt ? min(max(counts[t0 + t], 0), K) : 0;
      s += c4[u];
    }
    int inc = s;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
      const int y = __shfl_up(inc, o, 64);
      if (lane >= o) inc += y;
    }
    if (lane == 63) wsum[wv] = inc;
    __syncthreads();
    int base = 0;
#pragma unroll
    for (int w = 0; w < 4; ++w) base += w < wv ? wsum[w] : 0;
    int run = base + inc - s;
    if (tid == 0) pre[0] = 0;
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      run += c4[u];
      if (4 * tid + u < nt) pre[4 * tid + u + 1] = run;
    }
    __syncthreads();
    const int tot = pre[nt];
    for (int v0 = gw; v0 < tot; v0 += 64 * nw) {
      const int vl = v0 + lane * nw;                 // this lane's entry of the batch
      long long r_l = -1, d_l = 0;
      if (vl < tot) {
        int lo = 0, hi = nt - 1;                     // largest t with pre[t] <= vl
        while (lo < hi) {
          const int mid = (lo + hi + 1) >> 1;
          if (pre[mid] <= vl) lo = mid;
          else hi = mid - 1;
        }
        const int t = t0 + lo, k = vl - pre[lo];
        r_l = rows[(long long)t * r_st + k];
        d_l = (long long)t * K + k;
      }
      const int nb = min(64, (tot - v0 + nw - 1) / nw);
      stream_batch(op, src, R, src_bytes, r_l, d_l, false, 0ll, nb, dst, dst_stride, lane, wl);
    }
    __syncthreads();                                 // pre[] is rewritten for the next chunk
  }
}

// dst row dst_rows[i] = src row src_rows[i]; pairs with an invalid side are skipped.
__global__ void copy_kernel(const uint8_t* src, long long R_src, const long long* src_rows, uint8_t* dst,
                            long long R_dst, const long long* dst_rows, int row_bytes, int n) {
  const int chunks = row_bytes >> 4;
  const long long g = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  if (g >= (long long)n * chunks) return;
  const int i = (int)(g / chunks), c = (int)(g % chunks);
  const long long s = src_rows[i], d = dst_rows[i];
  if (s < 0 || s >= R_src || d < 0 || d >= R_dst) return;
  *(u32x4*)(dst + d * row_bytes + c * 16) = *(const u32x4*)(src + s * row_bytes + c * 16);
}

// Per token (one 256-thread block): entries of idx[t] in order; a valid host row h with rowmap[h] >= 0 goes to
// the HBM tier as line rowmap[h], other valid rows to the host tier as h. Both lists are compacted stably and padded
// with -1 to K; counts[t] = number of entries of each list. Thread tid takes 8 consecutive entries of each
// 2048-entry chunk, so all of its index and rowmap reads are in flight together (one dependent pair of memory round
// trips per chunk), and one block scan of the packed per-thread counts places them.
__global__ void __launch_bounds__(256) tier_split_kernel(const int* __restrict__ idx, long long idx_st, int K,
                                                         const int* __restrict__ rowmap, long long R,
                                                         int* __restrict__ hbm, long long hbm_st, int* __restrict__ hcnt,
                                                         int* __restrict__ host, long long host_st,
                                                         int* __restrict__ scnt) {
  __shared__ uint32_t wsum[4];
  const int t = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int* ir = idx + (long long)t * idx_st;
  int* hr = hbm + (long long)t * hbm_st;
  int* sr = host + (long long)t * host_st;
  uint32_t nh = 0, ns = 0;
  for (int k0 = 0; k0 < K; k0 += 2048) {
    int h[8], line[8];
    bool ok[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int k = k0 + 8 * tid + u;
      h[u] = k < K ? ir[k] : -1;
    }
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      ok[u] = h[u] >= 0 && (long long)h[u] < R;
      line[u] = ok[u] ? rowmap[h[u]] : -1;
    }
    uint32_t c = 0;                                  // hbm count | host count << 16
#pragma unroll
    for (int u = 0; u < 8; ++u) c += ok[u] ? (line[u] >= 0 ? 1u : 0x10000u) : 0u;
    uint32_t inc = c;
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
    const uint32_t ex = base + inc - c;
    uint32_t oh = nh + (ex & 0xffffu), os = ns + (ex >> 16);
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      if (ok[u] && line[u] >= 0) hr[oh++] = line[u];
      else if (ok[u]) sr[os++] = h[u];
    }
    nh += tot & 0xffffu;
    ns += tot >> 16;
    __syncthreads();                                 // wsum is rewritten for the next chunk
  }
  for (int k = nh + tid; k < K; k += 256) hr[k] = -1;
  for (int k = ns + tid; k < K; k += 256) sr[k] = -1;
  if (tid == 0) { hcnt[t] = (int)nh; scnt[t] = (int)ns; }
}

// ---- compact stage: bitmap of selected positions -> ranks
__global__ void zero_u32(uint32_t* p, long long n) {
  const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) p[i] = 0u;
}

__global__ void mark_kernel(const int* sidx, long long s_st, int M, int K, int tot, uint32_t* bits) {
  const long long g = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  if (g >= (long long)M * K) return;
  const int m = (int)(g / K), k = (int)(g % K);
  const int p = sidx[(long long)m * s_st + k];
  if (p >= 0 && p < tot) atomicOr(&bits[p >> 5], 1u << (p & 31));
}

// one 1024-thread block: exclusive prefix of popcounts over W words -> woff[W], total -> *U
__global__ void __launch_bounds__(1024) scan_kernel(const uint32_t* bits, int W, uint32_t* woff, int* U) {
  __shared__ uint32_t part[1024];
  __shared__ uint32_t wsum[17];
  const int tid = threadIdx.x;
  const int per = (W + 1023) / 1024;
  const int w0 = tid * per;
  uint32_t s = 0;
  for (int i = 0; i < per && w0 + i < W; ++i) s += __popc(bits[w0 + i]);
  // block exclusive scan of s
  const int lane = tid & 63, wv = tid >> 6;
  uint32_t inc = s;
  for (int o = 1; o < 64; o <<= 1) {
    const uint32_t t = __shfl_up(inc, o, 64);
    if (lane >= o) inc += t;
  }
  if (lane == 63) wsum[wv] = inc;
  __syncthreads();
  if (wv == 0) {
    const uint32_t w = lane < 16 ? wsum[lane] : 0u;
    uint32_t wi = w;
    for (int o = 1; o < 16; o <<= 1) {
      const uint32_t t = __shfl_up(wi, o, 64);
      if (lane >= o) wi += t;
    }
    if (lane < 16) wsum[lane] = wi - w;
    if (lane == 15) wsum[16] = wi;
  }
  __syncthreads();
  uint32_t run = wsum[wv] + inc - s;
  for (int i = 0; i < per && w0 + i < W; ++i) {
    woff[w0 + i] = run;
    run += __popc(bits[w0 + i]);
  }
  if (tid == 0) *U = (int)wsum[16];
  (void)part;
}

__device__ inline uint32_t rank_of(const uint32_t* bits, const uint32_t* woff, int p) {
  const uint32_t w = bits[p >> 5];
  return woff[p >> 5] + __popc(w & ((1u << (p & 31)) - 1u));
}

__global__ void emit_kernel(const uint32_t* bits, const uint32_t* woff, int tot, const long long* rows,
                            long long* sel) {
  const int p = blockIdx.x * blockDim.x + threadIdx.x;
  if (p >= tot) return;
  if (bits[p >> 5] & (1u << (p & 31))) sel[rank_of(bits, woff, p)] = rows[p];
}

__global__ void remap_kernel(const int* sidx, long long s_st, int M, int K, int tot, const uint32_t* bits,
                             const uint32_t* woff, int* sidx2, long long s2_st) {
  const long long g = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  if (g >= (long long)M * K) return;
  const int m = (int)(g / K), k = (int)(g % K);
  const int p = sidx[(long long)m * s_st + k];
  sidx2[(long long)m * s2_st + k] = (p >= 0 && p < tot) ? (int)rank_of(bits, woff, p) : -1;
}

// ---- Row400 -> GPU rows from HBM, 16 lanes per row: lane q of a row's group decodes latent block q (32 values, one
// block exponent k), so a row's decode is spread over 16 lanes and a wave decodes 4 rows at once; every thread
// decodes one block, and the grid covers all rows (occupancy, not a per-wave pipeline, hides the memory latency).
// For -4 <= k <= 6 (every block the writer produces from values up to 448 with amax / 7 >= 2^-5) the e4m3 code of
// magnitude nibble m is a byte table T_k[m]: 0, (k + 5) << 3, (k + 6) << 3, ((k + 6) << 3) | 4 for m = 0 .. 3 (the
// e2m2 subnormals) and (m << 1) + ((k + 6) << 3) for m >= 4 (exponent and 2 mantissa bits moved over); the lookup of
// 4 nibbles takes two v_perm_b32 over the 16-byte table and a byte select. Other blocks go through e2m2_to_e4m3 per
// value. The sign bit is ORed in after (-0 -> 0x80, as e2m2_to_e4m3).
__device__ inline uint32_t r4_lut4(uint32_t x, uint32_t t0, uint32_t t1, uint32_t t2, uint32_t t3) {
  const uint32_t s7 = x & 0x07070707u;
  const uint32_t lo = __builtin_amdgcn_perm(t1, t0, s7), hi = __builtin_amdgcn_perm(t3, t2, s7);
  // selector 12 gives byte 0x00, 13 gives 0xff: the mask of the nibbles with bit 3 set
  const uint32_t mask = __builtin_amdgcn_perm(0u, 0u, ((x >> 3) & 0x01010101u) | 0x0c0c0c0cu);
  return (hi & mask) | (lo & ~mask);
}
// bits 0..3 of t -> bit 7 of bytes 0..3 (four shifted copies of t; no two of them overlap)
__device__ inline uint32_t r4_sign4(uint32_t t) { return ((t << 7) * 0x204081u) & 0x80808080u; }

// Entry i of the launch: rows64 (n entries, dst row i), or the token lists rows32 [T][r_st] with counts (dst row
// t * K + k for k < counts[t], later entries skipped; no counts: every entry).
struct DecodeList {
  const long long* rows64; int n;
  const int* rows32; long long r_st; const int* counts; int T, K;
};

__global__ void __launch_bounds__(256) decode400_kernel(const uint8_t* __restrict__ src, long long R, DecodeList L,
                                                        uint8_t* __restrict__ dst, long long dst_stride, int fmt) {
  const long long g = (long long)blockIdx.x * 256 + threadIdx.x;
  const long long i = g >> 4;
  const int q = (int)(g & 15);
  long long r;
  if (L.rows64) {
    if (i >= L.n) return;
    r = L.rows64[i];
  } else {
    if (i >= (long long)L.T * L.K) return;
    const int t = (int)(i / L.K), k = (int)(i - (long long)t * L.K);
    if (L.counts && k >= L.counts[t]) return;
    r = L.rows32[(long long)t * L.r_st + k];
  }
  const bool ok = r >= 0 && r < R;
  const uint8_t* s = src + (ok ? r : 0) * ROW400;
  u32x4 nib = {0u, 0u, 0u, 0u};
  uint32_t sg = 0u;
  int k = 0;
  u32x4 rp = {0u, 0u, 0u, 0u};
  if (ok) {
    nib = *(const u32x4*)(s + 16 * q);
    sg = *(const uint32_t*)(s + R4_SIGN + 4 * q);
    k = (int)(int8_t)s[R4_K + q];
    if (fmt == 1 ? q < 4 : q < 8) {
      if (fmt == 1) rp = *(const u32x4*)(s + R4_ROPE + 16 * q);
      else { const uint2 v = *(const uint2*)(s + R4_ROPE + 8 * q); rp[0] = v.x; rp[1] = v.y; }
    }
  }
  uint8_t* d = dst + i * dst_stride;
  uint32_t c[8];
  if (k >= -4 && k <= 6) {
    const uint32_t kb = (uint32_t)(k + 6) << 3;             // 16 .. 96
    const uint32_t k4 = kb * 0x01010101u;
    const uint32_t t0 = (k4 & 0xffffff00u) + 0x03fff800u;    // 0, kb - 8, kb, kb + 4
    const uint32_t t1 = k4 + 0x0e0c0a08u, t2 = k4 + 0x16141210u, t3 = k4 + 0x1e1c1a18u;
#pragma unroll
    for (int w = 0; w < 4; ++w) {                            // values 8w .. 8w + 7
      const uint32_t ce = r4_lut4(nib[w] & 0x0f0f0f0fu, t0, t1, t2, t3);          // values 8w + 0, 2, 4, 6
      const uint32_t co = r4_lut4((nib[w] >> 4) & 0x0f0f0f0fu, t0, t1, t2, t3);   // values 8w + 1, 3, 5, 7
      c[2 * w] = __builtin_amdgcn_perm(co, ce, 0x05010400u) | r4_sign4((sg >> (8 * w)) & 15u);
      c[2 * w + 1] = __builtin_amdgcn_perm(co, ce, 0x07030602u) | r4_sign4((sg >> (8 * w + 4)) & 15u);
    }
  } else {
#pragma unroll
    for (int w = 0; w < 8; ++w) {
      uint32_t x = 0u;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int j = 4 * w + e;
        const uint32_t code = ((nib[j >> 3] >> (4 * (j & 7))) & 15u) | (((sg >> j) & 1u) << 4);
        x |= (uint32_t)e2m2_to_e4m3(code, k) << (8 * e);
      }
      c[w] = x;
    }
  }
  *(u32x4*)(d + 32 * q) = u32x4{c[0], c[1], c[2], c[3]};
  *(u32x4*)(d + 32 * q + 16) = u32x4{c[4], c[5], c[6], c[7]};
  if (fmt == 1) {
    if (q < 4) *(u32x4*)(d + D_LAT + 16 * q) = rp;
  } else {
    if (q < 4) *(float*)(d + SC_OFF + 4 * q) = ok ? 1.0f : 0.0f;
    if (q < 8) {
      uint32_t b[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const uint8_t x = (uint8_t)(rp[e >> 2] >> (8 * (e & 3)));
        b[e] = (x & 0x7fu) == 0x7fu ? 0x7fc0u : f2u(e4m3_to_f32(x)) >> 16;
      }
      *(u32x4*)(d + ROPE_OFF + 16 * q) = u32x4{b[0] | (b[1] << 16), b[2] | (b[3] << 16), b[4] | (b[5] << 16),
                                               b[6] | (b[7] << 16)};
    }
  }
}

}  // namespace gth
}  // namespace spmla

using namespace spmla;

extern "C" {

static int gather_launch(const void* src, long long R, int row_bytes, const long long* rows, int n, void* dst,
                         long long dst_stride, unsigned max_wg, void* stream) {
  if (n < 0 || R < 0 || row_bytes <= 0 || (row_bytes & 15)) return SPMLA_EARG;
  if (row_bytes > 1024) return SPMLA_ELIMIT;          // one 16-byte chunk per lane
  if (n == 0) return SPMLA_OK;
  if (!src || !rows || !dst) return SPMLA_EARG;
  if (((uintptr_t)src & 15) || ((uintptr_t)dst & 15) || (dst_stride & 15) || dst_stride < row_bytes) return SPMLA_EALIGN;
  unsigned grid = (unsigned)((n + 3) / 4);
  if (grid > max_wg) grid = max_wg;
  hipLaunchKernelGGL(gth::gather_kernel<gth::CopyRow>, dim3(grid), dim3(256), 0, (hipStream_t)stream,
                     (const uint8_t*)src, R, row_bytes, rows, n, (uint8_t*)dst, dst_stride, (const long long*)nullptr,
                     0ll, gth::CopyRow{row_bytes >> 4});
  return (int)hipGetLastError();
}

int spmla_gather(const void* src, long long R, int row_bytes, const long long* rows, int n, void* dst,
                 long long dst_stride, void* stream) {
  return gather_launch(src, R, row_bytes, rows, n, dst, dst_stride, 0xffffffffu, stream);
}

int spmla_gather_tiers(const void* src, long long R, int row_bytes, const int* rows, long long r_st, const int* counts,
                       int T, int K, void* dst, long long dst_stride, void* stream) {
  if (T < 0 || K < 0 || R < 0 || row_bytes <= 0 || (row_bytes & 15) || r_st < K) return SPMLA_EARG;
  if (row_bytes > 1024) return SPMLA_ELIMIT;
  if (T == 0 || K == 0) return SPMLA_OK;
  if (!src || !rows || !counts || !dst) return SPMLA_EARG;
  if (((uintptr_t)src & 15) || ((uintptr_t)dst & 15) || (dst_stride & 15) || dst_stride < row_bytes) return SPMLA_EALIGN;
  hipLaunchKernelGGL(gth::gather_tiers_kernel<gth::CopyRow>, dim3(64), dim3(256), 0, (hipStream_t)stream,
                     (const uint8_t*)src, R, row_bytes, rows, r_st, counts, T, K, (uint8_t*)dst, dst_stride,
                     gth::CopyRow{row_bytes >> 4});
  return (int)hipGetLastError();
}

// ---- the W-way row cache's fill: every miss m < state[1] with miss_dst[m] >= 0 gets its host row (Row656 bytes, a
// Row400 row decoded to Row656, or Row400 bytes into Row400 lines) at pool row miss_dst[m]; spmla_wcache_step
// produced the list
int spmla_wcache_fill(const void* host, long long R, int host_fmt, int pool_fmt, const long long* miss_rows,
                      const long long* miss_dst, const int* state, int n_max, void* pool, long long R_pool,
                      void* stream) {
  if (R < 0 || n_max < 0 || R_pool < 0 || (host_fmt != 0 && host_fmt != 2)) return SPMLA_EARG;
  if (pool_fmt != 0 && !(pool_fmt == 2 && host_fmt == 2)) return SPMLA_EARG;
  if (n_max == 0) return SPMLA_OK;
  if (!host || !miss_rows || !miss_dst || !state || !pool) return SPMLA_EARG;
  if (((uintptr_t)host & 15) || ((uintptr_t)pool & 15)) return SPMLA_EALIGN;
  const unsigned grid = (unsigned)min(64, (n_max + 3) / 4);
  if (pool_fmt == 2)
    hipLaunchKernelGGL(gth::gather_kernel<gth::CopyRow>, dim3(grid), dim3(256), 0, (hipStream_t)stream,
                       (const uint8_t*)host, R, ROW400, miss_rows, n_max, (uint8_t*)pool, (long long)ROW400, miss_dst,
                       R_pool, gth::CopyRow{ROW400 / 16}, state + 1);
  else if (host_fmt == 0)
    hipLaunchKernelGGL(gth::gather_kernel<gth::CopyRow>, dim3(grid), dim3(256), 0, (hipStream_t)stream,
                       (const uint8_t*)host, R, ROW656, miss_rows, n_max, (uint8_t*)pool, (long long)ROW656, miss_dst,
                       R_pool, gth::CopyRow{ROW656 / 16}, state + 1);
  else
    hipLaunchKernelGGL(gth::gather_kernel<gth::DecodeRow400>, dim3(grid), dim3(256), 0, (hipStream_t)stream,
                       (const uint8_t*)host, R, ROW400, miss_rows, n_max, (uint8_t*)pool, (long long)ROW656, miss_dst,
                       R_pool, gth::DecodeRow400{0}, state + 1);
  return (int)hipGetLastError();
}

// ---- Row400 (compact host rows) in, Row656 / Row576 out
static int row400_dst_bytes(int dst_fmt) { return dst_fmt == 0 ? ROW656 : (dst_fmt == 1 ? ROW576 : 0); }

int spmla_row400_gather(const void* src, long long R, const long long* rows, int n, void* dst, long long dst_stride,
                        int dst_fmt, int pcie, void* stream) {
  const int db = row400_dst_bytes(dst_fmt);
  if (n < 0 || R < 0 || db == 0) return SPMLA_EARG;
  if (n == 0) return SPMLA_OK;
  if (!src || !rows || !dst) return SPMLA_EARG;
  if (((uintptr_t)src & 15) || ((uintptr_t)dst & 15) || (dst_stride & 15) || dst_stride < db) return SPMLA_EALIGN;
  if (!pcie) {                      // HBM source: 16 lanes per row, every row's blocks in flight at once
    if ((long long)n * 16 > (1ll << 31) - 256) return SPMLA_ELIMIT;
    const gth::DecodeList L{rows, n, nullptr, 0, nullptr, 0, 0};
    hipLaunchKernelGGL(gth::decode400_kernel, dim3((unsigned)(((long long)n * 16 + 255) / 256)), dim3(256), 0,
                       (hipStream_t)stream, (const uint8_t*)src, R, L, (uint8_t*)dst, dst_stride, dst_fmt);
    return (int)hipGetLastError();
  }
  // pinned host source: a wave per row on 64 workgroups (PCIe-bound; see the gathers above)
  unsigned grid = (unsigned)((n + 3) / 4);
  if (grid > 64u) grid = 64u;
  hipLaunchKernelGGL(gth::gather_kernel<gth::DecodeRow400>, dim3(grid), dim3(256), 0, (hipStream_t)stream,
                     (const uint8_t*)src, R, ROW400, rows, n, (uint8_t*)dst, dst_stride, (const long long*)nullptr,
                     0ll, gth::DecodeRow400{dst_fmt});
  return (int)hipGetLastError();
}

int spmla_row576_gather(const void* src, long long R, const long long* rows, int n, void* dst, long long dst_stride,
                        void* stream) {
  if (n < 0 || R < 0) return SPMLA_EARG;
  if (n == 0) return SPMLA_OK;
  if (!src || !rows || !dst) return SPMLA_EARG;
  if (((uintptr_t)src & 15) || ((uintptr_t)dst & 15) || (dst_stride & 15) || dst_stride < ROW656) return SPMLA_EALIGN;
  hipLaunchKernelGGL(gth::gather_kernel<gth::DecodeRow576>, dim3((unsigned)((n + 3) / 4)), dim3(256), 0,
                     (hipStream_t)stream, (const uint8_t*)src, R, ROW576, rows, n, (uint8_t*)dst, dst_stride,
                     (const long long*)nullptr, 0ll, gth::DecodeRow576{});
  return (int)hipGetLastError();
}

int spmla_row400_copy(const void* src, long long R_src, const long long* src_rows, void* dst, long long R_dst,
                      const long long* dst_rows, int n, int dst_fmt, void* stream) {
  const int db = row400_dst_bytes(dst_fmt);
  if (n < 0 || R_src < 0 || R_dst < 0 || db == 0) return SPMLA_EARG;
  if (n == 0) return SPMLA_OK;
  if (!src || !dst || !src_rows || !dst_rows) return SPMLA_EARG;
  if (((uintptr_t)src & 15) || ((uintptr_t)dst & 15)) return SPMLA_EALIGN;
  hipLaunchKernelGGL(gth::gather_kernel<gth::DecodeRow400>, dim3((unsigned)((n + 3) / 4)), dim3(256), 0,
                     (hipStream_t)stream, (const uint8_t*)src, R_src, ROW400, src_rows, n, (uint8_t*)dst,
                     (long long)db, dst_rows, R_dst, gth::DecodeRow400{dst_fmt});
  return (int)hipGetLastError();
}

int spmla_row400_gather_tiers(const void* src, long long R, const int* rows, long long r_st, const int* counts, int T,
                              int K, void* dst, long long dst_stride, int dst_fmt, void* stream) {
  const int db = row400_dst_bytes(dst_fmt);
  if (T < 0 || K < 0 || R < 0 || r_st < K || db == 0) return SPMLA_EARG;
  if (T == 0 || K == 0) return SPMLA_OK;
  if (!src || !rows || !counts || !dst) return SPMLA_EARG;
  if (((uintptr_t)src & 15) || ((uintptr_t)dst & 15) || (dst_stride & 15) || dst_stride < db) return SPMLA_EALIGN;
  hipLaunchKernelGGL(gth::gather_tiers_kernel<gth::DecodeRow400>, dim3(64), dim3(256), 0, (hipStream_t)stream,
                     (const uint8_t*)src, R, ROW400, rows, r_st, counts, T, K, (uint8_t*)dst, dst_stride,
                     gth::DecodeRow400{dst_fmt});
  return (int)hipGetLastError();
}

int spmla_row400_decode_tiers(const void* src, long long R, const int* rows, long long r_st, const int* counts, int T,
                              int K, void* dst, long long dst_stride, int dst_fmt, void* stream) {
  const int db = row400_dst_bytes(dst_fmt);
  if (T < 0 || K < 0 || R < 0 || r_st < K || db == 0) return SPMLA_EARG;
  if (T == 0 || K == 0) return SPMLA_OK;
  if (!src || !rows || !dst) return SPMLA_EARG;
  if (((uintptr_t)src & 15) || ((uintptr_t)dst & 15) || (dst_stride & 15) || dst_stride < db) return SPMLA_EALIGN;
  if ((long long)T * K * 16 > (1ll << 31) - 256) return SPMLA_ELIMIT;
  const gth::DecodeList L{nullptr, 0, rows, r_st, counts, T, K};
  hipLaunchKernelGGL(gth::decode400_kernel, dim3((unsigned)(((long long)T * K * 16 + 255) / 256)), dim3(256), 0,
                     (hipStream_t)stream, (const uint8_t*)src, R, L, (uint8_t*)dst, dst_stride, dst_fmt);
  return (int)hipGetLastError();
}

// 64 workgroups x 4 waves = 256 rows in flight: 45.7 GB/s from pinned host memory (the full grid: 45.8 GB/s), on a
// quarter of the CUs.
int spmla_gather_pcie(const void* src, long long R, int row_bytes, const long long* rows, int n, void* dst,
                      long long dst_stride, void* stream) {
  return gather_launch(src, R, row_bytes, rows, n, dst, dst_stride, 64u, stream);
}

int spmla_copy_rows(const void* src, long long R_src, const long long* src_rows, void* dst, long long R_dst,
                    const long long* dst_rows, int row_bytes, int n, void* stream) {
  if (n < 0 || R_src < 0 || R_dst < 0 || row_bytes <= 0 || (row_bytes & 15)) return SPMLA_EARG;
  if (n == 0) return SPMLA_OK;
  if (!src || !dst || !src_rows || !dst_rows) return SPMLA_EARG;
  if (((uintptr_t)src & 15) || ((uintptr_t)dst & 15)) return SPMLA_EALIGN;
  const long long work = (long long)n * (row_bytes >> 4);
  hipLaunchKernelGGL(gth::copy_kernel, dim3((unsigned)((work + 255) / 256)), dim3(256), 0, (hipStream_t)stream,
                     (const uint8_t*)src, R_src, src_rows, (uint8_t*)dst, R_dst, dst_rows, row_bytes, n);
  return (int)hipGetLastError();
}

int spmla_tier_split(const int* idx, long long idx_st, int T, int K, const int* rowmap, long long R, int* hbm_idx,
                     long long hbm_st, int* hbm_cnt, int* host_idx, long long host_st, int* host_cnt, void* stream) {
  if (T < 0 || K < 0 || R < 0) return SPMLA_EARG;
  if (T == 0) return SPMLA_OK;
  if (!idx || !rowmap || !hbm_idx || !hbm_cnt || !host_idx || !host_cnt) return SPMLA_EARG;
  hipLaunchKernelGGL(gth::tier_split_kernel, dim3(T), dim3(256), 0, (hipStream_t)stream, idx, idx_st, K, rowmap, R,
                     hbm_idx, hbm_st, hbm_cnt, host_idx, host_st, host_cnt);
  return (int)hipGetLastError();
}

// workspace: 2 * ceil(tot / 32) uint32 words (bitmap + word offsets), caller-owned.
int spmla_compact_stage(const long long* rows, int tot, const int* sidx, long long s_st, int M, int K, void* workspace,
                        long long* sel, int* U, int* sidx2, long long s2_st, void* stream) {
  if (tot < 0 || M < 0 || K < 0) return SPMLA_EARG;
  if (!U || (tot > 0 && (!rows || !workspace || !sel)) || (M > 0 && K > 0 && (!sidx || !sidx2))) return SPMLA_EARG;
  hipStream_t s = (hipStream_t)stream;
  const int W = (tot + 31) / 32;
  uint32_t* bits = (uint32_t*)workspace;
  uint32_t* woff = bits + W;
  if (W > 0)
    hipLaunchKernelGGL(gth::zero_u32, dim3((W + 255) / 256), dim3(256), 0, s, bits, (long long)W);
  const long long mk = (long long)M * K;
  if (mk > 0 && W > 0)
    hipLaunchKernelGGL(gth::mark_kernel, dim3((unsigned)((mk + 255) / 256)), dim3(256), 0, s, sidx, s_st, M, K, tot, bits);
  hipLaunchKernelGGL(gth::scan_kernel, dim3(1), dim3(1024), 0, s, bits, W, woff, U);
  if (tot > 0)
    hipLaunchKernelGGL(gth::emit_kernel, dim3((tot + 255) / 256), dim3(256), 0, s, bits, woff, tot, rows, sel);
  if (mk > 0)
    hipLaunchKernelGGL(gth::remap_kernel, dim3((unsigned)((mk + 255) / 256)), dim3(256), 0, s, sidx, s_st, M, K, tot,
                       bits, woff, sidx2, s2_st);
  return (int)hipGetLastError();
}

}  // extern "C"
