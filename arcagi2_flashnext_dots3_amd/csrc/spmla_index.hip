// Indexer logits and exact top-k selection.
//
// Logits (dotsnote/engine/arcstats_pkg/arcstats/shard_logits_v2.py:49-123, shard_indexer.py:63-91; torch statement
// dotsnote/training/finetune/student.py:219-222):
//   logit[row][j] = min(sum_h w[row][h] * relu(q[row][h] . kcode[j]) * ks[j], 60000) for positions j < ctx[row]
//   (column j holds position j * P + rank of this rank's key store), -inf for j >= ctx (unless noinf); stored as fp32,
//   or rounded to fp16 (the reference's ARC_SHARD_F16OUT buffer, shard_indexer.py:28-29, :124).
//   gfx950: each wave loads the codes of its 32-key tiles straight into the registers of the MFMA B operand (three
//   tiles of loads in flight; the logits of a workgroup staged in LDS and written once its waves are done);
//   S = Q K^T on bf16 MFMA (32x32x16; e4m3 key codes convert exactly to bf16, two per instruction), 64 heads = 2 M
//   blocks, keys as the B operand; the head reduction is in-lane plus one cross-half exchange. (The fp8 MFMA would take the codes directly, but its internal accumulation keeps only
//   ~2^-12 of the largest product on gfx950, too coarse for the selection.)
//
// Top-k (dotsnote/engine/arcstats_pkg/arcstats/fast_topk.py:1-15, csrc/topk_select.cu:1-30 semantics):
//   per row, the K largest values among columns j < n = min(ctx, Lc) by torch's order-preserving key
//   (-0 < +0, NaN largest); equal keys -> lower column first; output positions sorted by (value desc, column asc),
//   -1 where the value is +-inf and in slots >= n. fp32 or fp16 logits: an fp16 key is the same order key of the
//   16-bit pattern placed in the top half of the 32-bit key (low half zero), so one radix code serves both.
//   gfx950: one 1024-thread workgroup per row, the row's keys in VGPRs (32 per thread, all loads in flight):
//   11/11/10-bit radix levels with an LDS histogram; keys above the boundary bin are appended at slots from a block
//   scan of per-thread counts (wave scans on DPP); once the boundary bin holds at most the candidate cap the remaining
//   levels run on those candidates alone; ties on the final key take the lowest columns. The K winners are
//   bitonic-sorted in LDS (only the stages whose pairs cross waves take a workgroup barrier); on the several-
//   workgroup path, whose lists arrive in column order, fp16 winners are ordered by a stable radix sort instead.
#include "spmla_common.h"
#include <limits.h>
#include <algorithm>

namespace spmla {
namespace idx {

// torch's order-preserving key of an fp32 value (the top-k's radix key; -0 < +0, NaN largest)
__device__ inline uint32_t okey(float v) {
  const uint32_t x = f2u(v);
  if (v != v) return 0xffffffffu;
  return (x & 0x80000000u) ? ~x : (x | 0x80000000u);
}
// the same key for an fp16 pattern, in the top 16 bits (low 16 bits zero; NaN largest)
__device__ inline uint32_t okey16(uint32_t h) {
  if ((h & 0x7fffu) > 0x7c00u) return 0xffff0000u;
  return ((h & 0x8000u) ? (~h & 0xffffu) : (h | 0x8000u)) << 16;
}

// ------------------------------------------------------------------------------------------------ logits
constexpr int LG_NWV = 8;                 // waves per logits workgroup (2 per SIMD: 256 registers each)
constexpr int LG_TPW = 16;                // 32-key tiles per wave and workgroup when the rows overfill the device

struct LogitParams {
  const uint16_t* q; long long q_st, q_sh;   // q[row][64][128] bf16
  const float* w; long long w_st;            // w[row][64]
  const uint8_t* store; long long R_local; int rpb; long long blk_stride;
  const int* bt; long long bt_st; int bs;    // block table [req][...], block size (positions per block)
  const int* req; const int* ctx;            // per row
  int rows, Lc, P, rank, noinf;
  void* out; long long out_st;              // fp32, or fp16 (F16OUT); stride in elements
  int bs_sh, rpb_sh, p_sh;                   // log2 of bs, rpb, P when a power of two, else -1
  long long lim;                             // R_local * P (< 2^31): valid block-table positions lie below
  int clamp;                                 // 1: logits clamped at 60000 (shard kernels); 0: unclamped (paged)
  const int* lo;                             // optional per-row first valid position (flat layout: cu_seqlen_ks)
  const float* kscale; long long k_st;       // flat layout: key j codes at store + j * k_st, scale kscale[j]
  int tpg;                                   // 32-key tiles per workgroup (the launcher's lg_grid)
  // optional level-0 top-k histograms (P == 1): workgroup (row, g) counts the top-k keys of its columns j <
  // min(ctx, Lc) into hist + row * hist_rs bytes + g * 2048 bins (its columns are top-k chunk g)
  uint32_t* hist; long long hist_rs;
};

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
__device__ inline uint32_t fp8lo_bf16x2(uint32_t w) {
  return __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w, 1.0f, false));
}
__device__ inline uint32_t fp8hi_bf16x2(uint32_t w) {
  return __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w, 1.0f, true));
}

// Logits workgroup: the waves of one CU (one workgroup per CU, so no later-dispatched workgroup waits behind an
// older one's issue priority) share a range of 32-key tiles of one row; each wave computes all 64 heads of one tile
// per step, its first tiles tb + w + k NW (NW = LG_NWV) and later ones claimed from an LDS counter. The key codes go straight from global memory into the
// registers of the MFMA B operand: lane (k, h) of a tile loads 16-byte chunks 2 kp + h (kp = 0..3) of key k, which
// are the key's dims 32 kp + 16 h .. + 15 in the order the operand takes them, and the key's scale. A wave keeps
// LG_D tiles of loads in flight: step t computes tile t, then loads the codes of tile t + LG_D (whose block-table
// entries were loaded at step t - LG_D) and the block-table entries of tile t + 2 LG_D, so the one wait of a step
// (for the loads of step t - LG_D) leaves LG_D - 1 steps of loads outstanding. A workgroup whose range holds at
// most LG_STAGE columns keeps its logits in LDS (with a per-tile mask of the columns to write) and writes them in
// one pass once every wave is done: the logit stores interleaved with the key reads cost 20% of the read rate at
// 131072 columns per row (measured on MI355X with a probe of the same access pattern: 181 us for the reads alone,
// 226 us with a 128-byte store per tile, 201 us with the stores staged to the end).
constexpr int LG_D = 3;                    // steps of loads in flight per wave
constexpr int LG_STAGE = 32768;            // columns a workgroup stages in LDS before writing them (128 KiB fp32)

// Key layouts: LY_ROW 132-byte rows [128 codes | scale] (the rank-sharded store); LY_SHUF vLLM's paged SHUFFLE
// layout (P = 1, rpb = keys per block): key t of a block has its 16-byte chunk c at (t / 16) * 2048 + (t % 16) * 16
// + 256 c and its scale at rpb * 128 + 4 t (dotsnote/engine/arcstats_pkg/arcstats/dsa_sm89.py:63-66); LY_FLAT the
// prefill gather: key j (column j) at store + j * k_st, scale kscale[j], valid for lo[row] <= j < ctx[row], no
// block table (dsa_sm89.py:97-118).
enum { LY_ROW = 0, LY_SHUF = 1, LY_FLAT = 2 };
typedef uint32_t u32x4u __attribute__((ext_vector_type(4), aligned(4)));   // 16 bytes at a 4-byte boundary
template <bool POW2, int LY, bool F16OUT = false>
__global__ void __launch_bounds__(LG_NWV * 64) logits_kernel(LogitParams p) {
  constexpr bool SHUF = LY == LY_SHUF, FLAT = LY == LY_FLAT;
  constexpr int D = LG_D;
  __shared__ uint32_t hh[1024];                             // level-0 histogram (p.hist): 2048 16-bit counts
  __shared__ float sbuf[LG_STAGE];                          // staged logits of the range's columns
  __shared__ uint32_t smask[LG_STAGE / 32];                 // per tile: the columns to write
  __shared__ int claim;                                     // next unclaimed tile of the range
  const int row = blockIdx.x;
  const int wv = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
  const int lane = threadIdx.x & 63;
  const bool stage = 32LL * p.tpg <= LG_STAGE;              // uniform
  const int half = lane >> 5, l32 = lane & 31;
  const int ctx = p.ctx[row];
  float* orow = (float*)p.out + (long long)row * p.out_st;            // fp32 output row
  _Float16* hrow = (_Float16*)p.out + (long long)row * p.out_st;      // fp16 output row
  auto put = [&](int j, float v) {
    if constexpr (F16OUT) hrow[j] = (_Float16)v;                       // round to nearest even (+-inf kept)
    else orow[j] = v;
  };
  // tiles [tb, te) of the row; keys j with j P + rank < ctx lie in tiles below tv (computed)
  const int tb = blockIdx.y * p.tpg;
  const int te = min(tb + p.tpg, (p.Lc + 31) >> 5);
  const long long nvalid = ctx > p.rank ? ((long long)ctx - p.rank + p.P - 1) / p.P : 0;   // keys below ctx
  const int tv = p.lim == 0 ? tb : (int)min((long long)te, max((long long)tb, (nvalid + 31) >> 5));
  if (!p.noinf)                                                         // keys of the range past ctx
    for (int j = 32 * tv + (int)threadIdx.x; j < 32 * te && j < p.Lc; j += LG_NWV * 64) put(j, -__builtin_inff());
  // the top-k's histogram covers columns below min(ctx, Lc) (P == 1: all in tiles below tv, none in the fill)
  uint32_t* hrow_out = p.hist ? (uint32_t*)((uint8_t*)p.hist + (long long)row * p.hist_rs) + blockIdx.y * 2048 : nullptr;
  if (tv <= tb) {                                           // uniform over the workgroup: no barrier below
    if (hrow_out)
      for (int b = (int)threadIdx.x; b < 2048; b += LG_NWV * 64) hrow_out[b] = 0u;
    return;
  }
  if (threadIdx.x == 0) claim = tb + 2 * LG_D * LG_NWV;     // steps 0 .. 2 LG_D - 1 take tiles tb + k NW + w
  if (hrow_out)
    for (int b = (int)threadIdx.x; b < 1024; b += LG_NWV * 64) hh[b] = 0u;
  __syncthreads();
  const int nh = hrow_out ? min(ctx, p.Lc) : 0;             // columns the histogram counts
  const int* btr = FLAT ? nullptr : p.bt + (long long)p.req[row] * p.bt_st;
  const int lo = p.lo ? p.lo[row] : 0;
  // n / d, n % d: shifts when every divisor is a power of two (POW2), else 32-bit division
  auto dv = [&](uint32_t n, uint32_t d, int sh) -> uint32_t { return POW2 ? n >> sh : n / d; };
  auto md = [&](uint32_t n, uint32_t d, int sh) -> uint32_t { return POW2 ? n & (d - 1u) : n % d; };
  // positions without a block-table entry read the range's first entry (key 32 tb < nvalid: in range)
  const int* bt_dummy = FLAT ? nullptr : btr + dv((uint32_t)(32 * tb * p.P + p.rank), (uint32_t)p.bs, p.bs_sh);
  // key r of tile id: its position, and whether it is a key of the row (id < tv: tiles past tv are no tiles)
  auto key_pos = [&](int id, int r, uint32_t& pos) -> bool {
    const int j = 32 * id + r;
    const long long ps = (long long)j * p.P + p.rank;
    pos = (uint32_t)ps;
    return id < tv && j < p.Lc && ps < ctx && ps >= lo;
  };
  // the block-table entry of this lane's key of tile id (a load from the range's first entry when there is none;
  // the value is first read when the tile's codes are loaded, LG_D steps later)
  auto load_bt = [&](int id) -> int {
    if constexpr (FLAT) return 0;
    uint32_t pos;
    const bool in = key_pos(id, l32, pos);
    return *(in ? btr + dv(pos, (uint32_t)p.bs, p.bs_sh) : bt_dummy);
  };
  // the codes (chunks 2 kp + half) and scale of this lane's key of tile id; keys that are none read row 0
  auto load_codes = [&](int id, int blk, u32x4 (&c)[4], float& sc) -> bool {
    uint32_t pos;
    bool ok = key_pos(id, l32, pos);
    const uint8_t* rp;
    const float* sp;
    uint32_t cs;                                       // bytes from chunk c to chunk c + 1
    if (FLAT) {                                        // key pos itself (pos < Lc = number of keys)
      rp = p.store + (long long)(ok ? pos : 0u) * p.k_st;
      sp = p.kscale + (ok ? pos : 0u);
      cs = 16;
    } else {
      ok = ok && blk >= 0;
      const long long tt = (long long)blk * p.bs + md(pos, (uint32_t)p.bs, p.bs_sh);
      ok = ok && tt < p.lim;
      const uint32_t lrow = ok ? dv((uint32_t)tt, (uint32_t)p.P, p.p_sh) : 0u;   // p.lim > 0: row 0 exists
      const uint8_t* kblk = p.store + (long long)dv(lrow, (uint32_t)p.rpb, p.rpb_sh) * p.blk_stride;
      const uint32_t kt = md(lrow, (uint32_t)p.rpb, p.rpb_sh);
      rp = SHUF ? kblk + (kt >> 4) * 2048u + (kt & 15u) * 16u : kblk + kt * 132u;            // chunk 0
      sp = (const float*)(SHUF ? kblk + (uint32_t)p.rpb * 128u + 4u * kt : rp + 128);      // scale
      cs = SHUF ? 256u : 16u;
    }
#pragma unroll
    for (int kp = 0; kp < 4; ++kp) {
      const u32x4u v = *(const u32x4u*)(rp + cs * (uint32_t)(2 * kp + half));
      c[kp] = u32x4{v[0], v[1], v[2], v[3]};
    }
    sc = *sp;
    return ok;
  };

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

  // step t computes tile t
  auto compute = [&](int id, const u32x4 (&c)[4], float sc, bool ok) {
    bf16x8 kb[8];
#pragma unroll
    for (int kp = 0; kp < 4; ++kp) {
      const u32x4 w4 = c[kp];
      i32x4 a0, a1;
      a0[0] = (int)fp8lo_bf16x2(w4[0]); a0[1] = (int)fp8hi_bf16x2(w4[0]);
      a0[2] = (int)fp8lo_bf16x2(w4[1]); a0[3] = (int)fp8hi_bf16x2(w4[1]);
      a1[0] = (int)fp8lo_bf16x2(w4[2]); a1[1] = (int)fp8hi_bf16x2(w4[2]);
      a1[2] = (int)fp8lo_bf16x2(w4[3]); a1[3] = (int)fp8hi_bf16x2(w4[3]);
      kb[2 * kp] = __builtin_bit_cast(bf16x8, a0);
      kb[2 * kp + 1] = __builtin_bit_cast(bf16x8, a1);
    }
    f32x16 acc0 = f32x16{}, acc1 = f32x16{};
#pragma unroll
    for (int ks = 0; ks < 8; ++ks) {
      acc0 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(qf[0][ks], kb[ks], acc0, 0, 0, 0);
      acc1 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(qf[1][ks], kb[ks], acc1, 0, 0, 0);
    }
    // relu as an integer max on the bit pattern (one instruction; fmaxf would also canonicalize its operand):
    // non-negative floats keep their value, negative ones (sign bit set: negative as int) become +0
    // (elements are copied out first: __builtin_bit_cast on an ext_vector element subscript reads element 0)
    float pa = 0.f, pb = 0.f;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const float s0 = acc0[i], s1 = acc1[i];
      pa = __builtin_fmaf(wl[0][i], __builtin_bit_cast(float, max(__builtin_bit_cast(int, s0), 0)), pa);
      pb = __builtin_fmaf(wl[1][i], __builtin_bit_cast(float, max(__builtin_bit_cast(int, s1), 0)), pb);
    }
    float part = pa + pb;
    part += __shfl_xor(part, 32, 64);
    const int j = 32 * id + l32;
    const float lg = p.clamp ? fminf(part * sc, 60000.f) : part * sc;
    const float v = ok ? lg : -__builtin_inff();
    const bool counted = half == 0 && j < nh;               // a top-k column: always written
    const bool wr = half == 0 && j < p.Lc && (ok || !p.noinf || counted);
    if (stage) {
      if (half == 0) sbuf[32 * (id - tb) + l32] = v;
      const uint64_t m = __ballot(wr);
      if (lane == 0) smask[id - tb] = (uint32_t)m;
    } else if (wr) {
      put(j, v);
    }
    if (counted) {                                          // the key of the value as stored
      uint32_t key;
      if constexpr (F16OUT) key = okey16(__builtin_bit_cast(uint16_t, (_Float16)v));
      else key = okey(v);
      const uint32_t bin = key >> 21;
      atomicAdd(&hh[bin >> 1], 1u << (16 * (bin & 1u)));
    }
  };

  // tiles of steps t .. t + 2D - 1 (slot t % 2D, wave-uniform): the first 2D steps take tiles tb + k NW + w, each
  // later one is claimed from the LDS counter 2D steps ahead (when its block-table entries are loaded), so the waves
  // finish together whatever each one's issue priority and memory service (with equal static shares the youngest
  // waves of a workgroup ended up to 31 us after the oldest at 131072 columns). A wave's tiles only grow, so it is
  // done once a whole round of 2D steps holds no tile below tv.
  // loads in flight: codes of steps t .. t + D - 1 (slot t % D), block-table entries of steps t + D .. t + 2D - 1
  // (slot t % 2D). Every step issues the same loads and claim (tiles at or past tv read the row-0 key and the
  // range's first block-table entry, cache hits, and are not computed), so the compiler's wait before a step's first
  // use of its codes counts the loads of the D - 1 steps after it on every path.
  int ids[2 * D];
#pragma unroll
  for (int k = 0; k < 2 * D; ++k) ids[k] = tb + wv + k * LG_NWV;
  u32x4 cd[D][4];
  float scv[D];
  bool okv[D];
  int btv[2 * D];
#pragma unroll
  for (int k = 0; k < 2 * D; ++k) btv[k] = load_bt(ids[k]);
#pragma unroll
  for (int k = 0; k < D; ++k) okv[k] = load_codes(ids[k], btv[k], cd[k], scv[k]);
  bool live = true;
#pragma unroll 1
  while (live) {
    live = false;
#pragma unroll
    for (int s = 0; s < 2 * D; ++s) {
      int nxt = 0;
      if (lane == 0) nxt = atomicAdd(&claim, 1);            // the tile of step t + 2D (an LDS atomic)
      if (ids[s] < tv) {                                    // uniform
        live = true;
        compute(ids[s], cd[s % D], scv[s % D], okv[s % D]);
      }
      okv[s % D] = load_codes(ids[(s + D) % (2 * D)], btv[(s + D) % (2 * D)], cd[s % D], scv[s % D]);
      ids[s] = __builtin_amdgcn_readfirstlane(nxt);
      btv[s] = load_bt(ids[s]);
    }
  }
  if (stage || hrow_out) __syncthreads();   // every wave has computed (and counted) its tiles
  if (stage) {                               // 4 columns per thread: one 16-byte (fp16: 8-byte) store when all go out
    const int ncol = 32 * (tv - tb);
    const bool vec = ((uintptr_t)p.out & (F16OUT ? 7u : 15u)) == 0 && (p.out_st & 3) == 0;   // j % 4 == 0 below
    for (int i = 4 * (int)threadIdx.x; i < ncol; i += 4 * LG_NWV * 64) {
      const int j = 32 * tb + i;
      const uint32_t m4 = (smask[i >> 5] >> (i & 31)) & 15u;
      const f32x4 v4 = *(const f32x4*)&sbuf[i];
      if (vec && m4 == 15u && j + 3 < p.Lc) {
        if constexpr (F16OUT) {
          typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
          *(f16x4*)(hrow + j) = f16x4{(_Float16)v4[0], (_Float16)v4[1], (_Float16)v4[2], (_Float16)v4[3]};
        } else {
          *(f32x4*)(orow + j) = v4;
        }
      } else {
#pragma unroll
        for (int k = 0; k < 4; ++k)
          if (((m4 >> k) & 1u) && j + k < p.Lc) put(j + k, v4[k]);
      }
    }
  }
  if (hrow_out)
    for (int b = (int)threadIdx.x; b < 2048; b += LG_NWV * 64) hrow_out[b] = (hh[b >> 1] >> (16 * (b & 1))) & 0xffffu;
}

// ------------------------------------------------------------------------------------------------ top-k
constexpr int TK_NT = 1024;
constexpr int TK_KMAX = 2048;
constexpr int TK_CAP = 8192;              // candidate list capacity (workspace and LDS)
constexpr int TK_CAP1 = 4096;             // the one-workgroup path's candidate threshold

// key of logit j of a row (fp32 or fp16 elements)
template <bool F16>
__device__ inline uint32_t lkey(const void* x, long long j) {
  if constexpr (F16) return okey16(((const uint16_t*)x)[j]);
  else return okey(((const float*)x)[j]);
}
// keys of +inf and -inf
template <bool F16>
__device__ inline bool inf_key(uint32_t k) {
  if constexpr (F16) return k == 0xfc000000u || k == 0x03ff0000u;
  else return k == 0xff800000u || k == 0x007fffffu;
}
// row `row` of a logits matrix with element stride st
template <bool F16>
__device__ inline const void* lrow(const void* lg, int row, long long st) {
  return (const uint8_t*)lg + (long long)row * st * (F16 ? 2 : 4);
}

// Inclusive prefix sum over the 64 lanes of a wave on the VALU: DPP row shifts 1, 2, 4, 8 scan each 16-lane row,
// then row_bcast:15 adds row 0's total to row 1 and row 2's to row 3, and row_bcast:31 adds rows 0-1's total to rows
// 2 and 3 (gfx9 DPP controls). A lane whose DPP source is outside its row adds 0.
__device__ inline uint32_t wave_incl_scan(uint32_t x) {
  x += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, 0x111, 0xf, 0xf, false);   // row_shr:1
  x += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, 0x112, 0xf, 0xf, false);   // row_shr:2
  x += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, 0x114, 0xf, 0xf, false);   // row_shr:4
  x += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, 0x118, 0xf, 0xf, false);   // row_shr:8
  x += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, 0x142, 0xa, 0xf, false);   // row_bcast:15, rows 1, 3
  x += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, 0x143, 0xc, 0xf, false);   // row_bcast:31, rows 2, 3
  return x;
}
// Minimum / maximum over the wave (uniform result): quad permutations and row mirrors within each 16-lane row,
// then the four rows' results through readlane.
template <bool MAX>
__device__ inline uint32_t wave_minmax(uint32_t x) {
  auto op = [](uint32_t a, uint32_t b) { return MAX ? (a > b ? a : b) : (a < b ? a : b); };
  x = op(x, (uint32_t)__builtin_amdgcn_mov_dpp((int)x, 0xb1, 0xf, 0xf, false));   // quad_perm [1, 0, 3, 2]
  x = op(x, (uint32_t)__builtin_amdgcn_mov_dpp((int)x, 0x4e, 0xf, 0xf, false));   // quad_perm [2, 3, 0, 1]
  x = op(x, (uint32_t)__builtin_amdgcn_mov_dpp((int)x, 0x141, 0xf, 0xf, false));  // row_half_mirror
  x = op(x, (uint32_t)__builtin_amdgcn_mov_dpp((int)x, 0x140, 0xf, 0xf, false));  // row_mirror
  const uint32_t a = (uint32_t)__builtin_amdgcn_readlane((int)x, 0), b = (uint32_t)__builtin_amdgcn_readlane((int)x, 16);
  const uint32_t c = (uint32_t)__builtin_amdgcn_readlane((int)x, 32), d = (uint32_t)__builtin_amdgcn_readlane((int)x, 48);
  return op(op(a, b), op(c, d));
}

// block-wide exclusive scan of a per-thread count (1024 threads = 16 waves): wave scans on the VALU, the 16 wave
// totals through LDS (wsum: 16-byte aligned, 16 words); every thread sums the totals of the waves before its own
__device__ inline uint32_t block_excl_scan(uint32_t v, uint32_t* wsum, uint32_t* total) {
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const uint32_t inc = wave_incl_scan(v);
  if (lane == 63) wsum[wv] = inc;
  __syncthreads();
  uint32_t before = 0u, tot = 0u;
#pragma unroll
  for (int q = 0; q < TK_NT / 256; ++q) {
    const u32x4 s4 = ((const u32x4*)wsum)[q];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      before += 4 * q + e < wv ? s4[e] : 0u;
      tot += s4[e];
    }
  }
  *total = tot;
  __syncthreads();                                   // wsum is free for the next scan
  return before + inc - v;
}

// bitonic sort of n (power of two) uint64 in LDS, descending. Thread t handles pairs t, t + 1024, ...; for a
// stride <= 64 both elements of its pairs lie in the 128-element block of its wave, so such a stage needs no
// workgroup barrier (LDS operations of one wave complete in issue order), only a compiler fence.
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
      const int next = stride > 1 ? stride >> 1 : size;   // stride of the next stage (size << 1 >> 1)
      if (stride >= 128 || next >= 128) __syncthreads();
      else __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
    }
  }
  __syncthreads();
}

// Lane-xor exchange of a 64-bit value. Masks 1 and 2 are DPP quad permutations and 32 is v_permlane32_swap, all on
// the SIMD's own VALU; 4, 8 and 16 go through the LDS crossbar (ds_swizzle, bit mode). The sort's stages are bound by
// the LDS pipe that the CU's 16 waves share, so every exchange moved to the VALU shortens them.
template <int M>
__device__ inline unsigned long long xchg64(unsigned long long v, int perm32) {
  (void)perm32;
  const int vlo = (int)(uint32_t)v, vhi = (int)(uint32_t)(v >> 32);
  int lo, hi;
  if constexpr (M == 1 || M == 2) {
    constexpr int ctl = M == 1 ? 0xB1 : 0x4E;          // quad_perm [1, 0, 3, 2] / [2, 3, 0, 1]
    lo = __builtin_amdgcn_mov_dpp(vlo, ctl, 0xF, 0xF, false);
    hi = __builtin_amdgcn_mov_dpp(vhi, ctl, 0xF, 0xF, false);
  } else if constexpr (M == 32) {
    const auto a = __builtin_amdgcn_permlane32_swap((uint32_t)vlo, (uint32_t)vlo, false, false);
    const auto b = __builtin_amdgcn_permlane32_swap((uint32_t)vhi, (uint32_t)vhi, false, false);
    const bool up = (__lane_id() & 32) != 0;
    lo = (int)(up ? a[0] : a[1]);
    hi = (int)(up ? b[0] : b[1]);
  } else {
    lo = __builtin_amdgcn_ds_swizzle(vlo, (M << 10) | 0x1f);
    hi = __builtin_amdgcn_ds_swizzle(vhi, (M << 10) | 0x1f);
  }
  return ((unsigned long long)(uint32_t)hi << 32) | (uint32_t)lo;
}

// One compare-exchange stage of the bitonic network held in VGPRs (block size SIZE, lane-xor stride S < 64);
// thread t of wave w holds entries e0 = 128w + l and e0 + 64 (l = lane).
template <int SIZE, int S>
__device__ inline void bstage(unsigned long long& x0, unsigned long long& x1, int e0, int l, int perm32) {
  const bool d0 = (e0 & SIZE) == 0, d1 = ((e0 + 64) & SIZE) == 0;
  const unsigned long long y0 = xchg64<S>(x0, perm32), y1 = xchg64<S>(x1, perm32);
  const bool lower = (l & S) == 0;
  // the lower element of a pair keeps the max when descending, the upper one the min (and the reverse)
  x0 = ((lower == d0) == (x0 > y0)) ? x0 : y0;
  x1 = ((lower == d1) == (x1 > y1)) ? x1 : y1;
}

// The stages of a SIZE block with strides <= 64 (stride 64: the thread's own two entries, same block).
template <int SIZE>
__device__ inline void bmerge(unsigned long long& x0, unsigned long long& x1, int e0, int l, int perm32) {
  if constexpr (SIZE >= 128) {
    if ((x0 < x1) == ((e0 & SIZE) == 0)) { const unsigned long long t = x0; x0 = x1; x1 = t; }
  }
  if constexpr (SIZE >= 64) bstage<SIZE, 32>(x0, x1, e0, l, perm32);
  if constexpr (SIZE >= 32) bstage<SIZE, 16>(x0, x1, e0, l, perm32);
  if constexpr (SIZE >= 16) bstage<SIZE, 8>(x0, x1, e0, l, perm32);
  if constexpr (SIZE >= 8) bstage<SIZE, 4>(x0, x1, e0, l, perm32);
  if constexpr (SIZE >= 4) bstage<SIZE, 2>(x0, x1, e0, l, perm32);
  bstage<SIZE, 1>(x0, x1, e0, l, perm32);
}

// The stages of a SIZE block with strides >= 128, through LDS (one pair per thread, a barrier per stage).
template <int SIZE>
__device__ inline void bmerge_lds(unsigned long long* a, unsigned long long& x0, unsigned long long& x1, int e0) {
  const int t = threadIdx.x;
  a[e0] = x0;
  a[e0 + 64] = x1;
  __syncthreads();
#pragma unroll
  for (int stride = SIZE >> 1; stride >= 128; stride >>= 1) {
    const int lo = 2 * t - (t & (stride - 1)), hi = lo + stride;
    const bool desc = (lo & SIZE) == 0;
    const unsigned long long x = a[lo], y = a[hi];
    if ((x < y) == desc) { a[lo] = y; a[hi] = x; }
    __syncthreads();
  }
  x0 = a[e0];
  x1 = a[e0 + 64];
}

// Bitonic sort of a[0, 2048) descending with the data in VGPRs: 56 of the 66 stages are in-thread or lane-xor
// exchanges (ds_swizzle), the 10 with strides >= 128 go through LDS.
__device__ inline void sort2048_desc(unsigned long long* a) {
  const int t = threadIdx.x, l = t & 63;
  const int e0 = 128 * (t >> 6) + l;
  const int perm32 = (l ^ 32) << 2;
  unsigned long long x0 = a[e0], x1 = a[e0 + 64];
  bmerge<2>(x0, x1, e0, l, perm32);
  bmerge<4>(x0, x1, e0, l, perm32);
  bmerge<8>(x0, x1, e0, l, perm32);
  bmerge<16>(x0, x1, e0, l, perm32);
  bmerge<32>(x0, x1, e0, l, perm32);
  bmerge<64>(x0, x1, e0, l, perm32);
  bmerge<128>(x0, x1, e0, l, perm32);
  bmerge_lds<256>(a, x0, x1, e0);
  bmerge<256>(x0, x1, e0, l, perm32);
  bmerge_lds<512>(a, x0, x1, e0);
  bmerge<512>(x0, x1, e0, l, perm32);
  bmerge_lds<1024>(a, x0, x1, e0);
  bmerge<1024>(x0, x1, e0, l, perm32);
  bmerge_lds<2048>(a, x0, x1, e0);
  bmerge<2048>(x0, x1, e0, l, perm32);
  __syncthreads();                                   // every thread has read a: write the sorted data back
  a[e0] = x0;
  a[e0 + 64] = x1;
  __syncthreads();
}

// Sorts a[0, n) descending (entries nonzero); pads with zeros to the sorting network's size.
__device__ inline void tk_sort_desc(unsigned long long* a, int n) {
  int np2 = 1;
  while (np2 < n) np2 <<= 1;
  if (np2 > 256 && np2 <= 2048) np2 = 2048;
  for (int i = n + (int)threadIdx.x; i < np2; i += TK_NT) a[i] = 0ull;
  __syncthreads();
  if (np2 == 2048) sort2048_desc(a);
  else if (np2 > 1) bitonic_desc(a, np2);
}

template <bool F16>
struct RowSrc {     // a logits row (fp32 or fp16): candidate j = column j
  const void* x; int n;
  __device__ uint32_t key(int j) const { return lkey<F16>(x, j); }
  __device__ float val(int j) const {
    if constexpr (F16) return (float)((const _Float16*)x)[j];
    else return ((const float*)x)[j];
  }
  __device__ int id(int j) const { return j; }
  __device__ static bool inf(uint32_t k) { return inf_key<F16>(k); }
};
struct MergeSrc {   // all-gathered payloads [P][nrows][2 * kl] = [values | positions]: candidate c = (c / kl, c % kl)
  const float* allp; long long nrows; int row, kl, n;
  __device__ const float* seg(int c, int& i) const {
    const int r = c / kl;
    i = c - r * kl;
    return allp + ((long long)r * nrows + row) * 2 * kl;
  }
  __device__ float val(int c) const { int i; const float* b = seg(c, i); return b[i]; }
  __device__ uint32_t key(int c) const { return okey(val(c)); }
  __device__ int id(int c) const { int i; const float* b = seg(c, i); return (int)f2u(b[kl + i]); }
  __device__ static bool inf(uint32_t k) { return inf_key<false>(k); }
};

// Four copies of the 2048-bin histogram (lane & 3 picks one) split same-bin atomics of a wave four ways; a copy
// stride of 2049 words keeps the copies of a bin in different banks.
constexpr int TK_HCOPY = 4;
constexpr int TK_HSTR = 2049;

struct TopkLds {
  uint32_t hist[TK_HCOPY * TK_HSTR];
  unsigned long long sel[TK_KMAX];
  unsigned long long cand[TK_CAP];
  __attribute__((aligned(16))) uint32_t wsum[17];
  uint32_t sh[8];
};

__device__ inline unsigned long long tk_pack(uint32_t key, int j) {
  return ((unsigned long long)key << 32) | (uint32_t)(~(uint32_t)j);
}

__device__ inline void tk_hist_add(TopkLds& L, uint32_t bin) {
  atomicAdd(&L.hist[(threadIdx.x & (TK_HCOPY - 1)) * TK_HSTR + bin], 1u);
}

// Radix level bookkeeping: digit d = (key >> shift) & dm of the keys under (prefix, mask).
__device__ inline int tk_shift(int level) { return level == 0 ? 21 : (level == 1 ? 10 : 0); }
__device__ inline uint32_t tk_dmask(int level) { return level == 2 ? 0x3ffu : 0x7ffu; }

// From the level's histogram: the boundary bin b holding the need-th largest key, the count above it and in it.
__device__ inline void tk_bin(TopkLds& L, uint32_t need, uint32_t& b, uint32_t& above, uint32_t& binc) {
  const int tid = threadIdx.x;
  const int b0 = 2047 - 2 * tid, b1 = b0 - 1;   // thread t owns bins 2047 - 2t, 2046 - 2t (descending)
  uint32_t h0 = 0, h1 = 0;
#pragma unroll
  for (int c = 0; c < TK_HCOPY; ++c) { h0 += L.hist[c * TK_HSTR + b0]; h1 += L.hist[c * TK_HSTR + b1]; }
  uint32_t tot;
  const uint32_t before = block_excl_scan(h0 + h1, L.wsum, &tot);
  if (before < need && before + h0 >= need) { L.sh[1] = (uint32_t)b0; L.sh[2] = before; L.sh[3] = h0; }
  if (before + h0 < need && before + h0 + h1 >= need) { L.sh[1] = (uint32_t)b1; L.sh[2] = before + h0; L.sh[3] = h1; }
  __syncthreads();
  b = L.sh[1]; above = L.sh[2]; binc = L.sh[3];
}

__device__ inline void tk_clear_hist(TopkLds& L) {
  for (int i = threadIdx.x; i < TK_HCOPY * TK_HSTR; i += TK_NT) L.hist[i] = 0;
  __syncthreads();
}

// Block-wide placement of per-thread selections: each thread passes how many entries it appends to sel and to cand;
// returns its first slot in each (after the bases *sb, *cb, which advance by the block totals on every thread).
__device__ inline void tk_slots(uint32_t ns, uint32_t nc, TopkLds& L, uint32_t& sb, uint32_t& cb, uint32_t& so,
                                uint32_t& co) {
  uint32_t tot;
  const uint32_t off = block_excl_scan(ns | (nc << 16), L.wsum, &tot);   // both totals < 65536
  so = sb + (off & 0xffffu);
  co = cb + (off >> 16);
  sb += tot & 0xffffu;
  cb += tot >> 16;
}

constexpr int TK_KPT = 32;                 // keys per thread per chunk (held in VGPRs)
constexpr int TK_CH = TK_KPT * TK_NT;      // 32768 columns per chunk
constexpr int TK_EPT = TK_CAP / TK_NT;     // boundary-bin candidates per thread at the full capacity

template <class Src>
__device__ inline void tk_load(const Src& src, int base, uint32_t (&k)[TK_KPT]) {
#pragma unroll
  for (int i = 0; i < TK_KPT; ++i) {
    const int j = base + i * TK_NT + (int)threadIdx.x;
    k[i] = j < src.n ? src.key(j) : 0u;
  }
}

// Finishes a selection from the boundary-bin candidates L.cand[0, nc) (all under (prefix, mask) of level lvl - 1):
// radix levels lvl..2 on the candidates held in registers; equal final keys go to the lowest columns. sb = entries
// already in L.sel.
template <int EPT = TK_EPT>                       // candidates per thread: nc <= EPT * TK_NT
__device__ __forceinline__ void tk_resolve_cands(TopkLds& L, int nc, int lvl, uint32_t prefix, uint32_t mask,
                                                 uint32_t need, uint32_t sb, int ncols) {
  const int tid = threadIdx.x;
  unsigned long long e[EPT];
  uint32_t vm = 0;                                   // bit i: e[i] is a candidate
  int t = tid;                                       // opaque copy: keeps the slot indices from being hoisted
  asm volatile("" : "+v"(t));
#pragma unroll
  for (int i = 0; i < EPT; ++i) {              // consecutive candidates: the winners appended below keep their
    const int c = EPT * t + i;                  // order in L.cand (column order for the workspace path)
    vm |= (uint32_t)(c < nc) << i;
    e[i] = c < nc ? L.cand[c] : 0ull;
  }
  for (int level = lvl; level < 3; ++level) {
    const int shift = tk_shift(level);
    const uint32_t dm = tk_dmask(level);
    tk_clear_hist(L);
#pragma unroll
    for (int i = 0; i < EPT; ++i) {
      const uint32_t k = (uint32_t)(e[i] >> 32);
      if (((vm >> i) & 1u) && (k & mask) == prefix) tk_hist_add(L, (k >> shift) & dm);
    }
    __syncthreads();
    uint32_t b, above, binc;
    tk_bin(L, need, b, above, binc);
    const bool whole = above + binc == need;
    uint32_t selm = 0;
#pragma unroll
    for (int i = 0; i < EPT; ++i) {
      const uint32_t k = (uint32_t)(e[i] >> 32);
      const uint32_t d = (k >> shift) & dm;
      const bool in = ((vm >> i) & 1u) && (k & mask) == prefix;
      selm |= (uint32_t)(in && (d > b || (whole && d == b))) << i;
    }
    uint32_t cb = 0, so, co;
    tk_slots(__popc(selm), 0u, L, sb, cb, so, co);
#pragma unroll
    for (int i = 0; i < EPT; ++i)
      if ((selm >> i) & 1u) L.sel[so++] = e[i];
    if (whole) { __syncthreads(); return; }
    prefix |= b << shift;
    mask |= dm << shift;
    need -= above;
    if (level == 2) {
      // binc candidates carry the final key; the need lowest columns win
      uint32_t eqm = 0;
#pragma unroll
      for (int i = 0; i < EPT; ++i)
        eqm |= (uint32_t)(((vm >> i) & 1u) && (uint32_t)(e[i] >> 32) == prefix) << i;
      constexpr int BM_WPT = 8;                    // bitmap words per thread: TK_NT * 8 words in the histogram space
      static_assert(TK_NT * BM_WPT <= TK_HCOPY * TK_HSTR, "bitmap fits the histogram space");
      if (ncols <= 32 * TK_NT * BM_WPT) {
        // a bitmap of the tied columns in the histogram space (free after the last level), then each column's rank
        // among them from prefix sums of per-word bit counts: the need lowest are taken, no sort (the final output
        // sort orders every winner anyway)
        const int words = (ncols + 31) >> 5;
        __syncthreads();
        for (int w = tid; w < words; w += TK_NT) L.hist[w] = 0u;
        __syncthreads();
#pragma unroll
        for (int i = 0; i < EPT; ++i)
          if ((eqm >> i) & 1u) {
            const uint32_t j = ~(uint32_t)e[i];
            atomicOr(&L.hist[j >> 5], 1u << (j & 31u));
          }
        __syncthreads();
        const int w0 = tid * BM_WPT;
        uint32_t cnt = 0;
#pragma unroll
        for (int k = 0; k < BM_WPT; ++k)
          if (w0 + k < words) cnt += (uint32_t)__popc(L.hist[w0 + k]);
        uint32_t tot;
        uint32_t r = block_excl_scan(cnt, L.wsum, &tot);   // ranks of this thread's first tied column
#pragma unroll
        for (int k = 0; k < BM_WPT; ++k) {
          uint32_t bits = w0 + k < words ? L.hist[w0 + k] : 0u;
          while (bits && r < need) {
            const uint32_t j = 32u * (uint32_t)(w0 + k) + (uint32_t)(__ffs(bits) - 1);
            bits &= bits - 1u;
            L.sel[sb + r] = (((unsigned long long)prefix) << 32) | (uint32_t)~j;
            ++r;
          }
        }
        __syncthreads();
        return;
      }
      // wider rows: sort the tied candidates by column ascending
      __syncthreads();                             // every thread has read its candidates: L.cand is free
      uint32_t cb2 = 0, sb2 = 0;
      tk_slots(0u, __popc(eqm), L, sb2, cb2, so, co);
#pragma unroll
      for (int i = 0; i < EPT; ++i)
        if ((eqm >> i) & 1u) L.cand[co++] = (unsigned long long)(uint32_t)e[i] << 32;   // ~j high: desc = j asc
      __syncthreads();
      tk_sort_desc(L.cand, (int)binc);
      for (uint32_t i = tid; i < need; i += TK_NT) L.sel[sb + i] = (((unsigned long long)prefix) << 32) | (L.cand[i] >> 32);
      __syncthreads();
      return;
    }
  }
}

// Selects the K largest candidates (key desc, j asc) of src into L.sel (unordered); returns their number min(n, K).
// The row's keys sit in VGPRs (32 per thread; longer rows are re-read per 32768-column chunk with all loads of a
// chunk in flight). Each radix level builds an LDS histogram; the keys above the boundary bin are written to slots
// from one block scan of per-thread counts; a boundary bin of at most TK_CAP1 keys is finished on the candidates alone.
template <class Src>
__device__ __forceinline__ int tk_select(const Src& src, int K, TopkLds& L) {
  const int tid = threadIdx.x, n = src.n;
  if (n <= K) {
    for (int j = tid; j < n; j += TK_NT) L.sel[j] = tk_pack(src.key(j), j);
    __syncthreads();
    return n;
  }
  const int nch = (n + TK_CH - 1) / TK_CH;
  uint32_t key[TK_KPT];
  if (nch == 1) tk_load(src, 0, key);
  uint32_t prefix = 0, mask = 0, need = (uint32_t)K, sb = 0;
  for (int level = 0; level < 3; ++level) {
    const int shift = tk_shift(level);
    const uint32_t dm = tk_dmask(level);
    // the column of key[i] is recomputed per level from an opaque copy of tid: hoisting the 32 columns (and the
    // packed entries built from them) out of the level loop would spill them
    int t = tid;
    asm volatile("" : "+v"(t));
    tk_clear_hist(L);
    for (int c = 0; c < nch; ++c) {
      if (nch > 1) tk_load(src, c * TK_CH, key);
#pragma unroll
      for (int i = 0; i < TK_KPT; ++i) {
        const int j = c * TK_CH + i * TK_NT + t;
        if (j < n && (key[i] & mask) == prefix) tk_hist_add(L, (key[i] >> shift) & dm);
      }
    }
    __syncthreads();
    uint32_t b, above, binc;
    tk_bin(L, need, b, above, binc);
    const bool whole = above + binc == need;
    const bool fits = !whole && level < 2 && binc <= (uint32_t)TK_CAP1;
    uint32_t cb = 0;
    for (int c = 0; c < nch; ++c) {
      if (nch > 1) tk_load(src, c * TK_CH, key);
      uint32_t selm = 0, candm = 0;
#pragma unroll
      for (int i = 0; i < TK_KPT; ++i) {
        const int j = c * TK_CH + i * TK_NT + t;
        const uint32_t d = (key[i] >> shift) & dm;
        const bool in = j < n && (key[i] & mask) == prefix;
        selm |= (uint32_t)(in && (d > b || (whole && d == b))) << i;
        candm |= (uint32_t)(fits && in && d == b) << i;
      }
      uint32_t so, co;
      tk_slots(__popc(selm), __popc(candm), L, sb, cb, so, co);
#pragma unroll
      for (int i = 0; i < TK_KPT; ++i) {
        const int j = c * TK_CH + i * TK_NT + t;
        if ((selm >> i) & 1u) L.sel[so++] = tk_pack(key[i], j);
        if ((candm >> i) & 1u) L.cand[co++] = tk_pack(key[i], j);
      }
    }
    __syncthreads();
    if (whole) return K;
    if (fits) {
      tk_resolve_cands<TK_CAP1 / TK_NT>(L, (int)binc, level + 1, prefix | (b << shift), mask | (dm << shift), need - above, sb, n);
      return K;
    }
    prefix |= b << shift;
    mask |= dm << shift;
    need -= above;
  }
  // the boundary key is fully known (prefix); the need lowest columns holding it win, in column order
  uint32_t got = 0;
  for (int c = 0; c < nch && got < need; ++c) {
    if (nch > 1) tk_load(src, c * TK_CH, key);
#pragma unroll
    for (int i = 0; i < TK_KPT; ++i) {
      if (got < need) {                          // uniform: got is a block-wide total
        const int j = c * TK_CH + i * TK_NT + tid;
        const bool eq = j < n && key[i] == prefix;
        uint32_t tot;
        const uint32_t r = block_excl_scan(eq ? 1u : 0u, L.wsum, &tot);
        if (eq && got + r < need) L.sel[sb + got + r] = tk_pack(prefix, j);
        got += tot;
      }
    }
  }
  __syncthreads();
  return K;
}

// Sorts the nsel selected entries by (key desc, j asc) and writes src.id of the first kout slots to o
// (-1 where the value is +-inf and for slots >= nsel).
template <class Src>
__device__ __forceinline__ void tk_emit_sorted(const Src& src, int nsel, int kout, int* o, TopkLds& L) {
  const int tid = threadIdx.x;
  tk_sort_desc(L.sel, nsel);
  for (int s = tid; s < kout; s += TK_NT) {
    int r = -1;
    if (s < nsel) {
      const unsigned long long e = L.sel[s];
      const uint32_t key = (uint32_t)(e >> 32);
      const int j = (int)(~(uint32_t)e);
      if (!Src::inf(key)) r = src.id(j);                  // +-inf: no position
    }
    o[s] = r;
  }
}

// Stable LSD radix sort of L.sel[0, n) (n <= 2048) by key (the high word) descending, then the emit of
// tk_emit_sorted. Entries with equal keys keep their order in L.sel, so lists appended in column order come out
// (key desc, column asc) with no sort on the columns. Keys are offset by the smallest key, and only the bytes that
// the offsets span are sorted (fp16 keys: their low half is zero). One pass: wave-local stable ranks from 16 ballots
// (entries 2t, 2t + 1 of thread t, waves in order), per-wave digit counts, one scan over (digit, wave), a scatter.
// LDS: L.cand as the scatter buffer, L.hist for the counts and offsets.
template <class Src, bool F16>
__device__ __forceinline__ void tk_emit_radix(const Src& src, int n, int kout, int* o, TopkLds& L) {
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  unsigned long long* tmp = L.cand;
  uint32_t* whist = L.hist;                      // [digit][wave] counts of the pass
  uint32_t* woff = L.hist + 4096;                // [digit][wave] first slot of the wave's entries of the digit
  uint32_t* red = (uint32_t*)(L.cand + TK_KMAX); // 16 waves x (min, max)
  static_assert(2 * 4096 <= TK_HCOPY * TK_HSTR && TK_CAP >= TK_KMAX + 16, "radix sort LDS");
  for (int i = tid; i < 4096; i += TK_NT) whist[i] = 0u;
  const bool v0 = 2 * tid < n, v1 = 2 * tid + 1 < n;   // entries past n: zero, sorted last
  unsigned long long x0 = v0 ? L.sel[2 * tid] : 0ull, x1 = v1 ? L.sel[2 * tid + 1] : 0ull;
  uint32_t kmn = 0xffffffffu, kmx = 0u;
  if (v0) { kmn = (uint32_t)(x0 >> 32); kmx = kmn; }
  if (v1) { kmn = min(kmn, (uint32_t)(x1 >> 32)); kmx = max(kmx, (uint32_t)(x1 >> 32)); }
  kmn = wave_minmax<false>(kmn);
  kmx = wave_minmax<true>(kmx);
  if (lane == 0) { red[2 * wv] = kmn; red[2 * wv + 1] = kmx; }
  __syncthreads();
#pragma unroll
  for (int v = 0; v < TK_NT / 64; ++v) { kmn = min(kmn, red[2 * v]); kmx = max(kmx, red[2 * v + 1]); }
  const uint32_t range = kmx > kmn ? kmx - kmn : 0u;
  const int first = F16 ? 2 : 0;                 // lowest byte that can differ
  const int last = range ? (31 - __builtin_clz(range)) >> 3 : -1;
  const unsigned long long below = (1ull << lane) - 1ull;
  for (int byte = first; byte <= last; ++byte) {   // uniform
    const int sh = 8 * byte;
    // padding entries (key 0: every real key is at least -inf's 0x007fffff) take digit 255 in every pass
    const uint32_t k0 = (uint32_t)(x0 >> 32), k1 = (uint32_t)(x1 >> 32);
    const uint32_t d0 = k0 ? 255u - ((k0 - kmn) >> sh & 255u) : 255u;
    const uint32_t d1 = k1 ? 255u - ((k1 - kmn) >> sh & 255u) : 255u;
    // lanes whose entry 0 / entry 1 has this lane's digit d0 (ma / mb) or d1 (mc / md)
    unsigned long long ma = ~0ull, mb = ~0ull, mc = ~0ull, md = ~0ull;
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const unsigned long long b0 = __ballot((d0 >> k) & 1u), b1 = __ballot((d1 >> k) & 1u);
      const unsigned long long s0 = (unsigned long long)(long long)-(int)((d0 >> k) & 1u);
      const unsigned long long s1 = (unsigned long long)(long long)-(int)((d1 >> k) & 1u);
      ma &= ~(b0 ^ s0); mb &= ~(b1 ^ s0); mc &= ~(b0 ^ s1); md &= ~(b1 ^ s1);
    }
    // stable rank among the wave's entries of the same digit (order: lane, then entry)
    const uint32_t r0 = (uint32_t)(__popcll(ma & below) + __popcll(mb & below));
    const uint32_t r1 = (uint32_t)(__popcll(mc & below) + __popcll(md & below)) + (d0 == d1 ? 1u : 0u);
    if (r0 == 0u) whist[d0 * 16 + wv] = (uint32_t)(__popcll(ma) + __popcll(mb));
    if (r1 == 0u) whist[d1 * 16 + wv] = (uint32_t)(__popcll(mc) + __popcll(md));
    __syncthreads();
    uint32_t c[16], tot = 0u, incl = 0u;
    if (tid < 256) {                              // digit tid: offsets over the waves, then over the digits
      u32x4* hp = (u32x4*)(whist + tid * 16);
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const u32x4 v = hp[q];
        hp[q] = u32x4{0u, 0u, 0u, 0u};           // cleared for the next pass
#pragma unroll
        for (int e = 0; e < 4; ++e) { c[4 * q + e] = tot; tot += v[e]; }
      }
      incl = wave_incl_scan(tot);
      if (lane == 63) L.wsum[wv] = incl;
    }
    __syncthreads();
    if (tid < 256) {
      uint32_t bse = incl - tot;
      for (int v = 0; v < wv; ++v) bse += L.wsum[v];
      u32x4* op = (u32x4*)(woff + tid * 16);
#pragma unroll
      for (int q = 0; q < 4; ++q) op[q] = u32x4{bse + c[4 * q], bse + c[4 * q + 1], bse + c[4 * q + 2], bse + c[4 * q + 3]};
    }
    __syncthreads();
    tmp[woff[d0 * 16 + wv] + r0] = x0;
    tmp[woff[d1 * 16 + wv] + r1] = x1;
    __syncthreads();
    x0 = tmp[2 * tid];
    x1 = tmp[2 * tid + 1];
  }
  // entries 2t, 2t + 1 of the sorted order are in this thread's registers
#pragma unroll
  for (int e = 0; e < 2; ++e) {
    const int slot = 2 * tid + e;
    if (slot < kout) {
      int r = -1;
      const unsigned long long x = e ? x1 : x0;
      if (slot < n) {
        const uint32_t key = (uint32_t)(x >> 32);
        const int j = (int)(~(uint32_t)x);
        if (!Src::inf(key)) r = src.id(j);
      }
      o[slot] = r;
    }
  }
}

struct TopkParams {
  const void* lg; long long lg_st;                // fp32 or fp16 (the kernel's F16), stride in elements
  const int* ctx; int rows, Lc, K;
  int* out; long long out_st;
};

template <bool F16>
__global__ void __launch_bounds__(TK_NT) topk_kernel(TopkParams p) {
  __shared__ TopkLds L;
  const int row = blockIdx.x;
  int n = p.ctx[row];
  n = n < 0 ? 0 : (n > p.Lc ? p.Lc : n);
  const RowSrc<F16> src{lrow<F16>(p.lg, row, p.lg_st), n};
  const int nsel = tk_select(src, p.K, L);
  tk_emit_sorted(src, nsel, p.K, p.out + (long long)row * p.out_st, L);
}

// ---- top-k over several workgroups per row (workspace variant) -------------------------------------------
// Two radix levels run across G workgroups per row (chunks of at most CL columns):
//   hist:    the histogram of the level-0 11-bit digit over each chunk's keys;
//   collect: every workgroup sums the G histograms of the level and finds the boundary bin b of the row's
//            remaining need; it writes its chunk's keys above b (and in b when that completes the need) to the row's
//            winner list, and the keys in b to the candidate list when the bin holds at most p.cap keys. A chunk's
//            entries start at the offset the histograms of the chunks before it give; inside the chunk each wave
//            takes its slots from a block scan per pass over 8 consecutive columns per thread, so every list is
//            in column order (the finishing pass's stable radix sort of fp16 keys relies on it). Otherwise the
//            next level narrows the prefix to b, and this pass also builds its chunk's histogram of that level
//            (into the other half of the histogram buffer, which no workgroup of the row is reading) and, when the
//            workspace has the overflow area, writes its chunk's keys in b there (at the offset the level-0
//            histograms give), so that the next level's collect pass reads those keys instead of the row.
// A finishing pass (one workgroup per row) resolves the candidates' remaining levels, sorts the K winners and
// writes the positions. Rows with n <= K, and rows whose bin is still too large after two levels (heavy ties), run
// the one-workgroup selection there. Per-row state lives in the workspace, one header per level (the collect pass
// of level L reads header L and its first workgroup writes header L + 1).
enum : int { TKW_SELECT = 0, TKW_WHOLE = 1, TKW_CANDS = 2, TKW_FALLBACK = 3 };
struct TkwHdr { int state, prefix, mask, need, sb, binc, lvl, ovf; };   // 32 bytes; ovf: next level reads the overflow list

struct TopkWs {
  int G, CL;                                      // chunks per row, columns per chunk (multiple of 1024)
  long long row_bytes;                            // workspace bytes per row
  __host__ __device__ TkwHdr* hdr(uint8_t* ws, int row) const { return (TkwHdr*)(ws + row * row_bytes); }
  __host__ __device__ unsigned long long* sel(uint8_t* ws, int row) const {
    return (unsigned long long*)(ws + row * row_bytes + 3 * sizeof(TkwHdr));
  }
  __host__ __device__ unsigned long long* cand(uint8_t* ws, int row) const { return sel(ws, row) + TK_KMAX; }
  __host__ __device__ uint32_t* hist(uint8_t* ws, int row) const { return (uint32_t*)(cand(ws, row) + TK_CAP); }
};

__host__ inline TopkWs topk_ws_layout(int Lc) {
  TopkWs w;
  // chunks of 8192 columns, at most 4 per row (every collect workgroup reads all G histograms of its row; with
  // 8 chunks at 131072 columns the passes took 69.6 us against 58.8 with 4, B = 64)
  int G = (Lc + 8191) / 8192;
  if (G > 4) G = 4;
  if (G < 1) G = 1;
  int CL = (Lc + G - 1) / G;
  CL = (CL + 1023) / 1024 * 1024;
  w.G = G; w.CL = CL;
  w.row_bytes = 3 * (long long)sizeof(TkwHdr) + (long long)(TK_KMAX + TK_CAP) * 8 + 2LL * G * 2048 * 4 + 16;
  w.row_bytes = (w.row_bytes + 15) / 16 * 16;
  return w;
}

struct TopkWsParams {
  const void* lg; long long lg_st;                // fp32 or fp16 (the kernels' F16), stride in elements
  const int* ctx; int rows, Lc, K;
  int* out; long long out_st;
  uint8_t* ws; TopkWs w;
  unsigned long long* ovf;                        // optional overflow lists, G * CL entries per row (or null)
  int cap;                                        // boundary bins of at most cap keys go to the finishing pass
  int level;
};

__device__ inline int tkw_n(const TopkWsParams& p, int row) {
  const int n = p.ctx[row];
  return n < 0 ? 0 : (n > p.Lc ? p.Lc : n);
}

// the row's state entering level p.level (level 0: select everything, need K)
__device__ inline TkwHdr tkw_state(const TopkWsParams& p, int row) {
  if (p.level == 0) return TkwHdr{TKW_SELECT, 0, 0, p.K, 0, 0, 0, 0};
  return p.w.hdr(p.ws, row)[p.level];
}

template <bool F16>
__global__ void __launch_bounds__(TK_NT) topk_hist_kernel(TopkWsParams p) {
  __shared__ uint32_t hist[TK_HCOPY * TK_HSTR];
  const int row = blockIdx.x, g = blockIdx.y, tid = threadIdx.x;
  const int n = tkw_n(p, row);
  if (n <= p.K) return;
  const TkwHdr st = tkw_state(p, row);
  if (st.state != TKW_SELECT) return;
  const int shift = tk_shift(p.level);
  const uint32_t prefix = (uint32_t)st.prefix, mask = (uint32_t)st.mask;
  for (int i = tid; i < TK_HCOPY * TK_HSTR; i += TK_NT) hist[i] = 0;
  __syncthreads();
  const void* x = lrow<F16>(p.lg, row, p.lg_st);
  const int c0 = g * p.w.CL, c1 = min(c0 + p.w.CL, n);
  for (int base = c0; base < c1; base += 8 * TK_NT) {
    uint32_t k[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int j = base + i * TK_NT + tid;
      k[i] = j < c1 ? lkey<F16>(x, j) : 0u;
    }
#pragma unroll
    for (int i = 0; i < 8; ++i)
      if (base + i * TK_NT + tid < c1 && (k[i] & mask) == prefix)
        atomicAdd(&hist[(tid & (TK_HCOPY - 1)) * TK_HSTR + ((k[i] >> shift) & 0x7ffu)], 1u);
  }
  __syncthreads();
  uint32_t* out = p.w.hist(p.ws, row) + (long long)g * 2048;
  for (int b = tid; b < 2048; b += TK_NT) {
    uint32_t h = 0;
#pragma unroll
    for (int c = 0; c < TK_HCOPY; ++c) h += hist[c * TK_HSTR + b];
    out[b] = h;
  }
}

template <bool F16>
__global__ void __launch_bounds__(TK_NT) topk_collect_kernel(TopkWsParams p) {
  __shared__ __attribute__((aligned(16))) uint32_t wsum[17];
  __shared__ uint32_t sh[8];
  __shared__ uint32_t nh[TK_HCOPY * TK_HSTR];       // the next level's histogram of this chunk (when narrowing)
  const int row = blockIdx.x, g = blockIdx.y, tid = threadIdx.x;
  const TkwHdr st = tkw_state(p, row);              // read beside the row length: one round trip for both
  const int n = tkw_n(p, row);
  if (n <= p.K) return;
  TkwHdr* next = p.w.hdr(p.ws, row) + p.level + 1;
  if (st.state != TKW_SELECT) {                     // settled at an earlier level: carry the state forward
    if (g == 0 && tid == 0) *next = st;
    return;
  }
  const int shift = tk_shift(p.level);
  const uint32_t prefix = (uint32_t)st.prefix, mask = (uint32_t)st.mask, need = (uint32_t)st.need;
  // thread t owns bins 2047 - 2t, 2046 - 2t: totals over the G chunks and over the chunks before g
  const int b0 = 2047 - 2 * tid, b1 = b0 - 1;
  const uint32_t* hs = p.w.hist(p.ws, row) + (long long)(p.level & 1) * p.w.G * 2048;
  uint32_t t0 = 0, t1 = 0, q0 = 0, q1 = 0;
  for (int c = 0; c < p.w.G; ++c) {
    const uint32_t h0 = hs[(long long)c * 2048 + b0], h1 = hs[(long long)c * 2048 + b1];
    t0 += h0; t1 += h1;
    if (c < g) { q0 += h0; q1 += h1; }
  }
  // defaults: with histograms that do not add up to the row (a workspace that was never filled for these logits) no
  // thread finds the boundary; the lists below are bounds-checked either way, so such a call writes only its own lists
  if (tid == 0) { sh[1] = 0u; sh[2] = 0u; sh[3] = 0u; sh[4] = 0u; }
  uint32_t tot;
  const uint32_t before = block_excl_scan(t0 + t1, wsum, &tot);
  if (before < need && before + t0 >= need) { sh[1] = (uint32_t)b0; sh[2] = before; sh[3] = t0; }
  if (before + t0 < need && before + t0 + t1 >= need) { sh[1] = (uint32_t)b1; sh[2] = before + t0; sh[3] = t1; }
  __syncthreads();
  const uint32_t b = sh[1], above = sh[2], binc = sh[3];
  const bool whole = above + binc == need;
  const bool fits = !whole && binc <= (uint32_t)p.cap;
  // this chunk's offsets: winners of the chunks before g (bins above b, and b itself when whole); candidates in b
  const uint32_t mine = ((uint32_t)b0 > b || (whole && (uint32_t)b0 == b) ? q0 : 0u) +
                        ((uint32_t)b1 > b || (whole && (uint32_t)b1 == b) ? q1 : 0u);
  uint32_t sum;
  (void)block_excl_scan(mine, wsum, &sum);
  if ((uint32_t)b0 == b) sh[4] = q0;
  if ((uint32_t)b1 == b) sh[4] = q1;
  __syncthreads();
  const uint32_t sb = (uint32_t)st.sb + sum, cb = sh[4];   // this chunk's first winner / candidate slot
  const bool narrow = !whole && !fits && p.level + 1 < 2;   // uniform per row: the next level runs on bin b
  const int nshift = tk_shift(p.level + 1);
  // level 0 narrowing with an overflow area: the chunk's keys in b go to the row's overflow list (at cb, like the
  // candidates), where level 1 reads them
  const bool to_ovf = narrow && p.ovf != nullptr;
  unsigned long long* ovf_row = p.ovf ? p.ovf + (long long)row * p.w.G * p.w.CL : nullptr;
  if (narrow) {
    for (int i = tid; i < TK_HCOPY * TK_HSTR; i += TK_NT) nh[i] = 0;
    __syncthreads();
  }
  if (g == 0 && tid == 0) {
    TkwHdr h = st;
    h.prefix = (int)(prefix | (b << shift));
    h.mask = (int)(mask | (0x7ffu << shift));
    h.need = (int)(need - above);
    h.sb = st.sb + (int)above;
    h.binc = (int)binc;
    h.lvl = p.level + 1;
    h.ovf = 0;
    if (whole) { h.state = TKW_WHOLE; h.sb = st.sb + (int)need; }
    else if (fits) h.state = TKW_CANDS;
    else { h.state = p.level + 1 < 2 ? TKW_SELECT : TKW_FALLBACK; h.ovf = to_ovf ? 1 : 0; }
    *next = h;
  }
  unsigned long long* sel = p.w.sel(p.ws, row);
  unsigned long long* cand = to_ovf ? ovf_row : p.w.cand(p.ws, row);
  const uint32_t clim = to_ovf ? (uint32_t)(p.w.G * p.w.CL) : (uint32_t)TK_CAP;   // entries of the candidate list
  const void* x = lrow<F16>(p.lg, row, p.lg_st);
  // the keys this workgroup visits: logits columns c0 .. c1, or (a level narrowed with an overflow list) entries
  // c0 .. c1 of the overflow list: the previous level's bin keys of chunk g, at the offset its histograms give
  int c0 = g * p.w.CL, c1 = min(c0 + p.w.CL, n);
  const bool from_ovf = st.ovf != 0 && p.ovf != nullptr;
  if (from_ovf) {
    const uint32_t* h0 = p.w.hist(p.ws, row) + (long long)((p.level - 1) & 1) * p.w.G * 2048;
    const uint32_t pb = ((uint32_t)prefix >> tk_shift(p.level - 1)) & 0x7ffu;
    const uint32_t lim = (uint32_t)(p.w.G * p.w.CL);   // entries of the row's overflow list
    uint32_t o = 0;
    for (int c = 0; c < g; ++c) o += h0[(long long)c * 2048 + pb];
    const uint32_t e = o + h0[(long long)g * 2048 + pb];
    c0 = (int)min(o, lim);
    c1 = (int)min(max(e, o), lim);
  }
  // thread t visits the 8 consecutive entries 8t .. 8t + 7 of each 8192-entry pass, and the slots of a pass come
  // from one block scan of the per-thread counts: every list the pass appends to stays in column order (the
  // finishing pass's stable sort relies on it to order equal keys by column)
  const bool vec = !from_ovf && ((uintptr_t)x & 15u) == 0u;   // 16-byte aligned row: vector loads
  uint32_t sbase = sb, cbase = cb;                  // running slot bases of this chunk's lists
  for (int base = c0; base < c1; base += 8 * TK_NT) {
    uint32_t k[8];
    int jj[8];
    const int j0 = base + 8 * tid;
    if (from_ovf) {
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const unsigned long long e = j0 + i < c1 ? ovf_row[j0 + i] : 0ull;
        k[i] = (uint32_t)(e >> 32);
        jj[i] = (int)~(uint32_t)e;
      }
    } else if (vec && j0 + 8 <= c1) {
      if constexpr (F16) {
        const u32x4 v = *(const u32x4*)((const uint16_t*)x + j0);
#pragma unroll
        for (int i = 0; i < 4; ++i) { k[2 * i] = okey16(v[i] & 0xffffu); k[2 * i + 1] = okey16(v[i] >> 16); }
      } else {
        const f32x4 a = *(const f32x4*)((const float*)x + j0), b = *(const f32x4*)((const float*)x + j0 + 4);
#pragma unroll
        for (int i = 0; i < 4; ++i) { k[i] = okey(a[i]); k[4 + i] = okey(b[i]); }
      }
#pragma unroll
      for (int i = 0; i < 8; ++i) jj[i] = j0 + i;
    } else {
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        k[i] = j0 + i < c1 ? lkey<F16>(x, j0 + i) : 0u;
        jj[i] = j0 + i;
      }
    }
    uint32_t selm = 0, candm = 0, binm = 0;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const bool in = j0 + i < c1 && (k[i] & mask) == prefix;
      const uint32_t d = (k[i] >> shift) & 0x7ffu;
      selm |= (uint32_t)(in && (d > b || (whole && d == b))) << i;
      candm |= (uint32_t)(in && (fits || to_ovf) && d == b) << i;
      binm |= (uint32_t)(in && d == b) << i;
    }
    // both counts stay below 2^16: a pass holds 8192 entries
    uint32_t tot;
    const uint32_t off = block_excl_scan((uint32_t)__popc(selm) | ((uint32_t)__popc(candm) << 16), wsum, &tot);
    uint32_t so = sbase + (off & 0xffffu), co = cbase + (off >> 16);
    sbase += tot & 0xffffu;
    cbase += tot >> 16;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      if ((selm >> i) & 1u) { if (so < (uint32_t)TK_KMAX) sel[so] = tk_pack(k[i], jj[i]); ++so; }
      if ((candm >> i) & 1u) { if (co < clim) cand[co] = tk_pack(k[i], jj[i]); ++co; }
      if (narrow && ((binm >> i) & 1u))
        atomicAdd(&nh[(tid & (TK_HCOPY - 1)) * TK_HSTR + ((k[i] >> nshift) & 0x7ffu)], 1u);
    }
  }
  if (narrow) {                                     // level L + 1's histograms go to the other half of the buffer
    __syncthreads();
    uint32_t* out = p.w.hist(p.ws, row) + (long long)(((p.level + 1) & 1) * p.w.G + g) * 2048;
    for (int bb = tid; bb < 2048; bb += TK_NT) {
      uint32_t h = 0;
#pragma unroll
      for (int c = 0; c < TK_HCOPY; ++c) h += nh[c * TK_HSTR + bb];
      out[bb] = h;
    }
  }
}

template <bool F16, int CAPK>                      // CAPK: the launch's candidate cap (p.cap)
__global__ void __launch_bounds__(TK_NT) topk_finish_kernel(TopkWsParams p) {
  __shared__ TopkLds L;
  const int row = blockIdx.x, tid = threadIdx.x;
  const int n = tkw_n(p, row);
  const RowSrc<F16> src{lrow<F16>(p.lg, row, p.lg_st), n};
  int* o = p.out + (long long)row * p.out_st;
  int nsel = 0;
  const TkwHdr st = p.w.hdr(p.ws, row)[p.level];   // read beside the row length (unused when n <= K)
  const bool full = n <= p.K || (st.state != TKW_WHOLE && st.state != TKW_CANDS);
  if (full) {
    nsel = tk_select(src, p.K, L);                  // few columns, or ties too heavy for the lists
  } else {
    // the header's counts, kept inside the lists (they are, whenever the histograms were this row's)
    const int nsb = min(max(st.sb, 0), p.K), nbc = min(max(st.binc, 0), CAPK);
    const uint32_t nneed = (uint32_t)min(max(st.need, 0), p.K - nsb);
    const unsigned long long* sel = p.w.sel(p.ws, row);
    for (int i = tid; i < nsb; i += TK_NT) L.sel[i] = sel[i];
    if (st.state == TKW_CANDS) {
      const unsigned long long* cand = p.w.cand(p.ws, row);
      for (int i = tid; i < nbc; i += TK_NT) L.cand[i] = cand[i];
    }
    __syncthreads();
    if (st.state == TKW_CANDS)
      tk_resolve_cands<CAPK / TK_NT>(L, nbc, st.lvl, (uint32_t)st.prefix, (uint32_t)st.mask, nneed, (uint32_t)nsb, n);
    if constexpr (F16) {
      // fp16 keys: at most two radix passes (the keys' low half is zero), faster than the bitonic network here;
      // fp32 keys need three or four, slower than it (measured on the bench's indexer logits)
      tk_emit_radix<RowSrc<F16>, F16>(src, p.K, p.K, o, L);   // the lists arrive in column order
      return;
    }
    nsel = p.K;
  }
  tk_emit_sorted(src, nsel, p.K, o, L);
}

// fast_topk.local (dotsnote/engine/arcstats_pkg/arcstats/fast_topk.py:52-66, csrc/topk_select.cu:1-13, :75-201):
// the row's valid columns are j < ceil((ctx - rank) / P) (clipped to Lc); the top kl of them go to the payload
// pk[row] = [values fp32 | positions j * P + rank as int32 bits] in ascending column order; fewer than kl valid
// columns: the rest is padded with -inf values and positions s * P + rank.
struct LocalParams {
  const void* lg; long long lg_st;                // fp32 or fp16 (the kernel's F16), stride in elements
  const int* ctx; int rows, rank, P, Lc, kl;
  float* pk;
};

template <bool F16>
__global__ void __launch_bounds__(TK_NT) topk_local_kernel(LocalParams p) {
  __shared__ TopkLds L;
  const int row = blockIdx.x, tid = threadIdx.x;
  const int c = p.ctx[row];
  int n = c > p.rank ? (int)(((long long)c - p.rank + p.P - 1) / p.P) : 0;
  if (n > p.Lc) n = p.Lc;
  const RowSrc<F16> src{lrow<F16>(p.lg, row, p.lg_st), n};
  const int nsel = tk_select(src, p.kl, L);
  // ascending column order: sort descending on ~j (the low word of a selected entry)
  for (int i = tid; i < nsel; i += TK_NT) L.sel[i] = (unsigned long long)(uint32_t)L.sel[i] << 32;
  tk_sort_desc(L.sel, nsel);
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

// ---- scratch of the no-allocation top-k entry point (spmla_topk_scratch) ---------------------------------------
// File-scope device memory (each GPU holds its own copy from module load until the process ends). Host code never
// passes `scratch` itself to a kernel: its name is a host-side stand-in, not a device address. The device address
// comes from hipGetSymbolAddress, once per device, and is kept in scratch_dev[].
constexpr long long TOPK_SCRATCH_BYTES = 16ll << 20;
static __device__ __align__(256) uint8_t scratch[TOPK_SCRATCH_BYTES];

}  // namespace idx
}  // namespace spmla

#include <mutex>

namespace {
constexpr int SCRATCH_MAX_DEV = 64;
std::mutex scratch_mu;
void* scratch_dev[SCRATCH_MAX_DEV] = {};

// Device address of this device's `scratch` array (looked up on the first call on the device).
int scratch_ptr(void** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return (int)e;
  if (dev < 0 || dev >= SCRATCH_MAX_DEV) return spmla::SPMLA_ELIMIT;
  std::lock_guard<std::mutex> lock(scratch_mu);
  if (scratch_dev[dev] == nullptr) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(spmla::idx::scratch));
    if (e != hipSuccess) return (int)e;
    if (p == nullptr) return (int)hipErrorInvalidSymbol;
    scratch_dev[dev] = p;
  }
  *out = scratch_dev[dev];
  return spmla::SPMLA_OK;
}
}  // namespace

namespace spmla {
namespace idx {
// the passes of spmla_topk_ws on fp32 (F16 false) or fp16 logits
template <bool F16>
static void topk_ws_passes(TopkWsParams p, hipStream_t stream, bool hist = true) {
  p.level = 0;
  if (hist) hipLaunchKernelGGL(topk_hist_kernel<F16>, dim3(p.rows, p.w.G), dim3(TK_NT), 0, stream, p);
  for (int level = 0; level < 2; ++level) {        // the level-1 histograms come from the level-0 collect
    p.level = level;
    hipLaunchKernelGGL(topk_collect_kernel<F16>, dim3(p.rows, p.w.G), dim3(TK_NT), 0, stream, p);
  }
  p.level = 2;                                      // header 2: the state after both levels
  if (p.cap > TK_CAP1) hipLaunchKernelGGL((topk_finish_kernel<F16, TK_CAP>), dim3(p.rows), dim3(TK_NT), 0, stream, p);
  else hipLaunchKernelGGL((topk_finish_kernel<F16, TK_CAP1>), dim3(p.rows), dim3(TK_NT), 0, stream, p);
}

}  // namespace idx
}  // namespace spmla

using namespace spmla;

// Logits grid: one 12-wave workgroup per CU. With at most as many rows as CUs, each row's tiles are split over
// CUs / rows workgroups, one round of the whole grid (a wave pays its two-round-trip prologue, ~6 us under load,
// once); with more rows, workgroups of LG_TPW tiles per wave, rounds fine enough for a short tail.
inline int lg_cus() {
  static std::atomic<int> cached[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) dev = 0;
  int n = cached[dev].load(std::memory_order_relaxed);
  if (n <= 0) {
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
    cached[dev].store(n, std::memory_order_relaxed);
  }
  return n;
}
inline dim3 lg_grid(int rows, int cols, int& tpg) {
  const long long tiles = ((long long)cols + 31) / 32;      // per row
  const long long cus = lg_cus();
  const long long g = rows <= cus ? cus / rows : std::max(1LL, tiles / ((long long)idx::LG_NWV * idx::LG_TPW));
  tpg = (int)std::max(1LL, (tiles + g - 1) / g);
  return dim3(rows, (unsigned)((tiles + tpg - 1) / tpg));
}


extern "C" {

static int logits_row(const void* q, long long q_st, long long q_sh, const float* w, long long w_st,
                      const void* store, long long R_local, int rows_per_block, long long block_stride,
                      const int* block_table, long long bt_st, int block_size, const int* req, const int* ctx,
                      int rows, int H, int D, int Lc, int P, int rank, int noinf, void* out, long long out_st,
                      int out_dtype, void* stream, uint32_t* hist, long long hist_rs, int tpg, int gy) {
  if (rows < 0 || Lc < 0 || P <= 0 || rank < 0 || rank >= P || block_size <= 0 || rows_per_block <= 0) return SPMLA_EARG;
  if (out_dtype != 0 && out_dtype != 1) return SPMLA_EARG;
  if (rows == 0 || Lc == 0) return SPMLA_OK;
  if (H != 64 || D != 128) return SPMLA_ELIMIT;
  if (R_local < 0 || R_local > (long long)INT_MAX / P) return SPMLA_ELIMIT;   // 32-bit row arithmetic
  if (!q || !w || !store || !block_table || !req || !ctx || !out) return SPMLA_EARG;
  if (((uintptr_t)q & 15) || (q_st & 7) || (q_sh & 7) || ((uintptr_t)store & 3) || (block_stride & 3))
    return SPMLA_EALIGN;
  idx::LogitParams p{};
  p.q = (const uint16_t*)q; p.q_st = q_st; p.q_sh = q_sh; p.w = w; p.w_st = w_st;
  p.store = (const uint8_t*)store; p.R_local = R_local; p.rpb = rows_per_block; p.blk_stride = block_stride;
  p.bt = block_table; p.bt_st = bt_st; p.bs = block_size; p.req = req; p.ctx = ctx;
  p.rows = rows; p.Lc = Lc; p.P = P; p.rank = rank; p.noinf = noinf; p.out = out; p.out_st = out_st;
  auto log2_or = [](long long v) { return (v & (v - 1)) == 0 ? __builtin_ctzll((unsigned long long)v) : -1; };
  p.bs_sh = log2_or(block_size); p.rpb_sh = log2_or(rows_per_block); p.p_sh = log2_or(P);
  p.lim = R_local * P;
  p.clamp = 1;
  p.lo = nullptr; p.kscale = nullptr; p.k_st = 0;
  dim3 grid = lg_grid(rows, Lc, p.tpg);
  if (tpg > 0) {                                            // workgroup g = top-k chunk g < gy (the histogram's)
    p.tpg = tpg;
    grid = dim3(rows, (unsigned)gy);
  }
  p.hist = hist; p.hist_rs = hist_rs;
  const bool pow2 = p.bs_sh >= 0 && p.rpb_sh >= 0 && p.p_sh >= 0;
  if (out_dtype == 1) {
    if (pow2) hipLaunchKernelGGL((idx::logits_kernel<true, idx::LY_ROW, true>), grid, dim3(idx::LG_NWV * 64), 0, (hipStream_t)stream, p);
    else hipLaunchKernelGGL((idx::logits_kernel<false, idx::LY_ROW, true>), grid, dim3(idx::LG_NWV * 64), 0, (hipStream_t)stream, p);
  } else {
    if (pow2) hipLaunchKernelGGL((idx::logits_kernel<true, idx::LY_ROW>), grid, dim3(idx::LG_NWV * 64), 0, (hipStream_t)stream, p);
    else hipLaunchKernelGGL((idx::logits_kernel<false, idx::LY_ROW>), grid, dim3(idx::LG_NWV * 64), 0, (hipStream_t)stream, p);
  }
  return (int)hipGetLastError();
}

int spmla_index_logits(const void* q, long long q_st, long long q_sh, const float* w, long long w_st,
                       const void* store, long long R_local, int rows_per_block, long long block_stride,
                       const int* block_table, long long bt_st, int block_size, const int* req, const int* ctx,
                       int rows, int H, int D, int Lc, int P, int rank, int noinf, void* out, long long out_st,
                       int out_dtype, void* stream) {
  return logits_row(q, q_st, q_sh, w, w_st, store, R_local, rows_per_block, block_stride, block_table, bt_st,
                    block_size, req, ctx, rows, H, D, Lc, P, rank, noinf, out, out_st, out_dtype, stream, nullptr, 0, 0, 0);
}

int spmla_index_logits_hist(const void* q, long long q_st, long long q_sh, const float* w, long long w_st,
                            const void* store, long long R_local, int rows_per_block, long long block_stride,
                            const int* block_table, long long bt_st, int block_size, const int* req, const int* ctx,
                            int rows, int H, int D, int Lc, int noinf, void* out, long long out_st, int out_dtype,
                            void* topk_ws, long long ws_bytes, int K, void* stream) {
  if (rows < 0 || Lc < 0 || K <= 0 || (out_dtype != 0 && out_dtype != 1)) return SPMLA_EARG;
  if (K > idx::TK_KMAX) return SPMLA_ELIMIT;
  if (rows == 0 || Lc == 0) return SPMLA_OK;
  const idx::TopkWs tw = idx::topk_ws_layout(Lc);
  if (!topk_ws || ((uintptr_t)topk_ws & 15) || ws_bytes < (long long)rows * tw.row_bytes) return SPMLA_EARG;
  if (tw.CL >= 65536) return SPMLA_ELIMIT;                  // 16-bit counts per chunk: use the separate pass
  return logits_row(q, q_st, q_sh, w, w_st, store, R_local, rows_per_block, block_stride, block_table, bt_st,
                    block_size, req, ctx, rows, H, D, Lc, 1, 0, noinf, out, out_st, out_dtype, stream,
                    tw.hist((uint8_t*)topk_ws, 0), tw.row_bytes, tw.CL / 32, tw.G);
}

int spmla_paged_mqa_logits(const void* q, long long q_st, long long q_sh, const float* w, long long w_st,
                           const void* cache, long long num_blocks, int block_size, long long block_stride,
                           const int* block_table, long long bt_st, const int* req, const int* ctx, int rows, int H,
                           int D, int Lc, int noinf, float* out, long long out_st, void* stream) {
  if (rows < 0 || Lc < 0 || block_size <= 0 || (block_size & 15) || num_blocks < 0) return SPMLA_EARG;
  if (rows == 0 || Lc == 0) return SPMLA_OK;
  if (H != 64 || D != 128) return SPMLA_ELIMIT;
  if (num_blocks > (long long)INT_MAX / block_size) return SPMLA_ELIMIT;
  if (!q || !w || !cache || !block_table || !req || !ctx || !out) return SPMLA_EARG;
  if (((uintptr_t)q & 15) || (q_st & 7) || (q_sh & 7) || ((uintptr_t)cache & 3) || (block_stride & 3) ||
      block_stride < (long long)block_size * 132)
    return SPMLA_EALIGN;
  idx::LogitParams p{};
  p.q = (const uint16_t*)q; p.q_st = q_st; p.q_sh = q_sh; p.w = w; p.w_st = w_st;
  p.store = (const uint8_t*)cache; p.R_local = num_blocks * block_size; p.rpb = block_size;
  p.blk_stride = block_stride; p.bt = block_table; p.bt_st = bt_st; p.bs = block_size; p.req = req; p.ctx = ctx;
  p.rows = rows; p.Lc = Lc; p.P = 1; p.rank = 0; p.noinf = noinf; p.out = out; p.out_st = out_st;
  auto log2_or = [](long long v) { return (v & (v - 1)) == 0 ? __builtin_ctzll((unsigned long long)v) : -1; };
  p.bs_sh = log2_or(block_size); p.rpb_sh = p.bs_sh; p.p_sh = 0;
  p.lim = p.R_local;
  p.clamp = 0;
  p.lo = nullptr; p.kscale = nullptr; p.k_st = 0;
  const dim3 grid = lg_grid(rows, Lc, p.tpg);
  if (p.bs_sh >= 0)
    hipLaunchKernelGGL((idx::logits_kernel<true, idx::LY_SHUF>), grid, dim3(idx::LG_NWV * 64), 0, (hipStream_t)stream, p);
  else
    hipLaunchKernelGGL((idx::logits_kernel<false, idx::LY_SHUF>), grid, dim3(idx::LG_NWV * 64), 0, (hipStream_t)stream, p);
  return (int)hipGetLastError();
}

int spmla_mqa_logits(const void* q, long long q_st, long long q_sh, const float* w, long long w_st, const void* k,
                     long long k_st, const float* kscale, int N, const int* ks, const int* ke, int M, int H, int D,
                     float* out, long long out_st, void* stream) {
  if (M < 0 || N < 0) return SPMLA_EARG;
  if (M == 0 || N == 0) return SPMLA_OK;
  if (H != 64 || D != 128) return SPMLA_ELIMIT;
  if (!q || !w || !k || !kscale || !ks || !ke || !out) return SPMLA_EARG;
  if (((uintptr_t)q & 15) || (q_st & 7) || (q_sh & 7) || ((uintptr_t)k & 3) || (k_st & 3) || k_st < 128 ||
      ((uintptr_t)kscale & 3))
    return SPMLA_EALIGN;
  idx::LogitParams p{};
  p.q = (const uint16_t*)q; p.q_st = q_st; p.q_sh = q_sh; p.w = w; p.w_st = w_st;
  p.store = (const uint8_t*)k; p.R_local = N; p.rpb = 1; p.blk_stride = 0;
  p.bt = nullptr; p.bt_st = 0; p.bs = 1; p.req = nullptr; p.ctx = ke;
  p.rows = M; p.Lc = N; p.P = 1; p.rank = 0; p.noinf = 0; p.out = out; p.out_st = out_st;
  p.bs_sh = p.rpb_sh = p.p_sh = 0;
  p.lim = N;
  p.clamp = 0;
  p.lo = ks; p.kscale = kscale; p.k_st = k_st;
  const dim3 grid = lg_grid(M, N, p.tpg);
  hipLaunchKernelGGL((idx::logits_kernel<true, idx::LY_FLAT>), grid, dim3(idx::LG_NWV * 64), 0, (hipStream_t)stream, p);
  return (int)hipGetLastError();
}

int spmla_topk(const void* logits, long long lg_st, const int* ctx, int rows, int Lc, int K, int* out,
               long long out_st, int dtype, void* stream) {
  if (rows < 0 || Lc < 0 || K <= 0 || (dtype != 0 && dtype != 1)) return SPMLA_EARG;
  if (K > idx::TK_KMAX) return SPMLA_ELIMIT;
  if (rows == 0) return SPMLA_OK;
  if (!logits || !ctx || !out) return SPMLA_EARG;
  idx::TopkParams p;
  p.lg = logits; p.lg_st = lg_st; p.ctx = ctx; p.rows = rows; p.Lc = Lc; p.K = K; p.out = out; p.out_st = out_st;
  if (dtype == 1) hipLaunchKernelGGL(idx::topk_kernel<true>, dim3(rows), dim3(idx::TK_NT), 0, (hipStream_t)stream, p);
  else hipLaunchKernelGGL(idx::topk_kernel<false>, dim3(rows), dim3(idx::TK_NT), 0, (hipStream_t)stream, p);
  return (int)hipGetLastError();
}

// Workspace: the rows' headers, lists and histograms, then (optional) the rows' overflow lists of G * CL entries,
// used when a chunk's bin count fits the collect pass's 16-bit slot counters (CL < 2^16).
static long long topk_ws_base(int rows, int Lc) { return (long long)rows * idx::topk_ws_layout(Lc).row_bytes; }
static long long topk_ws_ovf(int rows, int Lc) {
  const idx::TopkWs w = idx::topk_ws_layout(Lc);
  return w.CL < 65536 ? (long long)rows * w.G * w.CL * 8 : 0;
}

long long spmla_topk_ws_bytes(int rows, int Lc, int K) {
  if (rows < 0 || Lc < 0 || K <= 0) return 0;
  return topk_ws_base(rows, Lc) + topk_ws_ovf(rows, Lc);
}

static int topk_ws_run(const void* logits, long long lg_st, const int* ctx, int rows, int Lc, int K, int* out,
                       long long out_st, void* ws, long long ws_bytes, int dtype, void* stream, bool hist) {
  if (rows < 0 || Lc < 0 || K <= 0 || (dtype != 0 && dtype != 1)) return SPMLA_EARG;
  if (K > idx::TK_KMAX) return SPMLA_ELIMIT;
  if (rows == 0) return SPMLA_OK;
  if (!logits || !ctx || !out || !ws) return SPMLA_EARG;
  const long long base = topk_ws_base(rows, Lc), ovf = topk_ws_ovf(rows, Lc);
  if (((uintptr_t)ws & 15) || ws_bytes < base) return SPMLA_EARG;
  idx::TopkWsParams p;
  p.lg = logits; p.lg_st = lg_st; p.ctx = ctx; p.rows = rows; p.Lc = Lc; p.K = K; p.out = out; p.out_st = out_st;
  p.ws = (uint8_t*)ws; p.w = idx::topk_ws_layout(Lc);
  // with room for the overflow lists, a level that narrows hands its bin's keys to the next level in a list
  p.ovf = ovf > 0 && ws_bytes >= base + ovf ? (unsigned long long*)((uint8_t*)ws + base) : nullptr;
  // fp32 rows of at most 32768 columns: the finishing pass takes boundary bins of up to 8192 keys, so the level-1
  // collect has no row to refine on indexer logits (their level-0 bins hold up to ~21% of such a row); longer rows
  // keep 4096 (their bins pass 8192 anyway, and longer candidate lists only slow the finishing pass)
  p.cap = dtype == 0 && Lc <= 32768 ? idx::TK_CAP : idx::TK_CAP1;
  if (dtype == 1) idx::topk_ws_passes<true>(p, (hipStream_t)stream, hist);
  else idx::topk_ws_passes<false>(p, (hipStream_t)stream, hist);
  return (int)hipGetLastError();
}

int spmla_topk_ws(const void* logits, long long lg_st, const int* ctx, int rows, int Lc, int K, int* out,
                  long long out_st, void* ws, long long ws_bytes, int dtype, void* stream) {
  return topk_ws_run(logits, lg_st, ctx, rows, Lc, K, out, out_st, ws, ws_bytes, dtype, stream, true);
}

int spmla_topk_ws_prehist(const void* logits, long long lg_st, const int* ctx, int rows, int Lc, int K, int* out,
                          long long out_st, void* ws, long long ws_bytes, int dtype, void* stream) {
  return topk_ws_run(logits, lg_st, ctx, rows, Lc, K, out, out_st, ws, ws_bytes, dtype, stream, false);
}

long long spmla_topk_scratch_bytes(void) { return idx::TOPK_SCRATCH_BYTES; }

int spmla_topk_scratch(const void* logits, long long lg_st, const int* ctx, int rows, int Lc, int K, int* out,
                       long long out_st, int dtype, void* stream) {
  if (rows < 0 || Lc < 0 || K <= 0 || (dtype != 0 && dtype != 1)) return SPMLA_EARG;
  if (K > idx::TK_KMAX) return SPMLA_ELIMIT;
  if (rows == 0) return SPMLA_OK;
  if (!logits || !ctx || !out) return SPMLA_EARG;
  const long long full = spmla_topk_ws_bytes(rows, Lc, K), base = topk_ws_base(rows, Lc);
  if (full <= 0) return SPMLA_EARG;
  if (base > idx::TOPK_SCRATCH_BYTES) return SPMLA_ELIMIT;   // beyond the fixed scratch: use spmla_topk_ws
  const long long need = full <= idx::TOPK_SCRATCH_BYTES ? full : base;   // the overflow lists when they fit
  void* ws = nullptr;
  const int rc = scratch_ptr(&ws);
  if (rc != SPMLA_OK) return rc;
  return spmla_topk_ws(logits, lg_st, ctx, rows, Lc, K, out, out_st, ws, need, dtype, stream);
}

int spmla_topk_local(const void* logits, long long lg_st, const int* ctx, int rows, int rank, int P, int Lc, int kl,
                     float* pk, int dtype, void* stream) {
  if (rows < 0 || Lc < 0 || kl <= 0 || P <= 0 || rank < 0 || rank >= P || (dtype != 0 && dtype != 1))
    return SPMLA_EARG;
  if (kl > idx::TK_KMAX) return SPMLA_ELIMIT;
  if (rows == 0) return SPMLA_OK;
  if (!logits || !ctx || !pk) return SPMLA_EARG;
  idx::LocalParams p;
  p.lg = logits; p.lg_st = lg_st; p.ctx = ctx; p.rows = rows; p.rank = rank; p.P = P; p.Lc = Lc; p.kl = kl; p.pk = pk;
  if (dtype == 1) hipLaunchKernelGGL(idx::topk_local_kernel<true>, dim3(rows), dim3(idx::TK_NT), 0, (hipStream_t)stream, p);
  else hipLaunchKernelGGL(idx::topk_local_kernel<false>, dim3(rows), dim3(idx::TK_NT), 0, (hipStream_t)stream, p);
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
