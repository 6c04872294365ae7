// MLA's absorbed per-head matmuls with FP8 block-scaled weights, the steps either side of the sparse attention:
//   the query build  q[t][h][0:512]   = q_nope[t][h][0:128] @ W_UK_T[h]   (then q[t][h][512:576] = q_pe[t][h])
//   the output       y[t][h][0:128]   = attn_out[t][h][0:512] @ W_UV[h]
// Reference: dotsnote/engine/arcstats_pkg/arcstats/mla_fp8.py:20-57 (_bmm_fp8_kernel) and qcat.py (the decode
// query written in place into the concatenated [T, H, 576] buffer).
//   C[n][b][j] = sum_k A[n][b][k] * bf16(W[n][j][k] * S),  S = s[n][j][k / 128] (scale_k) else s[n][k][j / 128]
// The weight is dequantized exactly as the reference does: the e4m3 code widened to fp32, multiplied by its fp32
// block scale (rounded to fp32), rounded to bf16 (RNE); the products accumulate in fp32 on MFMA.
//
// gfx950 mapping: a wave computes one 32 x 32 output tile on v_mfma_f32_32x32x16_bf16 (A operand: lane l holds row
// l % 32, k = 8 (l / 32) .. + 7; B operand: column l % 32, the same k); a workgroup's 4 waves take BT row tiles x JT
// column tiles x KS slices of K of one head (partial tiles of a K split summed through LDS). At decode sizes (B = 64)
// the two matmuls are bound by memory latency, not bandwidth or MFMA, so the shapes aim at one round trip per wave and
// one resident round of waves: a wave issues all loads of up to 8 MFMA steps (128 values of k) before any math
// (branch-free: out-of-range rows and columns read a valid row whose result is not stored, chunks beyond K are zeroed
// by selects), the k-dependent scales of the W_UK_T form are staged per round in LDS (2 loads per lane instead of 8
// per step), and consecutive workgroup ids, which the dispatcher deals round-robin to the 8 XCDs, are remapped so
// that all tiles of a head share one XCD's L2 (each head's A and W leave HBM once).
//   K <= 128 (query build, K = 128): BT = 2, JT = 2, KS = 1 (64 x 64 per workgroup, whole K per wave)
//   K >  128 (output, K = 512):     BT = 1, JT = 1, KS = 4 (32 x 32 per workgroup, a quarter of K per wave)
#include "spmla_common.h"

namespace spmla {
namespace mla {

typedef float f32x2v __attribute__((ext_vector_type(2)));

struct BmmParams {
  const uint16_t* a; long long sa_n, sa_b, sa_k;      // bf16 A[n][b][k]
  const uint8_t* w; long long sw_n, sw_j, sw_k;       // e4m3 codes W[n][j][k]
  const float* s; long long ss_n, ss_0, ss_1;         // fp32 block scales
  void* c; long long sc_n, sc_b, sc_j;                // C[n][b][j] (bf16 or fp32)
  int N, B, J, K;
  const uint16_t* qpe; long long sp_t, sp_h;          // optional: q_pe[t][h][64] copied to C row + 512 (query build)
};

typedef __bf16 bf16x2v __attribute__((ext_vector_type(2)));

// bf16 of (e4m3 code widened to fp32) * scale, with the product rounded to fp32 first (the reference's
// `(w.to(float32) * s).to(bfloat16)`): exact widening of 2 codes, 2 fp32 multiplies, one v_cvt_pk_bf16_f32 (round to
// nearest even).
__device__ inline uint32_t deq2(uint32_t codes16, float s0, float s1) {
  const f32x2v f = __builtin_amdgcn_cvt_scalef32_pk_f32_fp8(codes16, 1.0f, false);
  const f32x2v y = f32x2v{f[0] * s0, f[1] * s1};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(y, bf16x2v));
}

template <bool SCALE_K, bool OUT_F32, bool CONTIG, int BT, int JT, int KS>
__global__ void __launch_bounds__(256) bmm_fp8_kernel(BmmParams p, int TJ, int TB) {
  static_assert(BT * JT * KS == 4, "4 waves per workgroup");
  constexpr int U = 8;                                  // MFMA steps per round (128 values of k)
  __shared__ f32x4 red[KS > 1 ? (KS - 1) * BT * JT : 1][4][64];   // partial tiles of K slices 1..KS-1, per tile
  __shared__ float ls[4][128];                          // per-wave scales of one round (SCALE_K false)
  // workgroup -> (head, column tile, row tile); the ids of one XCD (i % 8) take consecutive logical tiles
  const int G = (int)gridDim.x, i = (int)blockIdx.x;
  const int L = (G & 7) ? i : (i & 7) * (G >> 3) + (i >> 3);
  const int n = L / (TJ * TB), rem = L - n * (TJ * TB);
  const int jt = rem % TJ, bt = rem / TJ;
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const int r = lane & 31, h = lane >> 5;
  const int wb = wv % BT, wj = (wv / BT) % JT, ks = wv / (BT * JT);
  const int b0 = (bt * BT + wb) * 32, j0 = (jt * JT + wj) * 32;
  const int b = b0 + r, j = j0 + r;
  const uint16_t* arow = p.a + (long long)n * p.sa_n + (long long)min(b, p.B - 1) * p.sa_b;
  const uint8_t* wrow = p.w + (long long)n * p.sw_n + (long long)min(j, p.J - 1) * p.sw_j;
  const float* sn = p.s + (long long)n * p.ss_n;
  const int jb = (jt * JT * 32) >> 7;                   // the workgroup's 128-column scale block (SCALE_K false)
  const int steps = (p.K + 15) / 16, per = (steps + KS - 1) / KS;
  const int s0 = ks * per, s1 = min(steps, s0 + per);
  f32x16 acc = f32x16{};
  for (int st = s0; st < s1; st += U) {
    u32x4 av[U];
    uint32_t wc[U][2];
    const int kb = st * 16;
    // issue every load of the round: the scales first (the first step needs them), then A and code chunks
    float s_lo, s_hi;
    const int kbl = kb >> 7;
    if (SCALE_K) {                                      // a round meets at most two 128-blocks of k
      s_lo = sn[(long long)min(j, p.J - 1) * p.ss_0 + (long long)kbl * p.ss_1];
      s_hi = sn[(long long)min(j, p.J - 1) * p.ss_0 + (long long)min(kbl + 1, (p.K - 1) >> 7) * p.ss_1];
    } else {                                            // lane l fetches the scales of k = kb + l and kb + 64 + l
      s_lo = sn[(long long)min(kb + lane, p.K - 1) * p.ss_0 + (long long)jb * p.ss_1];
      s_hi = sn[(long long)min(kb + 64 + lane, p.K - 1) * p.ss_0 + (long long)jb * p.ss_1];
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int kk = min(kb + 16 * u + 8 * h, p.K - 8);   // clamped; chunks at or beyond K are zeroed below
      if (CONTIG) {
        av[u] = *(const u32x4*)(arow + kk);
        const uint2 x = *(const uint2*)(wrow + kk);
        wc[u][0] = x.x; wc[u][1] = x.y;
      } else {
#pragma unroll
        for (int e = 0; e < 4; ++e)
          av[u][e] = (uint32_t)arow[(kk + 2 * e) * p.sa_k] | ((uint32_t)arow[(kk + 2 * e + 1) * p.sa_k] << 16);
        wc[u][0] = wc[u][1] = 0;
#pragma unroll
        for (int e = 0; e < 8; ++e) wc[u][e >> 2] |= (uint32_t)wrow[(kk + e) * p.sw_k] << (8 * (e & 3));
      }
    }
    if (!SCALE_K) {
      ls[wv][lane] = s_lo;
      ls[wv][64 + lane] = s_hi;
      __builtin_amdgcn_wave_barrier();
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const bool kok = st + u < s1 && kb + 16 * u + 8 * h < p.K;   // K % 8 == 0: a chunk is whole or absent
      float sc[8];
      if (SCALE_K) {
        const float sv = ((kb + 16 * u) >> 7) == kbl ? s_lo : s_hi;
#pragma unroll
        for (int e = 0; e < 8; ++e) sc[e] = sv;
      } else {
        const f32x4 x0 = *(const f32x4*)&ls[wv][16 * u + 8 * h];
        const f32x4 x1 = *(const f32x4*)&ls[wv][16 * u + 8 * h + 4];
#pragma unroll
        for (int e = 0; e < 4; ++e) { sc[e] = x0[e]; sc[4 + e] = x1[e]; }
      }
      u32x4 wv4, a4;
      wv4[0] = deq2(wc[u][0] & 0xffffu, sc[0], sc[1]);
      wv4[1] = deq2(wc[u][0] >> 16, sc[2], sc[3]);
      wv4[2] = deq2(wc[u][1] & 0xffffu, sc[4], sc[5]);
      wv4[3] = deq2(wc[u][1] >> 16, sc[6], sc[7]);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        a4[e] = kok ? av[u][e] : 0u;
        wv4[e] = kok ? wv4[e] : 0u;
      }
      acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a4), __builtin_bit_cast(bf16x8, wv4),
                                                    acc, 0, 0, 0);
    }
    if (!SCALE_K) __builtin_amdgcn_wave_barrier();
  }
  if (KS > 1) {                                         // K slices 1..KS-1 hand their tiles to slice 0 in LDS
    if (ks > 0) {
#pragma unroll
      for (int q = 0; q < 4; ++q)
        red[(ks - 1) * BT * JT + wb + BT * wj][q][lane] =
            f32x4{acc[4 * q], acc[4 * q + 1], acc[4 * q + 2], acc[4 * q + 3]};
    }
    __syncthreads();
    if (ks == 0) {
#pragma unroll
      for (int v = 0; v < KS - 1; ++v)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const f32x4 x = red[v * BT * JT + wb + BT * wj][q][lane];
#pragma unroll
          for (int e = 0; e < 4; ++e) acc[4 * q + e] += x[e];
        }
    }
  }
  // C layout: column j0 + lane % 32, rows b0 + 8 (i / 4) + 4 h + i % 4
  if (ks == 0 && j < p.J) {
#pragma unroll
    for (int ii = 0; ii < 16; ++ii) {
      const int bb = b0 + 8 * (ii >> 2) + 4 * h + (ii & 3);
      if (bb < p.B) {
        const long long off = (long long)n * p.sc_n + (long long)bb * p.sc_b + (long long)j * p.sc_j;
        if (OUT_F32) ((float*)p.c)[off] = acc[ii];
        else ((uint16_t*)p.c)[off] = f2bf_rne(acc[ii]);
      }
    }
  }
  // query build: the column-tile 0 workgroups also copy q_pe of their rows into columns 512 .. 575 (8 x 16 B a row)
  if (p.qpe && jt == 0) {
    for (int e = threadIdx.x; e < BT * 32 * 8; e += 256) {
      const int bb = bt * BT * 32 + (e >> 3), q = e & 7;
      if (bb < p.B) {
        const u32x4 v = *(const u32x4*)(p.qpe + (long long)bb * p.sp_t + (long long)n * p.sp_h + q * 8);
        *(u32x4*)((uint16_t*)p.c + (long long)n * p.sc_n + (long long)bb * p.sc_b + 512 + q * 8) = v;
      }
    }
  }
}


// LDS-staged form for contiguous, 16-byte aligned operands with K % 16 == 0 (the shapes of both MLA matmuls).
// Loading fragments straight into the MFMA layout makes every 16-byte load touch 32 rows, so each 128-byte line is
// requested 4 times and the L2 request rate, not HBM, bounds the launch (measured: 13.5 / 12.1 us vs 11.0 / 8.0 us
// with the same loads coalesced). Here a round's A rows (bf16) and W rows (e4m3 codes) of the workgroup's tile are
// read with coalesced 16-byte loads (16 lanes cover a 256-byte row) into LDS rows padded by 16 / 8 bytes (fragment
// reads of 32 rows then fall on distinct banks); chunks at or beyond K are stored as zeros. Each wave then runs its 8
// MFMA steps (128 values of k of its slice) from LDS, dequantizing its 8 codes per step in registers. The MFMA
// computes C^T (W fragment as the row operand), so a lane ends with 4 consecutive columns of a row: the tile goes
// through LDS once more and leaves as full-row 16-byte stores.
//   tile: BT x 32 rows b, JT x 32 columns j; KS waves split each round's KR = 128 KS values of k.
template <bool SCALE_K, bool OUT_F32, int BT, int JT, int KS>
struct Staged {
  static constexpr int NT = 64 * BT * JT * KS;          // threads
  static constexpr int BM = 32 * BT, BN = 32 * JT, KR = 128 * KS;
  static constexpr int PA = KR * 2 + 16;                // A row pitch in LDS (bytes)
  static constexpr int PW = KR + 8;                     // code row pitch
  static constexpr int ESZ = OUT_F32 ? 4 : 2;
  static constexpr int PO = BN * ESZ + 16;              // output tile pitch
  static constexpr int AS = 0, WS = BM * PA, SS = WS + BN * PW;
  static constexpr int STAGE = SS + (SCALE_K ? 0 : KR * 4);
  static constexpr int RED = 0, OT = (KS - 1) * BT * JT * 4096;
  static constexpr int EPI = OT + BM * PO;
  static constexpr int LDS = STAGE > EPI ? STAGE : EPI;
  static constexpr int A_CH = BM * KR / 8, W_CH = BN * KR / 16;   // 16-byte chunks per round
  static_assert(JT <= 4, "a workgroup's columns must share one 128-column scale block");
  static_assert(LDS <= 160 * 1024, "LDS");
};

template <bool SCALE_K, bool OUT_F32, int BT, int JT, int KS>
__global__ void __launch_bounds__(64 * BT * JT * KS) bmm_fp8_staged_kernel(BmmParams p, int TJ, int TB) {
  using C = Staged<SCALE_K, OUT_F32, BT, JT, KS>;
  __shared__ __attribute__((aligned(16))) uint8_t sm[C::LDS];
  const int G = (int)gridDim.x, i = (int)blockIdx.x;
  const int L = (G & 7) ? i : (i & 7) * (G >> 3) + (i >> 3);   // tiles of a head on one XCD (ids i % 8 share one)
  const int n = L / (TJ * TB), rem = L - n * (TJ * TB);
  const int jt = rem % TJ, bt = rem / TJ;
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int c = lane & 31, h = lane >> 5;
  const int wb = wv % BT, wj = (wv / BT) % JT, ks = wv / (BT * JT);
  const int B0 = bt * C::BM, J0 = jt * C::BN;           // the workgroup's first row and column
  const uint16_t* an = p.a + (long long)n * p.sa_n;
  const uint8_t* wn = p.w + (long long)n * p.sw_n;
  const float* sn = p.s + (long long)n * p.ss_n;
  const int jb = J0 >> 7;
  f32x16 acc = f32x16{};
  for (int kb = 0; kb < p.K; kb += C::KR) {
    if (kb) __syncthreads();                            // the previous round's fragment reads are done
    // coalesced loads of the round: A chunk q = (row q / (KR / 8), 8 values), W chunk q = (row q / (KR / 16), 16 codes)
    u32x4 ra[(C::A_CH + C::NT - 1) / C::NT], rw[(C::W_CH + C::NT - 1) / C::NT];
#pragma unroll
    for (int e = 0; e < (C::A_CH + C::NT - 1) / C::NT; ++e) {
      const int q = tid + e * C::NT;
      const int row = min(q / (C::KR / 8), C::BM - 1), k = kb + (q % (C::KR / 8)) * 8;
      // branch-free: a clamped in-range address, zeros selected afterwards (a load under a branch costs a full wait)
      const u32x4 v = *(const u32x4*)(an + (long long)min(B0 + row, p.B - 1) * p.sa_b + min(k, p.K - 8));
      ra[e] = k < p.K ? v : u32x4{0, 0, 0, 0};
    }
#pragma unroll
    for (int e = 0; e < (C::W_CH + C::NT - 1) / C::NT; ++e) {
      const int q = tid + e * C::NT;
      const int row = min(q / (C::KR / 16), C::BN - 1), k = kb + (q % (C::KR / 16)) * 16;
      const u32x4 v = *(const u32x4*)(wn + (long long)min(J0 + row, p.J - 1) * p.sw_j + min(k, p.K - 16));
      rw[e] = k < p.K ? v : u32x4{0, 0, 0, 0};
    }
    float sv = 0.f;                                     // SCALE_K: this lane's column, this wave's 128-block of k
    float rs[(C::KR + C::NT - 1) / C::NT];              // else: the scales of k = kb + tid (+ NT ..) at block jb
    if (SCALE_K) {
      const int kblk = min((kb + 128 * ks) >> 7, (p.K - 1) >> 7);
      sv = sn[(long long)min(J0 + wj * 32 + c, p.J - 1) * p.ss_0 + (long long)kblk * p.ss_1];
    } else {
#pragma unroll
      for (int e = 0; e < (C::KR + C::NT - 1) / C::NT; ++e) {
        const int k = kb + tid + e * C::NT;
        const float v = sn[(long long)min(k, p.K - 1) * p.ss_0 + (long long)jb * p.ss_1];
        rs[e] = k < p.K ? v : 0.f;
      }
    }
    if (!SCALE_K) {
#pragma unroll
      for (int e = 0; e < (C::KR + C::NT - 1) / C::NT; ++e)
        if (tid + e * C::NT < C::KR) ((float*)(sm + C::SS))[tid + e * C::NT] = rs[e];
    }
#pragma unroll
    for (int e = 0; e < (C::A_CH + C::NT - 1) / C::NT; ++e) {
      const int q = tid + e * C::NT;
      if (q < C::A_CH) *(u32x4*)(sm + C::AS + (q / (C::KR / 8)) * C::PA + (q % (C::KR / 8)) * 16) = ra[e];
    }
#pragma unroll
    for (int e = 0; e < (C::W_CH + C::NT - 1) / C::NT; ++e) {
      const int q = tid + e * C::NT;
      if (q < C::W_CH) {                                // code rows are 8-byte aligned (pitch KR + 8)
        uint2* d = (uint2*)(sm + C::WS + (q / (C::KR / 16)) * C::PW + (q % (C::KR / 16)) * 16);
        d[0] = uint2{rw[e][0], rw[e][1]};
        d[1] = uint2{rw[e][2], rw[e][3]};
      }
    }
    __syncthreads();
    // 8 MFMA steps over this wave's slice: k = kb + 128 ks + 16 u + 8 h .. + 7 in lane (c, h)
    const uint8_t* fa = sm + C::AS + (wb * 32 + c) * C::PA + (128 * ks + 8 * h) * 2;
    const uint8_t* fw = sm + C::WS + (wj * 32 + c) * C::PW + 128 * ks + 8 * h;
    const float* fs = (const float*)(sm + C::SS) + 128 * ks + 8 * h;
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const u32x4 a4 = *(const u32x4*)(fa + 32 * u);
      const uint2 w2 = *(const uint2*)(fw + 16 * u);
      float sc[8];
      if (SCALE_K) {
#pragma unroll
        for (int e = 0; e < 8; ++e) sc[e] = sv;
      } else {
        const f32x4 x0 = *(const f32x4*)(fs + 16 * u), x1 = *(const f32x4*)(fs + 16 * u + 4);
#pragma unroll
        for (int e = 0; e < 4; ++e) { sc[e] = x0[e]; sc[4 + e] = x1[e]; }
      }
      u32x4 w4;
      w4[0] = deq2(w2.x & 0xffffu, sc[0], sc[1]);
      w4[1] = deq2(w2.x >> 16, sc[2], sc[3]);
      w4[2] = deq2(w2.y & 0xffffu, sc[4], sc[5]);
      w4[3] = deq2(w2.y >> 16, sc[6], sc[7]);
      acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, w4), __builtin_bit_cast(bf16x8, a4),
                                                    acc, 0, 0, 0);
    }
  }
  __syncthreads();                                      // staging area free: partial sums and the output tile
  if (KS > 1) {
    f32x4* red = (f32x4*)(sm + C::RED);
    const int slot = wb + BT * wj;
    if (ks > 0) {
#pragma unroll
      for (int q = 0; q < 4; ++q)
        red[(((ks - 1) * BT * JT + slot) * 4 + q) * 64 + lane] =
            f32x4{acc[4 * q], acc[4 * q + 1], acc[4 * q + 2], acc[4 * q + 3]};
    }
    __syncthreads();
    if (ks == 0) {
#pragma unroll
      for (int v = 0; v < KS - 1; ++v)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const f32x4 x = red[((v * BT * JT + slot) * 4 + q) * 64 + lane];
#pragma unroll
          for (int e = 0; e < 4; ++e) acc[4 * q + e] += x[e];
        }
    }
  }
  // C^T layout: lane (c, h) holds row b = wb * 32 + c, columns wj * 32 + 8 q + 4 h + e (acc[4 q + e])
  if (ks == 0) {
    uint8_t* ot = sm + C::OT + (wb * 32 + c) * C::PO;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int col = wj * 32 + 8 * q + 4 * h;
      if (OUT_F32) {
        *(f32x4*)(ot + col * 4) = f32x4{acc[4 * q], acc[4 * q + 1], acc[4 * q + 2], acc[4 * q + 3]};
      } else {
        const uint32_t lo = __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2v{acc[4 * q], acc[4 * q + 1]},
                                                                                 bf16x2v));
        const uint32_t hi = __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2v{acc[4 * q + 2], acc[4 * q + 3]},
                                                                                 bf16x2v));
        *(uint2*)(ot + col * 2) = uint2{lo, hi};
      }
    }
  }
  __syncthreads();
  constexpr int RC = C::BN * C::ESZ / 16;               // 16-byte chunks per output row
  for (int q = tid; q < C::BM * RC; q += C::NT) {
    const int row = q / RC, cc = q % RC;
    const int b = B0 + row, j = J0 + cc * (16 / C::ESZ);
    if (b < p.B && j < p.J)
      *(u32x4*)((uint8_t*)p.c + ((long long)n * p.sc_n + (long long)b * p.sc_b + j) * C::ESZ) =
          *(const u32x4*)(sm + C::OT + row * C::PO + cc * 16);
  }
  // query build: the column-tile 0 workgroups also copy q_pe of their rows into columns 512 .. 575 (8 x 16 B a row)
  if (p.qpe && jt == 0) {
    for (int e = tid; e < C::BM * 8; e += C::NT) {
      const int bb = B0 + (e >> 3), q = e & 7;
      if (bb < p.B) {
        const u32x4 v = *(const u32x4*)(p.qpe + (long long)bb * p.sp_t + (long long)n * p.sp_h + q * 8);
        *(u32x4*)((uint16_t*)p.c + (long long)n * p.sc_n + (long long)bb * p.sc_b + 512 + q * 8) = v;
      }
    }
  }
}

}  // namespace mla
}  // namespace spmla

using namespace spmla;

template <bool SK, bool OF, bool CT>
static void bmm_go(const mla::BmmParams& p, hipStream_t s) {
  if (p.K <= 128) {
    const int TJ = (p.J + 63) / 64, TB = (p.B + 63) / 64;
    hipLaunchKernelGGL((mla::bmm_fp8_kernel<SK, OF, CT, 2, 2, 1>), dim3((unsigned)(p.N * TJ * TB)), dim3(256), 0, s, p,
                       TJ, TB);
  } else {
    const int TJ = (p.J + 31) / 32, TB = (p.B + 31) / 32;
    hipLaunchKernelGGL((mla::bmm_fp8_kernel<SK, OF, CT, 1, 1, 4>), dim3((unsigned)(p.N * TJ * TB)), dim3(256), 0, s, p,
                       TJ, TB);
  }
}

template <bool SK, bool OF, int BT, int JT, int KS>
static void staged_go(const mla::BmmParams& p, hipStream_t s) {
  const int TJ = (p.J + 32 * JT - 1) / (32 * JT), TB = (p.B + 32 * BT - 1) / (32 * BT);
  hipLaunchKernelGGL((mla::bmm_fp8_staged_kernel<SK, OF, BT, JT, KS>), dim3((unsigned)(p.N * TJ * TB)),
                     dim3(64 * BT * JT * KS), 0, s, p, TJ, TB);
}

// K <= 128 (the query build): 64 x 128 tiles, 8 waves, one round; larger K (the output, K = 512): 64 x 64 tiles,
// 16 waves over 4 slices of 128 k, one round of 512. Measured at B = 64, H = 128 (back-to-back launches): query
// 6.2 us (64 x 64 / 4 waves 7.2, 32 x 128 6.9, 32 x 64 7.6); output 6.0 us (32 x 64 x 4 slices 6.3, 64 x 64 x 2
// slices 6.5, 32 x 128 x 2 6.7, 32 x 32 x 2 7.9, 32 x 32 x 4 8.6).
template <bool SK, bool OF>
static void staged_pick(const mla::BmmParams& p, hipStream_t s) {
  if (p.K <= 128) staged_go<SK, OF, 2, 4, 1>(p, s);
  else staged_go<SK, OF, 2, 2, 4>(p, s);
}

static int bmm_launch(mla::BmmParams& p, int scale_k, int out_f32, void* stream) {
  if (p.N < 0 || p.B < 0 || p.J < 0 || p.K < 0 || (p.K & 7)) return SPMLA_EARG;
  if (p.N == 0 || p.B == 0 || p.J == 0) return SPMLA_OK;
  if (!p.a || !p.w || !p.s || !p.c) return SPMLA_EARG;
  const bool contig = p.sa_k == 1 && p.sw_k == 1;
  if (contig && (((uintptr_t)p.a & 15) || (p.sa_n & 7) || (p.sa_b & 7))) return SPMLA_EALIGN;
  if (contig && (((uintptr_t)p.w & 7) || (p.sw_n & 7) || (p.sw_j & 7))) return SPMLA_EALIGN;
  if ((long long)p.N * ((p.J + 31) / 32) * ((p.B + 31) / 32) > 0x7fffffffLL) return SPMLA_ELIMIT;
  hipStream_t s = (hipStream_t)stream;
  const int esz = out_f32 ? 4 : 2;
  const bool staged = contig && (p.K & 15) == 0 && !((uintptr_t)p.w & 15) && !(p.sw_n & 15) && !(p.sw_j & 15) &&
                      !((uintptr_t)p.c & 15) && p.sc_j == 1 && !((p.sc_n * esz) & 15) && !((p.sc_b * esz) & 15) &&
                      !((p.J * esz) & 15);
  if (staged) {
    if (scale_k) {
      if (out_f32) staged_pick<true, true>(p, s);
      else staged_pick<true, false>(p, s);
    } else {
      if (out_f32) staged_pick<false, true>(p, s);
      else staged_pick<false, false>(p, s);
    }
    return (int)hipGetLastError();
  }
  const int v = (scale_k ? 4 : 0) | (out_f32 ? 2 : 0) | (contig ? 1 : 0);
  switch (v) {
    case 0: bmm_go<false, false, false>(p, s); break;
    case 1: bmm_go<false, false, true>(p, s); break;
    case 2: bmm_go<false, true, false>(p, s); break;
    case 3: bmm_go<false, true, true>(p, s); break;
    case 4: bmm_go<true, false, false>(p, s); break;
    case 5: bmm_go<true, false, true>(p, s); break;
    case 6: bmm_go<true, true, false>(p, s); break;
    default: bmm_go<true, true, true>(p, s); break;
  }
  return (int)hipGetLastError();
}

extern "C" {

int spmla_bmm_fp8(const void* a, long long sa_n, long long sa_b, long long sa_k, const void* w, long long sw_n,
                  long long sw_j, long long sw_k, const float* s, long long ss_n, long long ss_0, long long ss_1,
                  int scale_k, void* c, long long sc_n, long long sc_b, long long sc_j, int out_f32, int N, int B,
                  int J, int K, void* stream) {
  mla::BmmParams p;
  p.a = (const uint16_t*)a; p.sa_n = sa_n; p.sa_b = sa_b; p.sa_k = sa_k;
  p.w = (const uint8_t*)w; p.sw_n = sw_n; p.sw_j = sw_j; p.sw_k = sw_k;
  p.s = s; p.ss_n = ss_n; p.ss_0 = ss_0; p.ss_1 = ss_1;
  p.c = c; p.sc_n = sc_n; p.sc_b = sc_b; p.sc_j = sc_j;
  p.N = N; p.B = B; p.J = J; p.K = K; p.qpe = nullptr; p.sp_t = p.sp_h = 0;
  return bmm_launch(p, scale_k, out_f32, stream);
}

int spmla_mla_query(const void* q_nope, long long qn_st, long long qn_sh, const void* q_pe, long long qp_st,
                    long long qp_sh, const void* w_uk, const float* s_uk, int T, int H, void* q, long long q_st,
                    long long q_sh, void* stream) {
  if (T < 0 || H <= 0) return SPMLA_EARG;
  if (T == 0) return SPMLA_OK;
  if (!q_nope || !q_pe || !w_uk || !s_uk || !q) return SPMLA_EARG;
  if (((uintptr_t)q_pe & 15) || (qp_st & 7) || (qp_sh & 7) || ((uintptr_t)q & 15) || (q_st & 7) || (q_sh & 7))
    return SPMLA_EALIGN;
  mla::BmmParams p;
  // A[n = head][b = token][k] = q_nope[t][h][k]; W = codes [H][512][128] contiguous; s = [H][128][4] (scale over k)
  p.a = (const uint16_t*)q_nope; p.sa_n = qn_sh; p.sa_b = qn_st; p.sa_k = 1;
  p.w = (const uint8_t*)w_uk; p.sw_n = 512 * 128; p.sw_j = 128; p.sw_k = 1;
  p.s = s_uk; p.ss_n = 128 * 4; p.ss_0 = 4; p.ss_1 = 1;
  p.c = q; p.sc_n = q_sh; p.sc_b = q_st; p.sc_j = 1;
  p.N = H; p.B = T; p.J = 512; p.K = 128;
  p.qpe = (const uint16_t*)q_pe; p.sp_t = qp_st; p.sp_h = qp_sh;
  return bmm_launch(p, 0, 0, stream);
}

}  // extern "C"
