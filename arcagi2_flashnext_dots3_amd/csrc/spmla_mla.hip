// MLA's absorbed per-head matmuls with FP8 block-scaled weights, the steps either side of the sparse attention:
//   the query build  q[t][h][0:512]   = q_nope[t][h][0:128] @ W_UK_T[h]   (then q[t][h][512:576] = q_pe[t][h])
//   the output       y[t][h][0:128]   = attn_out[t][h][0:512] @ W_UV[h]
// Reference: dotsnote/engine/arcstats_pkg/arcstats/mla_fp8.py:20-57 (_bmm_fp8_kernel) and qcat.py (the decode
// query written in place into the concatenated [T, H, 576] buffer).
//   C[n][b][j] = sum_k A[n][b][k] * bf16(W[n][j][k] * S),  S = s[n][j][k / 128] (scale_k) else s[n][k][j / 128]
// The weight is dequantized exactly as the reference does: the e4m3 code widened to fp32, multiplied by its fp32
// block scale (rounded to fp32), rounded to bf16 (RNE); the products accumulate in fp32 on MFMA.
//
// gfx950 mapping: one workgroup = (head n, 64 columns j, 64 rows b), 4 waves of 32 x 32 output tiles on
// v_mfma_f32_32x32x16_bf16 (A operand: lane l holds row l % 32, k = 8 (l / 32) .. + 7; B operand: column l % 32,
// the same k). Fragments come straight from global memory (16-byte A loads, 8-byte code loads): at decode sizes the
// launch is bound by latency and the 8.4 MB of FP8 weights, not by MFMA.
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

// bf16 of (e4m3 code widened to fp32) * scale, with the product rounded to fp32 first (the reference's
// `(w.to(float32) * s).to(bfloat16)`).
__device__ inline uint32_t deq2(uint32_t codes16, float s0, float s1) {
  const f32x2v f = __builtin_amdgcn_cvt_scalef32_pk_f32_fp8(codes16, 1.0f, false);   // exact widening of 2 codes
  return (uint32_t)f2bf_rne(f[0] * s0) | ((uint32_t)f2bf_rne(f[1] * s1) << 16);
}

template <bool SCALE_K, bool OUT_F32>
__global__ void __launch_bounds__(256) bmm_fp8_kernel(BmmParams p) {
  const int n = blockIdx.x;
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const int r = lane & 31, h = lane >> 5;
  const int b0 = blockIdx.z * 64 + (wv & 1) * 32, j0 = blockIdx.y * 64 + (wv >> 1) * 32;
  const int b = b0 + r, j = j0 + r;
  const bool bok = b < p.B, jok = j < p.J;
  const uint16_t* arow = p.a + (long long)n * p.sa_n + (long long)(bok ? b : 0) * p.sa_b;
  const uint8_t* wrow = p.w + (long long)n * p.sw_n + (long long)(jok ? j : 0) * p.sw_j;
  const float* sn = p.s + (long long)n * p.ss_n;
  f32x16 acc = f32x16{};
  for (int k0 = 0; k0 < p.K; k0 += 16) {
    const int kk = k0 + 8 * h;                          // this lane's 8 values of k
    const bool kok = kk < p.K;                          // K % 8 == 0: a chunk is whole or absent
    u32x4 av = u32x4{0, 0, 0, 0};
    if (bok && kok) {
      if (p.sa_k == 1) {
        av = *(const u32x4*)(arow + kk);
      } else {
#pragma unroll
        for (int e = 0; e < 4; ++e)
          av[e] = (uint32_t)arow[(kk + 2 * e) * p.sa_k] | ((uint32_t)arow[(kk + 2 * e + 1) * p.sa_k] << 16);
      }
    }
    u32x4 wv4 = u32x4{0, 0, 0, 0};
    if (jok && kok) {
      uint32_t c[2];
      if (p.sw_k == 1) {
        const uint2 x = *(const uint2*)(wrow + kk);
        c[0] = x.x; c[1] = x.y;
      } else {
        c[0] = c[1] = 0;
#pragma unroll
        for (int e = 0; e < 8; ++e) c[e >> 2] |= (uint32_t)wrow[(kk + e) * p.sw_k] << (8 * (e & 3));
      }
      float sc[8];
      if (SCALE_K) {
        const float s = sn[(long long)j * p.ss_0 + (long long)(kk >> 7) * p.ss_1];
#pragma unroll
        for (int e = 0; e < 8; ++e) sc[e] = s;
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) sc[e] = sn[(long long)(kk + e) * p.ss_0 + (long long)(j >> 7) * p.ss_1];
      }
      wv4[0] = deq2(c[0] & 0xffffu, sc[0], sc[1]);
      wv4[1] = deq2(c[0] >> 16, sc[2], sc[3]);
      wv4[2] = deq2(c[1] & 0xffffu, sc[4], sc[5]);
      wv4[3] = deq2(c[1] >> 16, sc[6], sc[7]);
    }
    acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, av), __builtin_bit_cast(bf16x8, wv4), acc,
                                                  0, 0, 0);
  }
  // C layout: column j0 + lane % 32, rows b0 + 8 (i / 4) + 4 h + i % 4
  if (jok) {
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int bb = b0 + 8 * (i >> 2) + 4 * h + (i & 3);
      if (bb < p.B) {
        const long long off = (long long)n * p.sc_n + (long long)bb * p.sc_b + (long long)j * p.sc_j;
        if (OUT_F32) ((float*)p.c)[off] = acc[i];
        else ((uint16_t*)p.c)[off] = f2bf_rne(acc[i]);
      }
    }
  }
  // query build: the j-tile 0 workgroups also copy q_pe of their rows into columns 512 .. 575 (64 bf16 = 8 x 16 B)
  if (p.qpe && blockIdx.y == 0) {
    for (int e = threadIdx.x; e < 64 * 8; e += 256) {
      const int bb = blockIdx.z * 64 + (e >> 3), q = e & 7;
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

extern "C" {

static int bmm_launch(mla::BmmParams& p, int scale_k, int out_f32, void* stream) {
  if (p.N < 0 || p.B < 0 || p.J < 0 || p.K < 0 || (p.K & 7)) return SPMLA_EARG;
  if (p.N == 0 || p.B == 0 || p.J == 0) return SPMLA_OK;
  if (!p.a || !p.w || !p.s || !p.c) return SPMLA_EARG;
  if (p.sa_k == 1 && (((uintptr_t)p.a & 15) || (p.sa_n & 7) || (p.sa_b & 7))) return SPMLA_EALIGN;
  if (p.sw_k == 1 && (((uintptr_t)p.w & 7) || (p.sw_n & 7) || (p.sw_j & 7))) return SPMLA_EALIGN;
  if (p.N > 65535 || (p.J + 63) / 64 > 65535 || (p.B + 63) / 64 > 65535) return SPMLA_ELIMIT;
  const dim3 grid((unsigned)p.N, (unsigned)((p.J + 63) / 64), (unsigned)((p.B + 63) / 64));
  hipStream_t s = (hipStream_t)stream;
  if (scale_k) {
    if (out_f32) hipLaunchKernelGGL((mla::bmm_fp8_kernel<true, true>), grid, dim3(256), 0, s, p);
    else hipLaunchKernelGGL((mla::bmm_fp8_kernel<true, false>), grid, dim3(256), 0, s, p);
  } else {
    if (out_f32) hipLaunchKernelGGL((mla::bmm_fp8_kernel<false, true>), grid, dim3(256), 0, s, p);
    else hipLaunchKernelGGL((mla::bmm_fp8_kernel<false, false>), grid, dim3(256), 0, s, p);
  }
  return (int)hipGetLastError();
}

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
