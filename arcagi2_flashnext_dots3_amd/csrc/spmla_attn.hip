// Sparse-MLA decode / prefill attention over gathered Row656 KV rows, and the log-sum-exp merge of partials.
//
// Math (reference: dotsnote/kaggle/runtime_dataset/bench_offload_attn2.py:77-93 and
// dotsnote/engine/vllm_patch/vllm/v1/attention/ops/xpu_mla_sparse.py:77-161):
//   row r of token t = idx[t][k] (valid iff 0 <= idx < R); latent_d = e4m3(code_d) * scale[d / 128], rope bf16
//   s[h][k] = sm_scale * kv_scale * (q[h][:512] . latent + q[h][512:] . rope)           (fp32)
//   p = exp2(s * log2e - m), o[h] = kv_scale * sum_k p latent / sum_k p,  lse = ln sum_k exp(s)
//   invalid entries contribute nothing; a token with no valid entry gives o = 0 and lse = -inf.
//
// gfx950 mapping. One workgroup = (token t, group of 32 heads, split s); TEAMS x 4 waves.
//   * Rows are staged through a ring of NBUF 32-row tiles in LDS with direct global->LDS copies
//     (global_load_lds_dwordx4), chunk-major layout [chunk][row][16 B]: each MFMA operand read is a conflict-free
//     ds_read_b128 and the V^T operand is one ds_read_b64_tr_b8 (8 rows x 16 columns per 16-lane group).
//   * In a team, wave w owns latent scale group w (columns 128w..128w+127) and rope quarter w for QK, and the same
//     128 output columns for PV. QK on bf16 MFMA (32x32x16): e4m3 codes convert exactly to bf16, two per
//     v_cvt_scalef32_pk_bf16_fp8; the per-row group scale multiplies the fp32 partial. (fp8 MFMA is not used for
//     QK: its internal accumulation keeps only ~2^-12 of the largest product, measured on gfx950.)
//     Partial S^T tiles (32 rows x 32 heads) meet in LDS; wave w runs the online softmax of heads 8w..8w+7 and
//     publishes P and the rescale factor; PV on fp16 MFMA with P' = P * scale (fp16, RNE) and the codes in fp16.
//   * Lazy rescaling: the reference max m of a head moves only when a tile exceeds it by more than TAU (log2
//     units), so p <= 2^TAU: an exact softmax either way, fewer rescales of O.
//   * With TEAMS = 2 the two teams take alternate tiles (2 waves per SIMD hide each other's latencies); their
//     states merge in LDS at the end.
#include "spmla_common.h"
#include <stdlib.h>

namespace spmla {
namespace attn {

constexpr int HG = 32;                // heads per workgroup
constexpr int TR = 32;                // rows per tile
constexpr int KMAX = 2048;            // selected rows per (token, split) staged in LDS
constexpr float TAU = 4.0f;
constexpr float F16_MAX = 65504.0f;

// tile layout (bytes)
constexpr int T_LAT = 0;                       // 32 latent chunks: [c][r][16]
constexpr int T_ROPE = 32 * TR * 16;           // 8 rope chunks:    [e][r][16]   (16384)
constexpr int T_SC = T_ROPE + 8 * TR * 16;     // scales:           [g][r] f32   (20480)
constexpr int TILE = T_SC + 4 * TR * 4;        // 20992
constexpr int NCOPY = 22;                      // copy instructions per tile

// exchange layouts, in 16-byte units (4 rows of one head), padded to 33 heads per row block
constexpr int XS_UNITS = 4 * 8 * 33;           // S partials [w][rb][h]
constexpr int XP_UNITS = 8 * 33;               // P [rb][h]

template <int TEAMS, int NBUF>
struct Lds {
  static constexpr int TILES = 0;
  static constexpr int S = TILES + NBUF * TILE;
  static constexpr int P = S + TEAMS * XS_UNITS * 16;
  static constexpr int IDX = P + TEAMS * XP_UNITS * 16;
  static constexpr int MISC = IDX + KMAX * 4;              // per team: alpha[32], m[32], l[32]
  static constexpr int TOTAL = MISC + TEAMS * 3 * 32 * 4;
  static_assert(TOTAL <= 160 * 1024, "LDS budget");
};

#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"   // m0 is reserved; nothing else in these kernels uses it
// Direct global->LDS copies (lane l's bytes land at lds + size * l). Issued through inline asm so that the
// compiler does not track them: it would otherwise drain every outstanding copy (vmcnt(0)) at each
// workgroup barrier. Completion is tracked by hand with wait_vm<>() below. The LDS destination is
// wave-uniform; readfirstlane pins it to an SGPR for m0; one wait state separates the m0 write from the
// LDS-DMA instruction that reads it (an SALU m0 write -> LDS DMA hazard the assembler does not resolve).
__device__ inline void dma16(const void* g, SPMLA_LDS void* l) {
  const uint32_t a = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)l);
  asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(g), "s"(a) : "memory", "m0");
}
__device__ inline void dma4(const void* g, SPMLA_LDS void* l) {
  const uint32_t a = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)l);
  asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dword %0, off" ::"v"(g), "s"(a) : "memory", "m0");
}
#pragma clang diagnostic pop

// Workgroup barrier for data exchanged through LDS only. __syncthreads() adds workgroup-scope fences whose
// lowering waits for every outstanding vector-memory operation (vmcnt(0)), which would drain the copy ring.
__device__ inline void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

// vmcnt-only wait (expcnt and lgkmcnt left at their maxima), gfx9 encoding.
template <int N>
__device__ inline void wait_vm() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

// e4m3 pairs -> bf16 / f16 pairs (exact), through the compiler builtins so that the hazard recognizer sees the
// VALU writes that feed MFMA operands. The packed result is bit-cast whole (extracting single bf16 lanes from
// the builtin's vector result miscompiles on this toolchain).
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));
__device__ inline uint32_t fp8lo_bf16x2(uint32_t w) {
  return __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w, 1.0f, false));
}
__device__ inline uint32_t fp8hi_bf16x2(uint32_t w) {
  return __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w, 1.0f, true));
}
__device__ inline uint32_t fp8lo_f16x2(uint32_t w) {
  return __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w, 1.0f, false));
}
__device__ inline uint32_t fp8hi_f16x2(uint32_t w) {
  return __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w, 1.0f, true));
}
// two fp32 -> packed fp16 / bf16, round to nearest even (v_cvt_pk_f16_f32 / v_cvt_pk_bf16_f32)
__device__ inline uint32_t pk_f16(float a, float b) {
  const f16x2_t v = {(_Float16)a, (_Float16)b};
  return __builtin_bit_cast(uint32_t, v);
}
__device__ inline uint32_t pk_bf16(float a, float b) {
  const bf16x2_t v = {(__bf16)a, (__bf16)b};
  return __builtin_bit_cast(uint32_t, v);
}

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));

struct Params {
  const uint16_t* q; long long q_st, q_sh;        // q[t][h][576] bf16 (last dim contiguous)
  const uint8_t* pool; long long R;               // Row656 rows
  const int* idx; long long idx_st; int K;        // idx[t][k]
  const int* kcount;                              // optional per-token count of leading valid entries
  int T, H, S, HGN;                               // tokens, heads, splits, head groups
  float c;                                        // sm_scale * kv_scale * log2(e)
  float kv_scale;
  uint16_t* out; long long o_st, o_sh;            // S == 1: bf16 out[t][h][512]
  float* lse; long long lse_st;                   // S == 1: lse[t][h]
  float* opart; float* lsepart;                   // fp32 partials: opart[s][t][h][512], lsepart[s][t][h]
};

// Copy instructions of one tile are spread over all waves: wave v issues j = v, v + NWAVES, ...
template <int NWAVES>
__device__ constexpr int copies_of(int v) { return (NCOPY - v + NWAVES - 1) / NWAVES; }

template <int NWAVES>
__device__ inline void issue_tile(const uint8_t* __restrict__ pool, long long R, const SPMLA_LDS int* rid,
                                  SPMLA_LDS uint8_t* tile, int wave, int lane) {
  const int row_id = rid[lane & 31];
  const bool valid = row_id >= 0 && (long long)row_id < R;
  // an invalid row copies row 0 (present: the tile loop only runs when R > 0) and is zeroed by zero_tile()
  const uint8_t* src = pool + (valid ? (long long)row_id : 0ll) * ROW656;
  const int half = lane >> 5;
#pragma unroll
  for (int j = wave; j < NCOPY; j += NWAVES) {
    if (j < 16) dma16(src + (2 * j + half) * 16, tile + T_LAT + j * 1024);
    else if (j < 20) dma16(src + ROPE_OFF + (2 * (j - 16) + half) * 16, tile + T_ROPE + (j - 16) * 1024);
    else dma4(src + SC_OFF + (2 * (j - 20) + half) * 4, tile + T_SC + (j - 20) * 256);
  }
}

template <int NWAVES>
__device__ inline void zero_tile(long long R, const SPMLA_LDS int* rid, SPMLA_LDS uint8_t* tile, int wave, int lane) {
  const int row_id = rid[lane & 31];
  if (row_id >= 0 && (long long)row_id < R) return;
#pragma unroll
  for (int j = wave; j < NCOPY; j += NWAVES) {
    if (j < 16) *(SPMLA_LDS u32x4*)(tile + T_LAT + j * 1024 + lane * 16) = u32x4{0, 0, 0, 0};
    else if (j < 20) *(SPMLA_LDS u32x4*)(tile + T_ROPE + (j - 16) * 1024 + lane * 16) = u32x4{0, 0, 0, 0};
    else *(SPMLA_LDS uint32_t*)(tile + T_SC + (j - 20) * 256 + lane * 4) = 0u;
  }
}

// Wait until this wave's copies of every tile <= `upto` have landed, given that tiles up to `issued` were issued.
// In the steady state exactly LATER tiles are issued after `upto` (LATER = NBUF - 2 * TEAMS: the ring holds the
// tiles of the current and the next step plus LATER in flight), so the wait is a compile-time vmcnt; any other
// situation (ramp-up / tail) drains all copies, which is always safe.
template <int NWAVES, int LATER>
__device__ inline void wait_tiles(int upto, int issued, int wave) {
  const int later = issued - upto;
  const int n = copies_of<NWAVES>(wave);
  if (LATER > 0 && later == LATER) {
    if (n == 6) wait_vm<6 * LATER>();
    else if (n == 5) wait_vm<5 * LATER>();
    else if (n == 3) wait_vm<3 * LATER>();
    else if (n == 2) wait_vm<2 * LATER>();
    else wait_vm<0>();
  } else {
    wait_vm<0>();
  }
}

template <int TEAMS, int NBUF>
__global__ void __launch_bounds__(256 * TEAMS, 1) attn_kernel(Params p) {
  using L = Lds<TEAMS, NBUF>;
  constexpr int NWAVES = 4 * TEAMS;
  static_assert(NBUF >= 2 * TEAMS + 1, "ring must hold the tiles in use plus one in flight");
  extern __shared__ __attribute__((aligned(16))) uint8_t smem_generic[];
  SPMLA_LDS uint8_t* lds = (SPMLA_LDS uint8_t*)smem_generic;

  const int nwork = p.T * p.S * p.HGN;
  const int f = remap_xcd(blockIdx.x, nwork);
  if (f < 0) return;
  const int hg = f % p.HGN;
  const int ts = f / p.HGN;
  const int s = ts % p.S;
  const int t = ts / p.S;

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);   // wave-uniform: scalar control flow
  const int team = wave >> 2, w = wave & 3;
  const int half = lane >> 5, l32 = lane & 31;

  // ---- row range of this split
  const int kc = ((p.K + p.S - 1) / p.S + TR - 1) / TR * TR;
  const int kb = s * kc;
  int ke = kb + kc < p.K ? kb + kc : p.K;
  if (p.kcount) { const int c = p.kcount[t]; ke = ke < c ? ke : c; }
  const int nrow = ke > kb ? ke - kb : 0;
  const int ntile = p.R > 0 ? (nrow + TR - 1) / TR : 0;     // no rows to read: o = 0, lse = -inf

  SPMLA_LDS int* sidx = (SPMLA_LDS int*)(lds + L::IDX);
  SPMLA_LDS float* s_alpha = (SPMLA_LDS float*)(lds + L::MISC) + team * 96;
  SPMLA_LDS float* s_m = s_alpha + 32;
  SPMLA_LDS float* s_l = s_alpha + 64;
  SPMLA_LDS f32x4* xS = (SPMLA_LDS f32x4*)(lds + L::S) + team * XS_UNITS;
  SPMLA_LDS f32x4* xP = (SPMLA_LDS f32x4*)(lds + L::P) + team * XP_UNITS;
  SPMLA_LDS uint8_t* tiles = lds + L::TILES;

  // ---- stage the row ids of this range (out-of-range slots read as -1)
  const int* idxrow = p.idx + (long long)t * p.idx_st + kb;
  for (int i = tid; i < ntile * TR; i += 256 * TEAMS) sidx[i] = i < nrow ? idxrow[i] : -1;

  // ---- query fragments (bf16 B operands) for latent group w and rope quarter w.
  // k-pair kp (32 dims): lane half h holds dims 128w + 32kp + 16h + 0..15; MFMA 2kp uses the first 8, 2kp+1 the
  // next 8 (the same permutation as the K operand read below).
  const int h = hg * HG + l32;
  const bool hval = h < p.H;
  const uint16_t* qh = p.q + (long long)t * p.q_st + (long long)(hval ? h : 0) * p.q_sh;
  bf16x8 qf[8];
#pragma unroll
  for (int kp = 0; kp < 4; ++kp) {
    const uint16_t* src = qh + w * QGROUP + kp * 32 + half * 16;
    const u32x4 a = hval ? *(const u32x4*)src : u32x4{0, 0, 0, 0};
    const u32x4 b = hval ? *(const u32x4*)(src + 8) : u32x4{0, 0, 0, 0};
    qf[2 * kp] = __builtin_bit_cast(bf16x8, a);
    qf[2 * kp + 1] = __builtin_bit_cast(bf16x8, b);
  }
  bf16x8 qrope;
  {
    const u32x4 v = hval ? *(const u32x4*)(qh + D_LAT + w * 16 + half * 8) : u32x4{0, 0, 0, 0};
    qrope = __builtin_bit_cast(bf16x8, v);
  }

  // Complete the query loads now, before any tile copy is in flight: an explicit s_waitcnt the compiler sees, so
  // that it does not place its own vmcnt(0) for them inside the tile loop (which would drain the copy ring).
  wait_vm<0>();

  // softmax ownership: wave w of a team owns heads 8w..8w+7; lane -> head 8w + lane/8, rows 4*(lane%8) .. +3
  const int sm_h = w * 8 + (lane >> 3);
  const int sm_rb = lane & 7;
  float m_ref = -__builtin_inff();
  float l_part = 0.f;

  f32x16 O[4];
#pragma unroll
  for (int b = 0; b < 4; ++b) O[b] = f32x16{};

  __syncthreads();                              // sidx staged (plain global loads: a fence is fine here)

  // ---- prologue: NBUF - TEAMS tiles in flight (the ring keeps TEAMS slots for the tiles being computed)
  constexpr int AHEAD = NBUF - TEAMS;
  int issued = -1;
#pragma unroll 1
  for (int j = 0; j < AHEAD && j < ntile; ++j) {
    issue_tile<NWAVES>(p.pool, p.R, sidx + j * TR, tiles + j * TILE, wave, lane);
    issued = j;
  }
  // first step's tiles
  if (ntile > 0) {
    const int upto = ntile - 1 < TEAMS - 1 ? ntile - 1 : TEAMS - 1;
    wait_tiles<NWAVES, NBUF - 2 * TEAMS>(upto, issued, wave);
    for (int j = 0; j <= upto; ++j) zero_tile<NWAVES>(p.R, sidx + j * TR, tiles + j * TILE, wave, lane);
  }
  lds_barrier();

  const int nstep = (ntile + TEAMS - 1) / TEAMS;
  float sc[16];      // scale of group w for this lane's 16 C-layout rows (8q + 4half + j)
#pragma unroll 1
  for (int st = 0; st < nstep; ++st) {
    const int it = st * TEAMS + team;            // this team's tile
    const bool act = it < ntile;
    SPMLA_LDS uint8_t* tile = tiles + (it % NBUF) * TILE;

    // ---- QK partial for latent group w and rope quarter w
    if (act) {
      f32x16 acc = f32x16{};
#pragma unroll
      for (int kp = 0; kp < 4; ++kp) {
        const int c = 8 * w + 2 * kp + half;                   // 16-byte chunk of 16 latent codes
        const u32x4 raw = *(SPMLA_LDS u32x4*)(tile + T_LAT + c * 512 + l32 * 16);
        i32x4 a0, a1;
        a0[0] = (int)fp8lo_bf16x2(raw[0]); a0[1] = (int)fp8hi_bf16x2(raw[0]);
        a0[2] = (int)fp8lo_bf16x2(raw[1]); a0[3] = (int)fp8hi_bf16x2(raw[1]);
        a1[0] = (int)fp8lo_bf16x2(raw[2]); a1[1] = (int)fp8hi_bf16x2(raw[2]);
        a1[2] = (int)fp8lo_bf16x2(raw[3]); a1[3] = (int)fp8hi_bf16x2(raw[3]);
        acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a0), qf[2 * kp], acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a1), qf[2 * kp + 1], acc, 0, 0, 0);
      }
      const u32x4 ar = *(SPMLA_LDS u32x4*)(tile + T_ROPE + (2 * w + half) * 512 + l32 * 16);
      const f32x16 accr = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, ar), qrope, f32x16{}, 0, 0, 0);
#pragma unroll
      for (int qd = 0; qd < 4; ++qd) {
        const f32x4 v = *(SPMLA_LDS f32x4*)(tile + T_SC + w * 128 + (8 * qd + 4 * half) * 4);
        sc[4 * qd + 0] = v[0]; sc[4 * qd + 1] = v[1]; sc[4 * qd + 2] = v[2]; sc[4 * qd + 3] = v[3];
      }
      // S partial -> xS[w][rb][h], rb = 2qd + half (rows 8qd + 4half .. +3)
#pragma unroll
      for (int qd = 0; qd < 4; ++qd) {
        f32x4 v;
#pragma unroll
        for (int j = 0; j < 4; ++j) v[j] = __builtin_fmaf(sc[4 * qd + j], acc[4 * qd + j], accr[4 * qd + j]);
        xS[(w * 8 + 2 * qd + half) * 33 + l32] = v;
      }
    }
    lds_barrier();   // B2: partials ready; every wave is past PV of its previous tile

    // ---- refill the ring with the tiles whose slots the previous step freed
#pragma unroll 1
    for (int jt = issued + 1; jt < ntile && jt <= st * TEAMS + NBUF - 1; ++jt) {
      issue_tile<NWAVES>(p.pool, p.R, sidx + jt * TR, tiles + (jt % NBUF) * TILE, wave, lane);
      issued = jt;
    }

    // ---- online softmax for heads 8w .. 8w+7 of this team's tile
    if (act) {
      f32x4 sum = xS[(0 * 8 + sm_rb) * 33 + sm_h];
#pragma unroll
      for (int w2 = 1; w2 < 4; ++w2) {
        const f32x4 v = xS[(w2 * 8 + sm_rb) * 33 + sm_h];
        sum[0] += v[0]; sum[1] += v[1]; sum[2] += v[2]; sum[3] += v[3];
      }
      const i32x4 rid = *(SPMLA_LDS i32x4*)(sidx + it * TR + 4 * sm_rb);
      const float c = p.c;
      float x[4];
      float tmax = -__builtin_inff();
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const bool ok = rid[j] >= 0 && (long long)rid[j] < p.R;
        x[j] = ok ? c * sum[j] : -__builtin_inff();
        tmax = fmaxf(tmax, x[j]);
      }
      tmax = fmaxf(tmax, __shfl_xor(tmax, 1, 64));
      tmax = fmaxf(tmax, __shfl_xor(tmax, 2, 64));
      tmax = fmaxf(tmax, __shfl_xor(tmax, 4, 64));
      float alpha = 1.f;
      if (tmax > m_ref + TAU) {                 // also true for the first finite tile (m_ref = -inf)
        alpha = __builtin_amdgcn_exp2f(m_ref - tmax);   // exp2(-inf) = 0
        m_ref = tmax;
      }
      f32x4 pv;
      float ps = 0.f;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        pv[j] = x[j] > -__builtin_inff() ? __builtin_amdgcn_exp2f(x[j] - m_ref) : 0.f;
        ps += pv[j];
      }
      l_part = l_part * alpha + ps;
      xP[sm_rb * 33 + sm_h] = pv;
      if ((lane & 7) == 0) s_alpha[sm_h] = alpha;
    }
    // the next step's tiles must have landed before the barrier that precedes their QK
    {
      const int nxt = (st + 2) * TEAMS - 1 < ntile - 1 ? (st + 2) * TEAMS - 1 : ntile - 1;
      if ((st + 1) * TEAMS < ntile) {
        wait_tiles<NWAVES, NBUF - 2 * TEAMS>(nxt, issued, wave);
        for (int j = (st + 1) * TEAMS; j <= nxt; ++j)
          zero_tile<NWAVES>(p.R, sidx + j * TR, tiles + (j % NBUF) * TILE, wave, lane);
      }
    }
    lds_barrier();   // B3: P and alpha published; the next step's tiles complete

    // ---- PV for output columns 128w .. 128w+127 (fp16 MFMA)
    if (act) {
      const float al = s_alpha[l32];
      if (__ballot(al != 1.f)) {
#pragma unroll
        for (int b = 0; b < 4; ++b) O[b] *= al;
      }
      f16x8 pb[2];
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) {
        const f32x4 v0 = xP[(4 * ks + half) * 33 + l32];        // rows 16ks + 4half + 0..3   (qd = 2ks)
        const f32x4 v1 = xP[(4 * ks + 2 + half) * 33 + l32];    // rows 16ks + 8 + 4half + 0..3 (qd = 2ks+1)
        const float* s0 = sc + 8 * ks;
        i32x4 o;
        o[0] = (int)pk_f16(fminf(v0[0] * s0[0], F16_MAX), fminf(v0[1] * s0[1], F16_MAX));
        o[1] = (int)pk_f16(fminf(v0[2] * s0[2], F16_MAX), fminf(v0[3] * s0[3], F16_MAX));
        o[2] = (int)pk_f16(fminf(v1[0] * s0[4], F16_MAX), fminf(v1[1] * s0[5], F16_MAX));
        o[3] = (int)pk_f16(fminf(v1[2] * s0[6], F16_MAX), fminf(v1[3] * s0[7], F16_MAX));
        pb[ks] = __builtin_bit_cast(f16x8, o);
      }
      // V^T operand via LDS transpose reads: 16-lane group g reads 8 rows x 16 columns of one chunk.
      const int g = lane >> 4, gi = (lane & 15) >> 1, gc = lane & 1;
      const int hh = g >> 1;
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) {
        const int row = 16 * ks + 4 * hh + (gi & 3) + 8 * (gi >> 2);
#pragma unroll
        for (int b = 0; b < 4; ++b) {
          const int chunk = 8 * w + 2 * b + (g & 1);
          SPMLA_LDS i32x2* addr = (SPMLA_LDS i32x2*)(tile + T_LAT + chunk * 512 + row * 16 + gc * 8);
          const i32x2 raw = __builtin_amdgcn_ds_read_tr8_b64_v2i32(addr);
          i32x4 a;
          a[0] = (int)fp8lo_f16x2((uint32_t)raw[0]); a[1] = (int)fp8hi_f16x2((uint32_t)raw[0]);
          a[2] = (int)fp8lo_f16x2((uint32_t)raw[1]); a[3] = (int)fp8hi_f16x2((uint32_t)raw[1]);
          O[b] = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a), pb[ks], O[b], 0, 0, 0);
        }
      }
    }
  }

  // ---- finalize: per-head (m, l) from the owner waves; with two teams merge team 1 into team 0 through LDS
  {
    float lt = l_part;
    lt += __shfl_xor(lt, 1, 64);
    lt += __shfl_xor(lt, 2, 64);
    lt += __shfl_xor(lt, 4, 64);
    lds_barrier();
    if ((lane & 7) == 0) { s_l[sm_h] = lt; s_m[sm_h] = m_ref; }
    lds_barrier();
  }
  float mh = s_m[l32], lh = s_l[l32];
  if (TEAMS == 2) {
    // team 1 parks its O (x its own normalizer weight) in the ring's LDS; team 0 adds it
    SPMLA_LDS float* s_m1 = (SPMLA_LDS float*)(lds + L::MISC) + 96 + 32;
    SPMLA_LDS float* s_l1 = s_m1 + 32;
    SPMLA_LDS float* s_m0 = (SPMLA_LDS float*)(lds + L::MISC) + 32;
    const float m0 = s_m0[l32], m1 = s_m1[l32];
    const float M = fmaxf(m0, m1);
    const float w0 = m0 > -__builtin_inff() ? __builtin_amdgcn_exp2f(m0 - M) : 0.f;
    const float w1 = m1 > -__builtin_inff() ? __builtin_amdgcn_exp2f(m1 - M) : 0.f;
    SPMLA_LDS f32x4* park = (SPMLA_LDS f32x4*)(lds + L::TILES);     // 4 waves x 4 blocks x 16 floats x 64 lanes
    if (team == 1) {
#pragma unroll
      for (int b = 0; b < 4; ++b)
#pragma unroll
        for (int qd = 0; qd < 4; ++qd)
          park[((w * 4 + b) * 4 + qd) * 64 + lane] =
              f32x4{O[b][4 * qd] * w1, O[b][4 * qd + 1] * w1, O[b][4 * qd + 2] * w1, O[b][4 * qd + 3] * w1};
    }
    lds_barrier();
    if (team == 1) return;
#pragma unroll
    for (int b = 0; b < 4; ++b)
#pragma unroll
      for (int qd = 0; qd < 4; ++qd) {
        const f32x4 v = park[((w * 4 + b) * 4 + qd) * 64 + lane];
#pragma unroll
        for (int j = 0; j < 4; ++j) O[b][4 * qd + j] = O[b][4 * qd + j] * w0 + v[j];
      }
    lh = s_l1[l32] * w1 + s_l[l32] * w0;
    mh = M;
  }
  const float inv = lh > 0.f ? p.kv_scale / lh : 0.f;
  if (!hval) return;
  const float lse_v = lh > 0.f ? (mh + log2f(lh)) * 0.69314718055994531f : -__builtin_inff();
  if (p.opart == nullptr) {
    uint16_t* orow = p.out + (long long)t * p.o_st + (long long)h * p.o_sh;
#pragma unroll
    for (int b = 0; b < 4; ++b) {
#pragma unroll
      for (int qd = 0; qd < 4; ++qd) {
        const int v0 = w * 128 + 32 * b + 8 * qd + 4 * half;
        const uint32_t w0 = pk_bf16(O[b][4 * qd] * inv, O[b][4 * qd + 1] * inv);
        const uint32_t w1 = pk_bf16(O[b][4 * qd + 2] * inv, O[b][4 * qd + 3] * inv);
        *(uint2*)(orow + v0) = make_uint2(w0, w1);
      }
    }
    if (w == 0 && half == 0) p.lse[(long long)t * p.lse_st + h] = lse_v;
  } else {
    float* orow = p.opart + (((long long)s * p.T + t) * p.H + h) * D_LAT;
#pragma unroll
    for (int b = 0; b < 4; ++b) {
#pragma unroll
      for (int qd = 0; qd < 4; ++qd) {
        const int v0 = w * 128 + 32 * b + 8 * qd + 4 * half;
        *(f32x4*)(orow + v0) = f32x4{O[b][4 * qd] * inv, O[b][4 * qd + 1] * inv, O[b][4 * qd + 2] * inv,
                                     O[b][4 * qd + 3] * inv};
      }
    }
    if (w == 0 && half == 0) p.lsepart[((long long)s * p.T + t) * p.H + h] = lse_v;
  }
}

// ---- LSE merge ------------------------------------------------------------------------------------------
// o = sum_i w_i o_i, w_i = exp(lse_i - L), L = ln sum_i exp(lse_i); all parts -inf -> o = 0, L = -inf.
// Reference: dotsnote/engine/arcstats_pkg/arcstats/sparse_offload.py:519-538 (split partials) and the
// merge_attn_states call of VP/model_executor/layers/attention/sparse_mla_attention.py:1091-1097 (tiers).
// One wave per (t, h); lane covers 8 consecutive output columns. Parts are fp32 or bf16.
struct MergeParams {
  const void* o; int o_bf16; long long o_ps, o_st, o_sh;   // part i of (t, h) at o + i*o_ps + t*o_st + h*o_sh
  const float* lse; long long l_ps, l_st;                   // lse[i*l_ps + t*l_st + h]
  int n, T, H;
  uint16_t* out; long long out_st, out_sh;                  // bf16
  float* out_f32;                                           // optional fp32 output (same strides)
  float* lse_out; long long lo_st;
};

__global__ void __launch_bounds__(256) merge_kernel(MergeParams p) {
  const int wv = blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (wv >= p.T * p.H) return;
  const int t = wv / p.H, h = wv % p.H;
  float M = -__builtin_inff();
  for (int i = 0; i < p.n; ++i) M = fmaxf(M, p.lse[i * p.l_ps + t * p.l_st + h]);
  float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
  float L = 0.f;
  if (M > -__builtin_inff()) {
    for (int i = 0; i < p.n; ++i) {
      const float li = p.lse[i * p.l_ps + t * p.l_st + h];
      if (!(li > -__builtin_inff())) continue;
      const float w = expf(li - M);
      L += w;
      const long long off = i * p.o_ps + t * p.o_st + h * p.o_sh + lane * 8;
      if (p.o_bf16) {
        const u32x4 v = *(const u32x4*)((const uint16_t*)p.o + off);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          acc[2 * e] += w * u2f(v[e] << 16);
          acc[2 * e + 1] += w * u2f(v[e] & 0xffff0000u);
        }
      } else {
        const f32x4 a = *(const f32x4*)((const float*)p.o + off);
        const f32x4 b = *(const f32x4*)((const float*)p.o + off + 4);
#pragma unroll
        for (int e = 0; e < 4; ++e) { acc[e] += w * a[e]; acc[4 + e] += w * b[e]; }
      }
    }
  }
  const float inv = L > 0.f ? 1.f / L : 0.f;
  const long long oo = t * p.out_st + h * p.out_sh + lane * 8;
  if (p.out) {
    u32x4 v;
#pragma unroll
    for (int e = 0; e < 4; ++e)
      v[e] = (uint32_t)f2bf_rne(acc[2 * e] * inv) | ((uint32_t)f2bf_rne(acc[2 * e + 1] * inv) << 16);
    *(u32x4*)(p.out + oo) = v;
  }
  if (p.out_f32) {
    *(f32x4*)(p.out_f32 + oo) = f32x4{acc[0] * inv, acc[1] * inv, acc[2] * inv, acc[3] * inv};
    *(f32x4*)(p.out_f32 + oo + 4) = f32x4{acc[4] * inv, acc[5] * inv, acc[6] * inv, acc[7] * inv};
  }
  if (lane == 0 && p.lse_out) p.lse_out[t * p.lo_st + h] = L > 0.f ? M + logf(L) : -__builtin_inff();
}

}  // namespace attn
}  // namespace spmla

using namespace spmla;

extern "C" {

// Workgroup shape of spmla_attn_splitk: 1 or 2 teams of 4 waves (SPMLA_ATTN_TEAMS, default 2).
int spmla_attn_teams(void) {
  static int teams = 0;
  if (!teams) {
    const char* e = getenv("SPMLA_ATTN_TEAMS");
    teams = (e && e[0] == '1') ? 1 : 2;
  }
  return teams;
}

// See include/spmla.h for the contract.
int spmla_attn_splitk(const void* q, long long q_st, long long q_sh, const void* pool, long long R,
                      const int* idx, long long idx_st, int K, const int* kcount, int T, int H, float sm_scale,
                      float kv_scale, int S, void* out, long long o_st, long long o_sh, float* lse,
                      long long lse_st, float* opart, float* lsepart, void* stream) {
  if (T < 0 || H <= 0 || K < 0 || S <= 0 || R < 0) return SPMLA_EARG;
  if (T == 0) return SPMLA_OK;
  if (!q || !idx || (R > 0 && !pool)) return SPMLA_EARG;
  const bool f32part = opart != nullptr;   // fp32 partials (any S) instead of the bf16 output (S == 1 only)
  if (f32part ? !lsepart : (S != 1 || !out || !lse)) return SPMLA_EARG;
  if (((uintptr_t)q & 15) || (q_st & 7) || (q_sh & 7)) return SPMLA_EALIGN;
  if (out && (((uintptr_t)out & 7) || (o_st & 3) || (o_sh & 3))) return SPMLA_EALIGN;
  if (((K + S - 1) / S + attn::TR - 1) / attn::TR * attn::TR > attn::KMAX) return SPMLA_ELIMIT;
  attn::Params p;
  p.q = (const uint16_t*)q; p.q_st = q_st; p.q_sh = q_sh;
  p.pool = (const uint8_t*)pool; p.R = R;
  p.idx = idx; p.idx_st = idx_st; p.K = K; p.kcount = kcount;
  p.T = T; p.H = H; p.S = S; p.HGN = (H + attn::HG - 1) / attn::HG;
  p.c = sm_scale * kv_scale * 1.4426950408889634f;
  p.kv_scale = kv_scale;
  p.out = (uint16_t*)out; p.o_st = o_st; p.o_sh = o_sh; p.lse = lse; p.lse_st = lse_st;
  p.opart = f32part ? opart : nullptr; p.lsepart = lsepart;
  const long long nwork = (long long)T * S * p.HGN;
  if (nwork > (1ll << 30)) return SPMLA_ELIMIT;
  const int grid = (int)((nwork + 7) / 8 * 8);
  const int teams = spmla_attn_teams();
  if (teams == 2) {
    constexpr int NB = 5;
    using Lt = attn::Lds<2, NB>;
    static bool attr = false;
    if (!attr) {
      hipError_t e = hipFuncSetAttribute((const void*)attn::attn_kernel<2, NB>,
                                         hipFuncAttributeMaxDynamicSharedMemorySize, Lt::TOTAL);
      if (e != hipSuccess) return (int)e;
      attr = true;
    }
    hipLaunchKernelGGL((attn::attn_kernel<2, NB>), dim3(grid), dim3(512), Lt::TOTAL, (hipStream_t)stream, p);
  } else {
    constexpr int NB = 6;
    using Lt = attn::Lds<1, NB>;
    static bool attr = false;
    if (!attr) {
      hipError_t e = hipFuncSetAttribute((const void*)attn::attn_kernel<1, NB>,
                                         hipFuncAttributeMaxDynamicSharedMemorySize, Lt::TOTAL);
      if (e != hipSuccess) return (int)e;
      attr = true;
    }
    hipLaunchKernelGGL((attn::attn_kernel<1, NB>), dim3(grid), dim3(256), Lt::TOTAL, (hipStream_t)stream, p);
  }
  return (int)hipGetLastError();
}

int spmla_lse_merge(const void* parts, int parts_bf16, long long o_ps, long long o_st, long long o_sh,
                    const float* lse, long long l_ps, long long l_st, int n, int T, int H, void* out,
                    long long out_st, long long out_sh, float* out_f32, float* lse_out, long long lo_st,
                    void* stream) {
  if (n <= 0 || T < 0 || H <= 0) return SPMLA_EARG;
  if (T == 0) return SPMLA_OK;
  if (!parts || !lse || (!out && !out_f32)) return SPMLA_EARG;
  const int eb = parts_bf16 ? 2 : 4;
  if (((uintptr_t)parts & 15) || ((o_ps * eb) & 15) || ((o_st * eb) & 15) || ((o_sh * eb) & 15))
    return SPMLA_EALIGN;
  if ((out && (((uintptr_t)out & 15) || (out_st & 7) || (out_sh & 7))) ||
      (out_f32 && (((uintptr_t)out_f32 & 15) || (out_st & 3) || (out_sh & 3))))
    return SPMLA_EALIGN;
  attn::MergeParams p;
  p.o = parts; p.o_bf16 = parts_bf16; p.o_ps = o_ps; p.o_st = o_st; p.o_sh = o_sh;
  p.lse = lse; p.l_ps = l_ps; p.l_st = l_st; p.n = n; p.T = T; p.H = H;
  p.out = (uint16_t*)out; p.out_st = out_st; p.out_sh = out_sh; p.out_f32 = out_f32;
  p.lse_out = lse_out; p.lo_st = lo_st;
  const long long waves = (long long)T * H;
  hipLaunchKernelGGL(attn::merge_kernel, dim3((unsigned)((waves + 3) / 4)), dim3(256), 0, (hipStream_t)stream, p);
  return (int)hipGetLastError();
}

}  // extern "C"
