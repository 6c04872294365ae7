// Head-group attention: one workgroup of 4 waves per (work item, column group of 32, split); each wave streams its
// own 32-row tiles (codes into a private LDS double buffer by direct global->LDS copies, rope straight into VGPRs)
// and keeps its own online softmax, so the waves never wait for each other inside the loop. Two instances:
//   * attn_kernel<false>, the decode kernel of spmla_attn / spmla_attn_splitk / spmla_attn_merge when a launch has
//     few tokens (spmla_attn.hip chooses): work item = token, columns = 32 of its heads;
//   * attn_kernel<true>, request-packed MTP decode (spmla_attn_packed) over the union rows of spmla_mtp_union: work
//     item = request, columns = tokens x heads; a column's softmax keeps only the rows its token selected (per-row
//     token masks, ballots). Reference: dotsnote/engine/arcstats_pkg/arcstats/csrc/offload_attn.cu:700-1153
//     (pk_attn_kernel).
//   * attn_kernel<false, true>, the same decode over Row576 rows (spmla_attn576: 512 + 64 e4m3 codes, one
//     per-tensor kv_scale): no per-group scales, so the latent MFMAs run as one chain into S (no scale combine), P'
//     is P itself in f16 for every group, and the rope codes are widened to bf16 (exact) in registers.
//
// Math (reference: dotsnote/kaggle/runtime_dataset/bench_offload_attn2.py:77-93 and
// dotsnote/engine/vllm_patch/vllm/v1/attention/ops/xpu_mla_sparse.py:77-161):
//   latent_d = e4m3(code_d) * scale[d / 128], rope bf16 (Row576: latent_d = e4m3(code_d), rope e4m3, no scales);
//   s = sm_scale * kv_scale * (q . row) (fp32);
//   p = exp2(s * log2e - m), o = kv_scale * sum p latent / sum p, lse = ln sum exp(s).
//
// gfx950 mapping (per wave): S^T (32 rows x 32 columns) on bf16 MFMA (32x32x16) with the codes converted exactly to
// bf16 and one fp32 scale combine per 128-value group; PV on f16 MFMA with P' = P * scale in fp16 and the codes read
// transposed with ds_read_b64_tr_b8; lazy rescaling (a column's reference max moves only when a tile exceeds it by
// more than TAU, so p <= 2^TAU); a power-of-two factor 2^-eps carried by P, O and l keeps P' inside f16's range for
// any row scale; the 4 waves' (m, l, O) merge through LDS at the end.
#include "spmla_common.h"
#include <stdlib.h>

namespace spmla {
namespace pk {

constexpr int HG = 32;                // heads per workgroup
constexpr int NW = 4;                 // waves per workgroup
constexpr int TR = 32;                // rows per tile
constexpr float TAU = 6.0f;

// tile layout (bytes): 32 code chunks [c][r][16] (chunk-major: each MFMA operand read is one conflict-free
// ds_read_b128, each V^T operand one ds_read_b64_tr_b8), then the row scales transposed to [g][r] fp32 (the copy
// writes them in that order: one 4-byte copy per (row, group))
constexpr int T_SCT = 32 * TR * 16;            // 16384
constexpr int TILE = T_SCT + 4 * TR * 4;       // 16896
constexpr int NBUF = 2;
// Query in LDS (shared by the 4 waves): the rope (64 dims) and latent groups 2, 3 (dims 256..511) of each head;
// latent groups 0, 1 stay in VGPRs. Row stride padded so 16-byte reads of 32 consecutive heads hit distinct banks.
constexpr int QRS = (64 + 256) * 2 + 16;       // 656
constexpr int QPIECES = (64 + 256) / 8;        // 16-byte pieces per head in LDS
constexpr int L_TILES = 0;
constexpr int L_QROPE = NW * NBUF * TILE;      // 135168
constexpr int L_ML = L_QROPE + HG * QRS;       // 156160: per wave m[32], l[32]
constexpr int L_TOTAL = L_ML + NW * 64 * 4;    // 157184
static_assert(L_TOTAL <= 160 * 1024, "LDS budget");
static_assert(8 * 4 * 64 * 16 <= NBUF * TILE, "merge staging (8 output tiles) fits a wave's tile buffers");

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

// The value of lane l ^ 32 (v_permlane32_swap: one VALU op; __shfl_xor would be an LDS round trip per tile).
__device__ inline float half_swap(float x) {
  const uint32_t u = __builtin_bit_cast(uint32_t, x);
  const auto r = __builtin_amdgcn_permlane32_swap(u, u, false, false);
  return __builtin_bit_cast(float, (__lane_id() & 32) ? r[0] : r[1]);
}

// QK MFMAs with the accumulator in VGPRs. The compiler builtin puts every MFMA result in AGPRs when the function
// uses AGPRs, which here would evict part of the PV accumulator around each QK phase; inline asm pins the QK
// accumulator (read by the scale FMAs) to VGPRs. Hazards the compiler cannot see inside asm are covered here:
// "s_nop 1" before the MFMA for VALU-written operands (2 wait states), and after the last MFMA of a chain
// 16 wait states before any VALU reads the result (8-pass XDL write -> VALU read). Back-to-back MFMAs of one
// chain have srcC == vdst exactly, which the hardware forwards.
__device__ inline f32x16 qk_first(bf16x8 a, bf16x8 b) {
  f32x16 d;
  asm("s_nop 1\n\tv_mfma_f32_32x32x16_bf16 %0, %1, %2, 0" : "=&v"(d) : "v"(a), "v"(b));
  return d;
}
__device__ inline f32x16 qk_next(bf16x8 a, bf16x8 b, f32x16 c) {
  asm("s_nop 1\n\tv_mfma_f32_32x32x16_bf16 %0, %1, %2, %0" : "+v"(c) : "v"(a), "v"(b));
  return c;
}
__device__ inline f32x16 qk_last(bf16x8 a, bf16x8 b, f32x16 c) {
  asm("s_nop 1\n\tv_mfma_f32_32x32x16_bf16 %0, %1, %2, %0\n\ts_nop 7\n\ts_nop 7" : "+v"(c) : "v"(a), "v"(b));
  return c;
}

// O *= a for the 256 AGPR accumulator values of a lane, one register at a time through one VGPR. Written as
// inline asm on the AGPRs: a plain C++ multiply makes the register allocator move the whole accumulator into
// VGPRs (and spill), although the rescale is a rare path.
__device__ inline void scale_acc(f32x16 (&O)[16], float a) {
#pragma unroll
  for (int b = 0; b < 16; ++b)
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      float tmp;
      asm volatile("v_accvgpr_read_b32 %1, %0\n\tv_mul_f32 %1, %1, %2\n\tv_accvgpr_write_b32 %0, %1"
                   : "+a"(O[b][e]), "=&v"(tmp)
                   : "v"(a));
    }
}

struct Params {
  const uint16_t* q; long long q_st, q_sh;        // q[t][h][576] bf16 (last dim contiguous)
  const uint8_t* pool; long long R;               // Row656 rows (Row576 in attn_kernel<false, true>)
  const int* idx; long long idx_st; int K;        // idx[t][k]
  const int* kcount;                              // optional per-token count of leading valid entries
  int T, H, S, HGN;                               // tokens, heads, splits, head groups
  float c;                                        // sm_scale * kv_scale * log2(e)
  float kv_scale;
  uint16_t* out; long long o_st, o_sh;            // bf16 out[t][h][512] (when opart is null)
  float* lse; long long lse_st;                   // lse[t][h]
  float* opart; float* lsepart;                   // fp32 partials: opart[s][t][h][512], lsepart[s][t][h]
  // optional prior partial merged into the bf16 output (S == 1): normalized fp32 o and natural-log lse
  const float* prior_o; long long po_st, po_sh;
  const float* prior_lse; long long pl_st;
  // request-packed MTP decode (attn_kernel<true>): work item t is a request; its rows are its union list (idx = u,
  // idx_st = nmax, kcount = union sizes) and mk[t * idx_st + i] is row i's token mask. Column c of a workgroup is
  // token t0 + (c >> (5 - tsh)) (t0 = cu[t] or t * ql) and head hg * (32 >> tsh) + c % (32 >> tsh); a column's
  // softmax keeps the rows its token selected. T = total tokens (output rows), NR = requests.
  const uint8_t* mk; const int* cu; int ql, tsh, NR;
};

// Source of invalid and padding rows: zero codes, zero scales, zero rope (their P is 0, and 0 * 0 stays 0 in PV).
__device__ __attribute__((aligned(16))) uint8_t zero_row[ROW656];

template <bool PK, bool R5 = false>
__global__ void __launch_bounds__(256, 1) attn_kernel(Params p) {
  constexpr int RB = R5 ? ROW576 : ROW656;      // row bytes
  constexpr int NRP = R5 ? 2 : 4;               // 16-byte rope pieces per lane: e4m3 (32 B) or bf16 (64 B)
  extern __shared__ __attribute__((aligned(16))) uint8_t smem_generic[];
  SPMLA_LDS uint8_t* lds = (SPMLA_LDS uint8_t*)smem_generic;

  const int nwork = (PK ? p.NR : p.T) * p.S * p.HGN;
  const int f = remap_xcd(blockIdx.x, nwork);
  if (f < 0) return;
  const int hg = f % p.HGN;
  const int ts = f / p.HGN;
  const int s = ts % p.S;
  const int t = ts / p.S;
  // columns -> (token, head): 32 heads of token t, or (packed) 2^tsh tokens of request t x (32 >> tsh) heads
  int t0 = t, ntok = 1;
  if (PK) {
    t0 = p.cu ? p.cu[t] : min(t * p.ql, p.T);
    const int t1 = p.cu ? p.cu[t + 1] : min(t0 + p.ql, p.T);
    ntok = min(max(t1 - t0, 0), min(1 << p.tsh, 6));
  }
  const int csh = PK ? 5 - p.tsh : 5;          // log2 heads per token in a workgroup
  auto col_tok = [&](int c) -> int { return PK ? t0 + (c >> csh) : t; };
  auto col_head = [&](int c) -> int { return PK ? (hg << csh) + (c & ((1 << csh) - 1)) : hg * HG + c; };
  auto col_ok = [&](int c) -> bool { return (!PK || (c >> csh) < ntok) && col_head(c) < p.H; };

  const int tid = threadIdx.x, lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);   // wave-uniform: scalar control flow
  const int half = lane >> 5, l32 = lane & 31;

  // ---- row range of this split
  const int kc = ((p.K + p.S - 1) / p.S + TR - 1) / TR * TR;
  const int kb = s * kc;
  int ke = kb + kc < p.K ? kb + kc : p.K;
  if (p.kcount) { const int c = p.kcount[t]; ke = ke < c ? ke : c; }
  const int nrow = ke > kb ? ke - kb : 0;
  const int ntile = p.R > 0 ? (nrow + TR - 1) / TR : 0;     // no rows to read: o = 0, lse = -inf

  SPMLA_LDS uint8_t* qrope = lds + L_QROPE;

  // ---- prologue, two memory round trips: (1) the row ids of this wave's first two tiles and the query parts
  // that go to LDS; (2) the first tile's copy, its rope and the latent query fragments (in flight while the query
  // staging is written). Row ids of later tiles are loaded one tile ahead, into registers.
  const int* idxrow = p.idx + (long long)t * p.idx_st + kb;
  const int h = col_head(l32);
  const bool hval = col_ok(l32);
  const uint8_t* mkrow = PK ? p.mk + (long long)t * p.idx_st + kb : nullptr;
  auto mk_raw = [&](int tile) -> uint32_t {   // token mask of this lane's row in `tile` (packed decode)
    const int i = tile * TR + l32;
    uint32_t m = 0u;
    if (PK && i < nrow) m = mkrow[i];
    return m;
  };
  auto row_raw = [&](int tile) -> int {       // index entry of this lane's row in `tile` (-1: past the end)
    const int i = tile * TR + l32;
    int x = -1;
    if (i < nrow) x = idxrow[i];
    return x;
  };
  auto row_ok = [&](int x) -> int { return (x >= 0 && (long long)x < p.R) ? x : -1; };   // -1: none / invalid
  int rcur = row_ok(row_raw(w)), rnxt = row_ok(row_raw(w + NW));
  int rnn = -1;                        // raw entry two tiles ahead: loaded in one iteration, checked in the next
  uint32_t mcur = mk_raw(w), mnxt = mk_raw(w + NW), mnn = 0u;
  {
    u32x4 qv[HG * QPIECES / 256];
#pragma unroll
    for (int k = 0; k < HG * QPIECES / 256; ++k) {          // 32 heads x 40 pieces (rope, latent groups 2, 3)
      const int i = tid + 256 * k, qh = i / QPIECES, part = i % QPIECES;
      const bool ok = col_ok(qh);
      const uint16_t* qsrc = p.q + (long long)(ok ? col_tok(qh) : 0) * p.q_st + (long long)(ok ? col_head(qh) : 0) * p.q_sh;
      const uint16_t* src = part < 8 ? qsrc + D_LAT + part * 8 : qsrc + 2 * QGROUP + (part - 8) * 8;
      qv[k] = *(const u32x4*)src & (ok ? 0xffffffffu : 0u);
    }
    wait_vm<0>();
#pragma unroll
    for (int k = 0; k < HG * QPIECES / 256; ++k) {
      const int i = tid + 256 * k;
      *(SPMLA_LDS u32x4*)(qrope + (i / QPIECES) * QRS + (i % QPIECES) * 16) = qv[k];
    }
  }
  const int ntw = ntile > w ? (ntile - w + NW - 1) / NW : 0;   // tiles w, w + 4, ...
  SPMLA_LDS uint8_t* mybuf = lds + L_TILES + w * NBUF * TILE;
  // rope of this lane's row: Row656, dims 16 ks + 8 half .. + 7 of MFMA ks (bf16); Row576, the 32 e4m3 codes of
  // dims 32 half .. 32 half + 31, MFMA ks taking dims 32 half + 8 ks .. + 7 (the query rope is read to match)
  u32x4 rp[NRP];
  auto load_rope = [&](const uint8_t* src) {
#pragma unroll
    for (int ks = 0; ks < NRP; ++ks)
      rp[ks] = R5 ? *(const u32x4*)(src + D_LAT + 32 * half + 16 * ks)
                  : *(const u32x4*)(src + ROPE_OFF + ks * 32 + half * 16);
  };
  if (ntw > 0) {
    const uint8_t* src = rcur >= 0 ? p.pool + (long long)rcur * RB : zero_row;
#pragma unroll
    for (int i = 0; i < 16; ++i) dma16(src + (2 * i + half) * 16, mybuf + i * 1024);
    if constexpr (!R5) {
      dma4(src + SC_OFF + half * 4, mybuf + T_SCT);
      dma4(src + SC_OFF + (2 + half) * 4, mybuf + T_SCT + 256);
    }
    load_rope(src);
  }
  // latent query fragments of groups 0, 1 (bf16 B operands), k-pair kp (32 dims = chunks 2kp, 2kp + 1): lane half
  // h holds the dims of chunk 2kp + h; MFMA 2kp + e uses its bytes 8e .. 8e + 7 (the K operand is read the same
  // way). They are waited for with the first tile.
  const uint16_t* qrow = p.q + (long long)(hval ? col_tok(l32) : 0) * p.q_st + (long long)(hval ? h : 0) * p.q_sh;
  bf16x8 qf[16];
  const uint32_t qmask = hval ? 0xffffffffu : 0u;       // heads past H: zero query
#pragma unroll
  for (int kp = 0; kp < 8; ++kp) {
    const uint16_t* src = qrow + (2 * kp + half) * 16;
    const u32x4 a = *(const u32x4*)src & qmask;
    const u32x4 b = *(const u32x4*)(src + 8) & qmask;
    qf[2 * kp] = __builtin_bit_cast(bf16x8, a);
    qf[2 * kp + 1] = __builtin_bit_cast(bf16x8, b);
  }
  lds_barrier();                                // query staging visible to all waves (copies stay in flight)
  wait_vm<0>();                                 // query fragments (and the first tile) landed

  const float c = p.c;
  float m_run = -__builtin_inff();     // reference max of this lane's head (log2 units)
  float l_run = 0.f;                   // sum of p over this lane's 16 rows of every tile
  bool started = false;                // wave-uniform: O holds contributions
  int eps = 0;                         // P, O and l_run carry a factor 2^-eps (f16 range of P')
  float elim = 0.f;                    // 2^(9 + eps) once eps is set

  f32x16 O[16];
#pragma unroll
  for (int b = 0; b < 16; ++b) O[b] = f32x16{};

  // per-lane V^T transpose-read address (16-lane group G reads 8 rows x 16 columns: lane 2i + c supplies row i,
  // bytes 8c .. 8c + 7; the rows follow the C-layout rows of the lane's P values)
  const int G = lane >> 4, gi = (lane & 15) >> 1, gc = lane & 1;
  const int tr_off = ((G & 1) * 32 + 8 * (gi >> 2) + 4 * (G >> 1) + (gi & 3)) * 16 + gc * 8;

#pragma unroll 1
  for (int j = 0; j < ntw; ++j) {
    wait_vm<0>();                               // tile j copied, its rope loaded
    SPMLA_LDS uint8_t* tb = mybuf + (j & 1) * TILE;
    const int tix = w + NW * j;

    // ---- first LDS reads of the tile: query rope, K group 0, the row ids of this and of the next tile
    u32x4 qr[4], kr[4];
#pragma unroll
    for (int ks = 0; ks < 4; ++ks)
      qr[ks] = *(SPMLA_LDS u32x4*)(qrope + l32 * QRS + (R5 ? 32 * half + 8 * ks : 16 * ks + 8 * half) * 2);
#pragma unroll
    for (int kq = 0; kq < 4; ++kq) kr[kq] = *(SPMLA_LDS u32x4*)(tb + (2 * kq + half) * 512 + l32 * 16);
    const bool more = j + 1 < ntw;
    // the entries loaded one iteration ago are checked only now, after the wait above: checking them where they
    // are loaded would stall every tile on a global-memory round trip
    if (j > 0) { rnxt = row_ok(rnn); mnxt = mnn; }
    rnn = j + 2 < ntw ? row_raw(tix + 2 * NW) : -1;
    if (PK) mnn = j + 2 < ntw ? mk_raw(tix + 2 * NW) : 0u;
    __builtin_amdgcn_sched_barrier(0);

    // ---- rope part of S^T (operands in VGPRs / LDS)
    f32x16 S;
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      bf16x8 a;
      if constexpr (R5) {                          // 8 e4m3 rope codes -> bf16 (exact)
        const uint32_t w0 = rp[ks >> 1][2 * (ks & 1)], w1 = rp[ks >> 1][2 * (ks & 1) + 1];
        i32x4 x;
        x[0] = (int)fp8lo_bf16x2(w0); x[1] = (int)fp8hi_bf16x2(w0);
        x[2] = (int)fp8lo_bf16x2(w1); x[3] = (int)fp8hi_bf16x2(w1);
        a = __builtin_bit_cast(bf16x8, x);
      } else {
        a = __builtin_bit_cast(bf16x8, rp[ks]);
      }
      const bf16x8 b = __builtin_bit_cast(bf16x8, qr[ks]);
      // Row576: the chain goes on through the latent groups (no scales to combine)
      S = ks == 0 ? qk_first(a, b) : ((ks == 3 && !R5) ? qk_last(a, b, S) : qk_next(a, b, S));
    }
    const unsigned vmask = (unsigned)__ballot(rcur >= 0);  // rows of the tile that exist
    // the next tile's copy is issued in four parts, one per latent group, between that group's MFMAs
    const uint8_t* nsrc = rnxt >= 0 ? p.pool + (long long)rnxt * RB : zero_row;
    SPMLA_LDS uint8_t* nbuf = mybuf + ((j + 1) & 1) * TILE;

    // ---- latent part of S^T: group g = chunks 8g .. 8g + 7; group g + 1's K is read while group g's MFMAs run
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      u32x4 kn[4];
      if (g < 3) {
#pragma unroll
        for (int kq = 0; kq < 4; ++kq) kn[kq] = *(SPMLA_LDS u32x4*)(tb + (2 * (4 * g + 4 + kq) + half) * 512 + l32 * 16);
      }
      if (more) {                                  // part g of the next tile's copy
#pragma unroll
        for (int i = 4 * g; i < 4 * g + 4; ++i) dma16(nsrc + (2 * i + half) * 16, nbuf + i * 1024);
        if (g == 3) {
          if constexpr (!R5) {
            dma4(nsrc + SC_OFF + half * 4, nbuf + T_SCT);
            dma4(nsrc + SC_OFF + (2 + half) * 4, nbuf + T_SCT + 256);
          }
          load_rope(nsrc);
        }
      }
      __builtin_amdgcn_sched_barrier(0);
      f32x16 acc;
#pragma unroll
      for (int kq = 0; kq < 4; ++kq) {
        const int kp = 4 * g + kq;
        const u32x4 raw = kr[kq];
        i32x4 a0, a1;
        a0[0] = (int)fp8lo_bf16x2(raw[0]); a0[1] = (int)fp8hi_bf16x2(raw[0]);
        a0[2] = (int)fp8lo_bf16x2(raw[1]); a0[3] = (int)fp8hi_bf16x2(raw[1]);
        a1[0] = (int)fp8lo_bf16x2(raw[2]); a1[1] = (int)fp8hi_bf16x2(raw[2]);
        a1[2] = (int)fp8lo_bf16x2(raw[3]); a1[3] = (int)fp8hi_bf16x2(raw[3]);
        bf16x8 b0, b1;
        if (g < 2) {
          b0 = qf[2 * kp];
          b1 = qf[2 * kp + 1];
        } else {                                   // dims 16 (2kp + half) + 8e of latent groups 2, 3, from LDS
          const SPMLA_LDS uint8_t* qp = qrope + l32 * QRS + 128 + ((2 * kp + half) * 16 - 2 * QGROUP) * 2;
          b0 = __builtin_bit_cast(bf16x8, *(const SPMLA_LDS u32x4*)qp);
          b1 = __builtin_bit_cast(bf16x8, *(const SPMLA_LDS u32x4*)(qp + 16));
        }
        if constexpr (R5) {
          S = qk_next(__builtin_bit_cast(bf16x8, a0), b0, S);
          S = (g == 3 && kq == 3) ? qk_last(__builtin_bit_cast(bf16x8, a1), b1, S)
                                  : qk_next(__builtin_bit_cast(bf16x8, a1), b1, S);
        } else {
          acc = kq == 0 ? qk_first(__builtin_bit_cast(bf16x8, a0), b0) : qk_next(__builtin_bit_cast(bf16x8, a0), b0, acc);
          acc = kq == 3 ? qk_last(__builtin_bit_cast(bf16x8, a1), b1, acc) : qk_next(__builtin_bit_cast(bf16x8, a1), b1, acc);
        }
      }
      if constexpr (!R5) {
#pragma unroll
        for (int qd = 0; qd < 4; ++qd) {
          const f32x4 sg = *(SPMLA_LDS f32x4*)(tb + T_SCT + (g * 32 + 8 * qd + 4 * half) * 4);
#pragma unroll
          for (int e = 0; e < 4; ++e) S[4 * qd + e] = __builtin_fmaf(acc[4 * qd + e], sg[e], S[4 * qd + e]);
        }
      }
      if (g < 3) {
#pragma unroll
        for (int q4 = 0; q4 < 4; ++q4) kr[q4] = kn[q4];
      }
    }

    // ---- PV operands of group 0 (scales, V^T codes) read while the softmax runs
    f32x4 ps[4];
    i32x2 tv[8];
    // 2 of the tile's 128 scales ([group][row]) per lane, for the range check of P' below
    f32x2 sc2 = {};
    if constexpr (!R5) {
      sc2 = *(SPMLA_LDS f32x2*)(tb + T_SCT + lane * 8);
#pragma unroll
      for (int qd = 0; qd < 4; ++qd) ps[qd] = *(SPMLA_LDS f32x4*)(tb + T_SCT + (8 * qd + 4 * half) * 4);
    }
#pragma unroll
    for (int f8 = 0; f8 < 8; ++f8)
      tv[f8] = __builtin_amdgcn_ds_read_tr8_b64_v2i32((SPMLA_LDS i32x2*)(tb + (f8 >> 1) * 1024 + (f8 & 1) * 256 + tr_off));
    __builtin_amdgcn_sched_barrier(0);

    // ---- rows that do not exist: -inf (C-layout row of value i: 8 (i / 4) + 4 half + i % 4)
    unsigned rm = vmask;                                 // rows of the tile this lane's column may use
    if (PK) {                                            // its token's rows (padding tokens: every row)
      const int ct = l32 >> csh;
      for (int jt = 0; jt < ntok; ++jt) {
        const unsigned bj = (unsigned)__ballot(rcur >= 0 && ((mcur >> jt) & 1u));
        if (ct == jt) rm = bj;
      }
    }
    const bool anymask = PK ? __ballot(rm != 0xffffffffu) != 0ull : vmask != 0xffffffffu;
    if (__builtin_expect(anymask, 0)) {                  // rare: keep it a branch, not 48 selects per tile
      asm volatile("" ::: "memory");
      const unsigned lm = rm >> (4 * half);
#pragma unroll
      for (int i = 0; i < 16; ++i)
        if (!((lm >> (8 * (i >> 2) + (i & 3))) & 1u)) S[i] = -__builtin_inff();
    }

    // ---- online softmax of this lane's head
    float mx = S[0];
#pragma unroll
    for (int i = 1; i < 16; ++i) mx = fmaxf(mx, S[i]);
    mx = fmaxf(mx, half_swap(mx)) * c;                      // c > 0; -inf stays -inf
    const bool need = mx > m_run + TAU;                      // also true for the first finite tile
    if (__ballot(need)) {
      const float mn = need ? mx : m_run;
      const float alpha = need ? (m_run > -__builtin_inff() ? __builtin_amdgcn_exp2f(m_run - mn) : 0.f) : 1.f;
      l_run *= alpha;
      if (started) scale_acc(O, alpha);
      m_run = mn;
    }
    // ---- f16 range of P' = P * scale: P carries a factor 2^-eps (O and l_run too; the merge adds eps back), so
    // that P' < 2^TAU * 2^9 = 2^15 while every row scale of the tile is below 2^(9 + eps). eps is set by the first
    // tile with a positive scale and rises (an exact power-of-two rescale of O and l_run) when a
    // later tile's largest such scale passes 2^(9 + eps) -- rare: scales sit near amax / 448 of their rows.
    if (!R5 && __ballot(fmaxf(sc2[0], sc2[1]) > elim)) {     // (a missing row's scales are the zero row's)
      float wm = fmaxf(sc2[0], sc2[1]);
#pragma unroll
      for (int o = 32; o >= 1; o >>= 1) wm = fmaxf(wm, __shfl_xor(wm, o, 64));
      wm = __builtin_bit_cast(float, __builtin_amdgcn_readfirstlane(__builtin_bit_cast(int, wm)));
      if (wm > elim) {                                   // then 2^(9 + en) > wm with en > eps (or eps unset)
        const int en = __builtin_amdgcn_frexp_expf(wm) - 9;
        const float f = __builtin_ldexpf(1.f, eps - en);
        l_run *= f;
        if (started) scale_acc(O, f);
        eps = en;
        elim = __builtin_ldexpf(1.f, 9 + eps);
      }
    }
    const float mref = (m_run > -__builtin_inff() ? m_run : 0.f) + (float)eps;
    float P[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      P[i] = __builtin_amdgcn_exp2f(__builtin_fmaf(S[i], c, -mref));   // exp2(-inf) = 0
      l_run += P[i];
    }
    started = true;

    // ---- PV: output columns of group g use P' = P * scale(row, g) (fp16). Group g + 1's scales and V^T codes are
    // read at the start of group g and its P' is formed between group g's MFMAs, so that VALU work overlaps the
    // matrix core instead of preceding each group's first MFMA.
    auto p_scaled = [&](const f32x4* sc, f16x8* pb) {
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) {
        const f32x4 s0 = sc[2 * ks], s1 = sc[2 * ks + 1];
        const float* pp = P + 8 * ks;
        i32x4 o;
        o[0] = (int)pk_f16(pp[0] * s0[0], pp[1] * s0[1]);
        o[1] = (int)pk_f16(pp[2] * s0[2], pp[3] * s0[3]);
        o[2] = (int)pk_f16(pp[4] * s1[0], pp[5] * s1[1]);
        o[3] = (int)pk_f16(pp[6] * s1[2], pp[7] * s1[3]);
        pb[ks] = __builtin_bit_cast(f16x8, o);
      }
    };
    f16x8 pb[2];
    if constexpr (R5) {                                  // P' = P (P <= 2^TAU), the same for every group
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) {
        const float* pp = P + 8 * ks;
        i32x4 o;
        o[0] = (int)pk_f16(pp[0], pp[1]); o[1] = (int)pk_f16(pp[2], pp[3]);
        o[2] = (int)pk_f16(pp[4], pp[5]); o[3] = (int)pk_f16(pp[6], pp[7]);
        pb[ks] = __builtin_bit_cast(f16x8, o);
      }
    } else {
      p_scaled(ps, pb);
    }
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      f32x4 pn[4];
      i32x2 vn[8];
      if (g < 3) {
        if constexpr (!R5) {
#pragma unroll
          for (int qd = 0; qd < 4; ++qd)
            pn[qd] = *(SPMLA_LDS f32x4*)(tb + T_SCT + ((g + 1) * 32 + 8 * qd + 4 * half) * 4);
        }
#pragma unroll
        for (int f8 = 0; f8 < 8; ++f8)
          vn[f8] = __builtin_amdgcn_ds_read_tr8_b64_v2i32(
              (SPMLA_LDS i32x2*)(tb + (4 * (g + 1) + (f8 >> 1)) * 1024 + (f8 & 1) * 256 + tr_off));
      }
      __builtin_amdgcn_sched_barrier(0);
      f16x8 pbn[2];
#pragma unroll
      for (int f8 = 0; f8 < 8; ++f8) {
        const int mt = 4 * g + (f8 >> 1), ks = f8 & 1;     // output columns 32 mt .. 32 mt + 31, rows 16 ks ..
        const i32x2 raw = tv[f8];
        i32x4 a;
        a[0] = (int)fp8lo_f16x2((uint32_t)raw[0]); a[1] = (int)fp8hi_f16x2((uint32_t)raw[0]);
        a[2] = (int)fp8lo_f16x2((uint32_t)raw[1]); a[3] = (int)fp8hi_f16x2((uint32_t)raw[1]);
        O[mt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a), pb[ks], O[mt], 0, 0, 0);
        if (!R5 && f8 == 3 && g < 3) p_scaled(pn, pbn);  // next group's P', behind four MFMAs
      }
      if (g < 3) {
        if constexpr (!R5) {
          pb[0] = pbn[0];
          pb[1] = pbn[1];
        }
#pragma unroll
        for (int f8 = 0; f8 < 8; ++f8) tv[f8] = vn[f8];
      }
    }
    rcur = rnxt;
    mcur = mnxt;
  }

  // ---- merge the 4 waves: per head M = max m_w, L = sum l_w 2^(m_w - M), O = sum O_w 2^(m_w - M) / L.
  // Two rounds of 8 output tiles (32 dims x 32 heads each): every wave stages its 8 tiles of the round, unscaled, in
  // its own tile buffers ([tile][qd][lane] f32x4, 32 KiB), which no other wave reads or copies into during the loop,
  // and wave w then reduces tiles 8r + 2w, 8r + 2w + 1 over the four waves. Round 0 is staged as soon as the wave's
  // own loop ends (its last copy landed at the top of its last tile), so only the slowest wave's staging follows
  // the barrier. (Keeping the reducing wave's own share in registers instead makes the compiler copy the whole
  // accumulator out of AGPRs at the loop exit.)
  l_run += half_swap(l_run);
  SPMLA_LDS float* s_ml = (SPMLA_LDS float*)(lds + L_ML);
  auto xo_at = [&](int v, int lb, int qd) -> SPMLA_LDS f32x4* {
    return (SPMLA_LDS f32x4*)(lds + L_TILES + v * NBUF * TILE) + (lb * 4 + qd) * 64 + lane;
  };
  auto stage = [&](int rnd) {
#pragma unroll
    for (int lb = 0; lb < 8; ++lb) {
#pragma unroll
      for (int qd = 0; qd < 4; ++qd) {
        const f32x16& o = O[8 * rnd + lb];
        *xo_at(w, lb, qd) = f32x4{o[4 * qd], o[4 * qd + 1], o[4 * qd + 2], o[4 * qd + 3]};
      }
    }
  };
  stage(0);
  // the wave's (O, l_run) are relative to 2^(m_run + eps)
  if (half == 0) { s_ml[w * 64 + l32] = m_run > -__builtin_inff() ? m_run + (float)eps : m_run; s_ml[w * 64 + 32 + l32] = l_run; }
  lds_barrier();
  // weight of wave v's partial for this lane's head: 2^(m_v - M) kv_scale / L (applied by the reducing wave, so
  // the partials go to LDS straight from the accumulator registers)
  float M = -__builtin_inff();
#pragma unroll
  for (int v = 0; v < NW; ++v) M = fmaxf(M, s_ml[v * 64 + l32]);
  float fv[NW];
  float L = 0.f;
#pragma unroll
  for (int v = 0; v < NW; ++v) {
    const float mv = s_ml[v * 64 + l32];
    fv[v] = mv > -__builtin_inff() ? __builtin_amdgcn_exp2f(mv - M) : 0.f;
    L += s_ml[v * 64 + 32 + l32] * fv[v];
  }
  float inv = L > 0.f ? p.kv_scale / L : 0.f;
  float lse_v = L > 0.f ? (M + log2f(L)) * 0.69314718055994531f : -__builtin_inff();
  // merge with a prior partial of the same (token, head): weights exp(lse_i - max) / sum, the lse of the union
  float wp = 0.f;
  if (p.prior_o) {
    const int hh = hg * HG + (lane & 31);
    const float lp = hh < p.H ? p.prior_lse[(long long)t * p.pl_st + hh] : -__builtin_inff();
    const float mf = fmaxf(lse_v, lp);
    if (mf > -__builtin_inff()) {
      const float a = expf(lse_v - mf), b = expf(lp - mf);     // exp(-inf) = 0
      const float z = a + b;
      inv *= a / z;
      wp = b / z;
      lse_v = mf + logf(z);
    }
  }
#pragma unroll
  for (int v = 0; v < NW; ++v) fv[v] *= inv;

  // output head of this lane, recomputed from the lane id (cheaper than keeping it live across the loop)
  const int oc = (int)(__builtin_amdgcn_mbcnt_hi(~0u, __builtin_amdgcn_mbcnt_lo(~0u, 0u)) & 31);
  const int ho = col_head(oc), to = col_tok(oc);
  const bool hoval = col_ok(oc);
#pragma unroll
  for (int rnd = 0; rnd < 2; ++rnd) {
    if (rnd == 1) {
      lds_barrier();                               // round 0's tiles are read
      stage(1);
      lds_barrier();
    }
#pragma unroll
    for (int bb = 0; bb < 2; ++bb) {
      const int lb = 2 * w + bb;
      const int mt = 8 * rnd + lb;
#pragma unroll
      for (int qd = 0; qd < 4; ++qd) {
        f32x4 acc = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int v = 0; v < NW; ++v) {
          const f32x4 x = *xo_at(v, lb, qd);
#pragma unroll
          for (int e = 0; e < 4; ++e) acc[e] = __builtin_fmaf(x[e], fv[v], acc[e]);
        }
        if (hoval) {
          const int col = 32 * mt + 8 * qd + 4 * half;      // C-layout rows of values 4qd .. 4qd + 3
          if (p.prior_o) {
            const f32x4 x = *(const f32x4*)(p.prior_o + (long long)t * p.po_st + (long long)ho * p.po_sh + col);
#pragma unroll
            for (int e = 0; e < 4; ++e) acc[e] = __builtin_fmaf(x[e], wp, acc[e]);
          }
          if (p.opart == nullptr) {
            uint16_t* orow = p.out + (long long)to * p.o_st + (long long)ho * p.o_sh;
            *(uint2*)(orow + col) = make_uint2(pk_bf16(acc[0], acc[1]), pk_bf16(acc[2], acc[3]));
          } else {
            float* orow = p.opart + (((long long)s * p.T + to) * p.H + ho) * D_LAT;
            *(f32x4*)(orow + col) = acc;
          }
        }
      }
    }
  }
  if (w == 0 && half == 0 && hoval) {
    if (p.opart == nullptr) p.lse[(long long)to * p.lse_st + ho] = lse_v;
    else p.lsepart[((long long)s * p.T + to) * p.H + ho] = lse_v;
  }
}

// Per-token launch of attn_kernel<false> (r576: attn_kernel<false, true> over Row576 rows): the arguments of
// spmla_attn_splitk / spmla_attn_merge / spmla_attn576, already checked by the caller (spmla_attn.hip, which chooses
// this kernel for launches with few tokens, and for every Row576 launch). Any K: row ids are read from global memory
// a tile ahead, not staged.
int launch_tokens(const void* q, long long q_st, long long q_sh, const void* pool, long long R, const int* idx,
                  long long idx_st, int K, const int* kcount, int T, int H, float sm_scale, float kv_scale, int S,
                  void* out, long long o_st, long long o_sh, float* lse, long long lse_st, float* opart,
                  float* lsepart, const float* prior_o, long long po_st, long long po_sh, const float* prior_lse,
                  long long pl_st, void* stream, bool r576) {
  Params p;
  p.q = (const uint16_t*)q; p.q_st = q_st; p.q_sh = q_sh;
  p.pool = (const uint8_t*)pool; p.R = R;
  p.idx = idx; p.idx_st = idx_st; p.K = K; p.kcount = kcount;
  p.T = T; p.H = H; p.S = S; p.HGN = (H + HG - 1) / HG;
  p.c = sm_scale * kv_scale * 1.4426950408889634f;
  p.kv_scale = kv_scale;
  p.out = (uint16_t*)out; p.o_st = o_st; p.o_sh = o_sh; p.lse = lse; p.lse_st = lse_st;
  p.opart = opart; p.lsepart = lsepart;
  p.prior_o = prior_o; p.po_st = po_st; p.po_sh = po_sh; p.prior_lse = prior_lse; p.pl_st = pl_st;
  p.mk = nullptr; p.cu = nullptr; p.ql = 1; p.tsh = 0; p.NR = T;
  const long long nwork = (long long)T * S * p.HGN;
  if (nwork > (1ll << 30)) return SPMLA_ELIMIT;
  const int grid = (int)((nwork + 7) / 8 * 8);
  if (r576) {
    static DynLds lds_attr5;
    if (const int e = lds_attr5.ensure((const void*)attn_kernel<false, true>, L_TOTAL)) return e;
    hipLaunchKernelGGL((attn_kernel<false, true>), dim3(grid), dim3(256), L_TOTAL, (hipStream_t)stream, p);
  } else {
    static DynLds lds_attr;
    if (const int e = lds_attr.ensure((const void*)attn_kernel<false>, L_TOTAL)) return e;
    hipLaunchKernelGGL(attn_kernel<false>, dim3(grid), dim3(256), L_TOTAL, (hipStream_t)stream, p);
  }
  return (int)hipGetLastError();
}

}  // namespace pk
}  // namespace spmla

using namespace spmla;

extern "C" {

int spmla_attn_packed(const void* q, long long q_st, long long q_sh, const void* pool, long long R, const int* u,
                      const unsigned char* mk, const int* cnt, int nmax, const int* cu, int ql, int nreq, int T,
                      int H, int tpg, float sm_scale, float kv_scale, int S, void* out, long long o_st,
                      long long o_sh, float* lse, long long lse_st, float* opart, float* lsepart, void* stream) {
  if (T < 0 || nreq < 0 || H <= 0 || nmax < 0 || S <= 0 || R < 0 || (!cu && ql <= 0)) return SPMLA_EARG;
  if (tpg != 1 && tpg != 2 && tpg != 4 && tpg != 8) return SPMLA_EARG;
  if (!cu && ql > 6) return SPMLA_EARG;                                // at most 6 tokens per request
  if (T == 0 || nreq == 0) return SPMLA_OK;
  if (!q || !u || !mk || !cnt || (R > 0 && !pool)) return SPMLA_EARG;
  const bool f32part = opart != nullptr;
  if (f32part ? !lsepart : (S != 1 || !out || !lse)) return SPMLA_EARG;
  if (((uintptr_t)q & 15) || (q_st & 7) || (q_sh & 7) || ((uintptr_t)pool & 15)) return SPMLA_EALIGN;
  if (out && (((uintptr_t)out & 7) || (o_st & 3) || (o_sh & 3))) return SPMLA_EALIGN;
  pk::Params p;
  p.q = (const uint16_t*)q; p.q_st = q_st; p.q_sh = q_sh;
  p.pool = (const uint8_t*)pool; p.R = R;
  p.idx = u; p.idx_st = nmax; p.K = nmax; p.kcount = cnt;
  p.T = T; p.H = H; p.S = S;
  p.tsh = tpg == 1 ? 0 : (tpg == 2 ? 1 : (tpg == 4 ? 2 : 3));
  p.HGN = (H + (pk::HG >> p.tsh) - 1) / (pk::HG >> p.tsh);
  p.c = sm_scale * kv_scale * 1.4426950408889634f;
  p.kv_scale = kv_scale;
  p.out = (uint16_t*)out; p.o_st = o_st; p.o_sh = o_sh; p.lse = lse; p.lse_st = lse_st;
  p.opart = f32part ? opart : nullptr; p.lsepart = lsepart;
  p.prior_o = nullptr; p.po_st = p.po_sh = 0; p.prior_lse = nullptr; p.pl_st = 0;
  p.mk = (const uint8_t*)mk; p.cu = cu; p.ql = ql; p.NR = nreq;
  const long long nwork = (long long)nreq * S * p.HGN;
  if (nwork > (1ll << 30)) return SPMLA_ELIMIT;
  const int grid = (int)((nwork + 7) / 8 * 8);
  static DynLds lds_attr;
  if (const int e = lds_attr.ensure((const void*)pk::attn_kernel<true>, pk::L_TOTAL)) return e;
  hipLaunchKernelGGL(pk::attn_kernel<true>, dim3(grid), dim3(256), pk::L_TOTAL, (hipStream_t)stream, p);
  return (int)hipGetLastError();
}

}  // extern "C"
