// Sparse-MLA decode / prefill attention over gathered Row656 KV rows, and the log-sum-exp merge of partials.
//
// Math (reference: dotsnote/kaggle/runtime_dataset/bench_offload_attn2.py:77-93 and
// dotsnote/engine/vllm_patch/vllm/v1/attention/ops/xpu_mla_sparse.py:77-161):
//   row r of token t = idx[t][k] (valid iff 0 <= idx < R); latent_d = e4m3(code_d) * scale[d / 128], rope bf16
//   s[h][k] = sm_scale * kv_scale * (q[h][:512] . latent + q[h][512:] . rope)           (fp32)
//   p = exp2(s * log2e - m), o[h] = kv_scale * sum_k p latent / sum_k p,  lse = ln sum_k exp(s)
//   invalid entries contribute nothing; a token with no valid entry gives o = 0 and lse = -inf.
//
// gfx950 mapping. One workgroup = (token t, group of up to 128 heads, split s of the token's rows), 4 waves, one per
// SIMD; wave w owns heads 32 w .. 32 w + 31 of the group: their query in VGPRs and their 32 x 512 fp32 output
// accumulator in AGPRs. All four waves walk the same 32-row tiles:
//   * staging: wave w copies the codes of scale group w (32 rows x 128 B), a quarter of the rows' bf16 rope and scale
//     w of all 32 rows into 3-deep LDS rings with direct global->LDS copies (global_load_lds_dwordx4), two tiles
//     ahead; entries that are invalid or past the split's end copy a file-scope zero row, so they feed exact zeros
//     into both products. A group's codes are stored chunk-major ([16-byte chunk][row]), row r at position
//     r ^ (4 ((r >> 3) & 1)), so that the row reads below are free of bank conflicts;
//   * QK: S^T (32 rows x 32 heads) with VGPR accumulators on f16 MFMA (32x32x16): each lane reads 16 codes of its row
//     (one b128 read feeds two MFMAs) and converts them exactly to f16 in registers (v_cvt_scalef32_pk_f16_fp8; every
//     e4m3 value is an f16); the query is converted to f16 once, exact in f16's normal range, as the reference's fp16
//     QK. One partial per 128-value scale group is combined with the rows' fp32 scales (a DPP operand: see
//     fmac4_dpp), so no product of a code and a scale is rounded; the rope on bf16 MFMA;
//   * V: during the QK MFMAs of tile j, wave w transposes its group of tile j + 1 with the 8-bit transposing read
//     (ds_read_b64_tr_b8: 8 rows of one dim per lane), converts it to f16 and writes the dim-major tile V^T [512 dims]
//     [32 rows in the P' operand's row order] (double-buffered), which the PV MFMAs of tile j + 1 read with full-rate
//     16-byte reads (a transposing read in the PV loop itself runs at a third of the rate). One barrier per tile;
//   * softmax: the C layout puts one head in each lane (16 rows; the other 16 in lane + 32): in-lane plus one
//     cross-half exchange, base 2, lazy rescaling (a head's reference max moves only when a tile exceeds it by more
//     than TAU, so p <= 2^TAU and O is rescaled rarely);
//   * PV: f16 MFMA, P' = P * scale(row, group) rounded to f16 (11 significant bits); a power-of-two factor 2^-eps
//     carried by P, O and l keeps P' inside f16's range for any row scale (see the softmax).
#include "spmla_common.h"

namespace spmla {
namespace attn {

constexpr int NW = 4;                 // waves per workgroup = head blocks
constexpr int HB = 32;                // heads per wave
constexpr int HGW = NW * HB;          // heads per workgroup
constexpr int TR = 32;                // rows per tile
constexpr int KMAX = 2048;            // rows per (token, split): their ids are staged in LDS
constexpr float TAU = 6.0f;
// Launches without the in-kernel split merge go to the head-group kernel (spmla_attn_hg.hip: 32 heads per
// workgroup, each wave streams its own rows, no barrier in the loop, no split merge) while they have at most this
// many (token, split, 32-head group) work items -- decode batches -- and to fwd_kernel above it (prefill chunks:
// there each row's staging and V^T conversion serve all 128 heads of a token, which pays once the launch fills the
// GPU with whole tokens). Measured at H = 128, K = 2048: T = 64 (256 items) 69-70 us against 82-84 us for
// fwd_kernel with 4 splits; T = 256 / 1024: 278 / 909 us against 251 / 796 us for fwd_kernel.
constexpr long long HG_TOKENS_MAX = 512;

// LDS map (bytes)
constexpr int STG_TILE = TR * 512;            // e4m3 codes of a tile: [group][16-byte chunk][row position]
constexpr int VT_TILE = 512 * TR * 2;         // f16 V^T [dim][4 blocks of 8 rows], block b stored at b ^ ((dim >> 1) & 3)
constexpr int RP_TILE = TR * 128;             // bf16 rope tile [32 rows][8 chunks], swizzled
constexpr int SC_TILE = 4 * TR * 4;           // fp32 scales [group][32], row order zrow (see issue_tile)
constexpr int NRING = 3;                      // depth of the staging, rope and scale rings
constexpr int L_STG = 0;
constexpr int L_VT = L_STG + NRING * STG_TILE;    // 49152: two V^T tiles
constexpr int L_RP = L_VT + 2 * VT_TILE;          // 114688
constexpr int L_SC = L_RP + NRING * RP_TILE;      // 126976
constexpr int L_QR = L_SC + NRING * SC_TILE;      // 128512: query rope, [wave][head][8 chunks] swizzled
constexpr int L_IDS = L_QR + NW * HB * 128;       // 144896: validated row ids of the split (-1: none)
constexpr int L_TOTAL = L_IDS + KMAX * 4;         // 153088
static_assert(L_TOTAL <= 160 * 1024, "LDS budget");

// Source of invalid and padding rows: zero codes, zero scales, zero rope.
__device__ __attribute__((aligned(16))) uint8_t zero_row[ROW656];

// position of row r in a staged chunk (an involution: bit 2 flipped with bit 3)
__device__ inline int spos(int r) { return r ^ (4 * ((r >> 3) & 1)); }
// rope tile and query rope: chunk c (8 values) of row r
__device__ inline int rp_off(int r, int c) { return r * 128 + 16 * (c ^ ((r >> 1) & 7)); }

// e4m3 pairs -> bf16 pairs (exact), through the compiler builtins so that the hazard recognizer sees the VALU
// writes. The packed result is bit-cast whole.
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
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
__device__ inline uint32_t pk_bf16(float a, float b) {      // v_cvt_pk_bf16_f32, round to nearest even
  const bf16x2_t v = {(__bf16)a, (__bf16)b};
  return __builtin_bit_cast(uint32_t, v);
}
__device__ inline uint32_t pk_f16(float a, float b) {       // round to nearest even
  const f16x2_t v = {(_Float16)a, (_Float16)b};
  return __builtin_bit_cast(uint32_t, v);
}
// 8 bf16 (one 16-byte chunk) times 2^k -> 8 f16: exact for |x 2^k| in [2^-14, 65504] (f16 carries 11 significant
// bits, bf16 8)
__device__ inline f16x8 bf16x8_to_f16(u32x4 r, int k) {
  f16x8 h;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    h[2 * e] = (_Float16)__builtin_ldexpf(__builtin_bit_cast(float, r[e] << 16), k);
    h[2 * e + 1] = (_Float16)__builtin_ldexpf(__builtin_bit_cast(float, r[e] & 0xffff0000u), k);
  }
  return h;
}
typedef short i16x4 __attribute__((ext_vector_type(4)));

// The value of lane l ^ 32 (v_permlane32_swap: one VALU op, no LDS round trip).
__device__ inline float half_swap(float x) {
  const uint32_t u = __builtin_bit_cast(uint32_t, x);
  const auto r = __builtin_amdgcn_permlane32_swap(u, u, false, false);
  return __builtin_bit_cast(float, (__lane_id() & 32) ? r[0] : r[1]);
}

// QK MFMAs with the accumulator in VGPRs. The compiler builtin puts every MFMA result in AGPRs when the function
// uses AGPRs, which here would evict part of the PV accumulator around each QK phase; inline asm pins the QK
// accumulator to VGPRs; the statements are volatile so that they keep their order (with the group combines pinned
// between them, at most one group partial is live). Hazards the compiler cannot see inside asm are covered here: "s_nop 1" before the MFMA for
// VALU-written operands (2 wait states), and after the last MFMA of a chain 16 wait states before any VALU reads
// the result (XDL write -> VALU read). Back-to-back MFMAs of one chain have srcC == vdst exactly (forwarded).
__device__ inline f32x16 qk_first(bf16x8 a, bf16x8 b) {
  f32x16 d;
  asm volatile("s_nop 1\n\tv_mfma_f32_32x32x16_bf16 %0, %1, %2, 0" : "=&v"(d) : "v"(a), "v"(b));
  return d;
}
__device__ inline f32x16 qk_next(bf16x8 a, bf16x8 b, f32x16 c) {
  asm volatile("s_nop 1\n\tv_mfma_f32_32x32x16_bf16 %0, %1, %2, %0" : "+v"(c) : "v"(a), "v"(b));
  return c;
}
// the same on f16 operands (latent chains)
__device__ inline f32x16 qkh_first(f16x8 a, f16x8 b) {
  f32x16 d;
  asm volatile("s_nop 1\n\tv_mfma_f32_32x32x16_f16 %0, %1, %2, 0" : "=&v"(d) : "v"(a), "v"(b));
  return d;
}
__device__ inline f32x16 qkh_next(f16x8 a, f16x8 b, f32x16 c) {
  asm volatile("s_nop 1\n\tv_mfma_f32_32x32x16_f16 %0, %1, %2, %0" : "+v"(c) : "v"(a), "v"(b));
  return c;
}
__device__ inline f32x16 qkh_last(f16x8 a, f16x8 b, f32x16 c) {
  asm volatile("s_nop 1\n\tv_mfma_f32_32x32x16_f16 %0, %1, %2, %0\n\ts_nop 7\n\ts_nop 7" : "+v"(c) : "v"(a), "v"(b));
  return c;
}

// O *= a for the 256 AGPR accumulator values of a lane, one register at a time through one VGPR (a plain C++
// multiply makes the register allocator move the whole accumulator into VGPRs; the rescale is a rare path).
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
  const uint8_t* pool; long long R;               // Row656 rows
  const int* idx; long long idx_st; int K;        // idx[t][k]
  const int* kcount;                              // optional per-token count of leading valid entries
  int T, H, S, HG;                                // tokens, heads, splits, head groups of 128
  float c;                                        // sm_scale * kv_scale * log2(e)
  float kv_scale;
  uint16_t* out; long long o_st, o_sh;            // bf16 out[t][h][512] (when opart is null)
  float* lse; long long lse_st;                   // lse[t][h]
  float* opart; float* lsepart;                   // fp32 partials: opart[s][t][h][512], lsepart[s][t][h]
  // optional prior partial merged into the bf16 output (S == 1): normalized fp32 o and natural-log lse
  const float* prior_o; long long po_st, po_sh;
  const float* prior_lse; long long pl_st;
  // split merge inside the kernel (S > 1 with the bf16 output): per (token, head group) arrival counters (zero
  // between launches), per split and head the lse and the partial's exponent, and the f16 partials in the lanes'
  // order ([split][token][head group][wave][mt][a][lane][4]); null otherwise
  int* ws_cnt; float* ws_lse; float* ws_exp; uint16_t* ws_o;
};

// Workspace of the in-kernel split merge (bytes, each part 256-byte aligned).
__host__ __device__ inline long long ws_align(long long b) { return (b + 255) / 256 * 256; }
inline long long ws_cnt_bytes(int T, int HG) { return ws_align(4ll * T * HG); }
inline long long ws_lse_bytes(int T, int HG, int S) { return ws_align(4ll * S * T * HG * HGW); }
inline long long ws_o_bytes(int T, int HG, int S) { return 2ll * S * T * HG * HGW * D_LAT; }

// Copies of tile jj for wave w: the codes of scale group w of the tile's 32 rows (copy i fills chunks 2 i and 2 i + 1:
// lane l copies chunk 2 i + l / 32 of row spos(l % 32) to position l % 32), rows 8 w .. 8 w + 7 of the rope tile (lane l
// fills stored chunk l % 8 of row 8 w + l / 8), and scale w of all 32 rows: lane l < 32 copies it for row
// zrow(l) = 8 (l % 4) + 4 (l / 16) + (l / 4) % 4 to float l of the group's 128 bytes (lanes 32 .. 63 are masked off),
// so that lane 4 hh + b of a group's floats holds rows 8 a + 4 hh + b, a = 0 .. 3, in one 16-byte slot.
// VM_TILE vector-memory instructions. x0 = id of row spos(lane & 31), x1 = id of row 8 w + lane / 8, x2 = id of row
// zrow(lane & 31) (read a step ahead, so that issuing the copies waits for nothing).
constexpr int VM_TILE = 6;
__device__ inline int zrow(int l) { return 8 * (l & 3) + 4 * ((l >> 4) & 1) + ((l >> 2) & 3); }
__device__ inline void issue_tile(const Params& p, SPMLA_LDS uint8_t* lds, int jj, int w, int lane, int x0, int x1,
                                  int x2) {
  const int hh = lane >> 5, rr = 8 * w + (lane >> 3);
  const uint8_t* src = (x0 >= 0 ? p.pool + (long long)x0 * ROW656 : zero_row) + 128 * w + 16 * hh;
  SPMLA_LDS uint8_t* stg = lds + L_STG + (jj % NRING) * STG_TILE + w * 4096;
#pragma unroll
  for (int i = 0; i < 4; ++i) dma16(src + 32 * i, stg + i * 1024);
  const uint8_t* rsrc = x1 >= 0 ? p.pool + (long long)x1 * ROW656 : zero_row;
  dma16(rsrc + ROPE_OFF + 16 * ((lane & 7) ^ ((rr >> 1) & 7)), lds + L_RP + (jj % NRING) * RP_TILE + w * 1024);
  const uint8_t* zsrc = x2 >= 0 ? p.pool + (long long)x2 * ROW656 : zero_row;
  if (lane < 32) dma4(zsrc + SC_OFF + 4 * w, lds + L_SC + (jj % NRING) * SC_TILE + w * 128);
}

// Row scales as DPP operands. z[a] of lane l = scale g of row 8 a + 4 hh + l % 4 (one 16-byte read per group); value
// i = 4 a + b of a C-layout accumulator (row 8 a + 4 hh + b) takes its scale from lane 4 (l / 4) + b of the same quad
// (quad_perm b,b,b,b), so one register per a serves the four rows of a quad. "s_nop 1": a VALU write of the DPP source needs 2 wait
// states before the DPP read (the compiler cannot see inside asm).
// s[4 A + b] += z (row of value 4 A + b) * x[4 A + b], b = 0..3
template <int A>
__device__ inline void fmac4_dpp(f32x16& s, float z, const f32x16& x) {
  asm volatile("s_nop 1\n\t"
               "v_fmac_f32_dpp %0, %4, %5 quad_perm:[0,0,0,0] row_mask:0xf bank_mask:0xf\n\t"
               "v_fmac_f32_dpp %1, %4, %6 quad_perm:[1,1,1,1] row_mask:0xf bank_mask:0xf\n\t"
               "v_fmac_f32_dpp %2, %4, %7 quad_perm:[2,2,2,2] row_mask:0xf bank_mask:0xf\n\t"
               "v_fmac_f32_dpp %3, %4, %8 quad_perm:[3,3,3,3] row_mask:0xf bank_mask:0xf"
               : "+v"(s[4 * A]), "+v"(s[4 * A + 1]), "+v"(s[4 * A + 2]), "+v"(s[4 * A + 3])
               : "v"(z), "v"(x[4 * A]), "v"(x[4 * A + 1]), "v"(x[4 * A + 2]), "v"(x[4 * A + 3]));
}
// P' of values 4 A .. 4 A + 3: (p z) with the row scales as above, as two packed f16 pairs (elements 2 (A & 1) and
// 2 (A & 1) + 1 of the operand dst)
template <int A>
__device__ inline void mul4_dpp_f16(u32x4& dst, float z, const float (&p)[16]) {
  const float p0 = p[4 * A], p1 = p[4 * A + 1], p2 = p[4 * A + 2], p3 = p[4 * A + 3];
  float t0, t1, t2, t3;
  asm volatile("s_nop 1\n\t"
               "v_mul_f32_dpp %0, %4, %5 quad_perm:[0,0,0,0] row_mask:0xf bank_mask:0xf\n\t"
               "v_mul_f32_dpp %1, %4, %6 quad_perm:[1,1,1,1] row_mask:0xf bank_mask:0xf\n\t"
               "v_mul_f32_dpp %2, %4, %7 quad_perm:[2,2,2,2] row_mask:0xf bank_mask:0xf\n\t"
               "v_mul_f32_dpp %3, %4, %8 quad_perm:[3,3,3,3] row_mask:0xf bank_mask:0xf"
               : "=&v"(t0), "=&v"(t1), "=&v"(t2), "=&v"(t3)
               : "v"(z), "v"(p0), "v"(p1), "v"(p2), "v"(p3));
  dst[2 * (A & 1)] = pk_f16(t0, t1);
  dst[2 * (A & 1) + 1] = pk_f16(t2, t3);
}

// 8 e4m3 codes (two dwords) -> 8 f16, exact
__device__ inline f16x8 codes8_f16(uint32_t a, uint32_t b) {
  return __builtin_bit_cast(f16x8, u32x4{fp8lo_f16x2(a), fp8hi_f16x2(a), fp8lo_f16x2(b), fp8hi_f16x2(b)});
}

// bf16 output of a wave's 32 heads through LDS: the C-layout values of block mt (head l32, dims 32 mt + 8 a + 4 hh +
// b in v[4 a + b]) go to the wave's region [head][512] (row stride 1040 B: heads 16 apart share banks, so a write
// costs 2 passes); then every head row leaves as 64 lanes x 16 B. Used after the last tile's barrier (the LDS is
// free); heads >= H are not written.
constexpr int OROW = 1040;
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
static_assert(NW * HB * OROW <= L_IDS, "output staging fits below the flag word");
__device__ inline void put_block(SPMLA_LDS uint8_t* reg, int lane, int mt, const float (&v)[16]) {
  const int l32 = lane & 31, hh = lane >> 5;
#pragma unroll
  for (int a = 0; a < 4; ++a)
    *(SPMLA_LDS u32x2*)(reg + l32 * OROW + (32 * mt + 8 * a + 4 * hh) * 2) =
        u32x2{pk_bf16(v[4 * a], v[4 * a + 1]), pk_bf16(v[4 * a + 2], v[4 * a + 3])};
}
__device__ inline void flush_rows(const Params& p, SPMLA_LDS uint8_t* reg, int t, int hbase, int lane) {
  const bool al16 = !(((uintptr_t)p.out | (uintptr_t)(p.o_st * 2) | (uintptr_t)(p.o_sh * 2)) & 15);
  const int nh = p.H - hbase < HB ? p.H - hbase : HB;
  uint16_t* ob = p.out + (long long)t * p.o_st + (long long)hbase * p.o_sh + 8 * lane;
  for (int r = 0; r < nh; ++r) {
    const u32x4 v = *(SPMLA_LDS u32x4*)(reg + r * OROW + 16 * lane);
    uint16_t* dst = ob + (long long)r * p.o_sh;
    if (al16) *(u32x4*)dst = v;
    else { *(uint2*)dst = make_uint2(v[0], v[1]); *(uint2*)(dst + 4) = make_uint2(v[2], v[3]); }
  }
}

// The in-kernel split merge for NS splits, run by the last split to arrive at (token t, head group hg): o = sum_u
// f[u] * partial_u with f[u] = e^(lse_u - M) kv_scale 2^exp_u / Z (the f16 partials of every split, this one's
// included), one output block at a time with the next block's loads in flight; lse = M + ln Z.
template <int NS>
__device__ inline void merge_splits(const Params& p, SPMLA_LDS uint8_t* reg, int t, int hg, int hbase, int w,
                                    int lane) {
  const int l32 = lane & 31, hh = lane >> 5;
  float lu[NS], f[NS];
  uint64_t* pu[NS];
  float lmax = -__builtin_inff();
#pragma unroll
  for (int u = 0; u < NS; ++u) {
    const long long bu = ((long long)u * p.T + t) * p.HG + hg;
    lu[u] = __builtin_bit_cast(float, __hip_atomic_load((uint32_t*)p.ws_lse + bu * HGW + w * HB + l32,
                                                        __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
    f[u] = (float)(int)__hip_atomic_load((uint32_t*)p.ws_exp + bu * HGW + w * HB + l32, __ATOMIC_RELAXED,
                                         __HIP_MEMORY_SCOPE_AGENT);
    pu[u] = (uint64_t*)(p.ws_o + (bu * NW + w) * (16 * 4 * 64 * 4)) + lane;
    lmax = fmaxf(lmax, lu[u]);
  }
  float z = 0.f;
#pragma unroll
  for (int u = 0; u < NS; ++u) {
    lu[u] = lmax > -__builtin_inff() ? expf(lu[u] - lmax) : 0.f;     // exp(-inf) = 0
    z += lu[u];
  }
  const float zi = z > 0.f ? p.kv_scale / z : 0.f;
#pragma unroll
  for (int u = 0; u < NS; ++u) f[u] = lu[u] * zi * __builtin_ldexpf(1.f, (int)f[u]);
  const int h = hbase + l32;
  if (h < p.H && hh == 0) p.lse[(long long)t * p.lse_st + h] = lmax > -__builtin_inff() ? lmax + logf(z) : lmax;
  uint64_t x[2][NS][4];
#pragma unroll
  for (int u = 0; u < NS; ++u)
#pragma unroll
    for (int a = 0; a < 4; ++a) x[0][u][a] = __hip_atomic_load(pu[u] + a * 64, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
#pragma unroll
  for (int mt = 0; mt < 16; ++mt) {
    if (mt + 1 < 16) {
#pragma unroll
      for (int u = 0; u < NS; ++u)
#pragma unroll
        for (int a = 0; a < 4; ++a)
          x[(mt + 1) & 1][u][a] =
              __hip_atomic_load(pu[u] + ((mt + 1) * 4 + a) * 64, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    float v[16];
#pragma unroll
    for (int e = 0; e < 16; ++e) v[e] = 0.f;
#pragma unroll
    for (int u = 0; u < NS; ++u)
#pragma unroll
      for (int a = 0; a < 4; ++a) {
        const f16x2_t lo = __builtin_bit_cast(f16x2_t, (uint32_t)x[mt & 1][u][a]);
        const f16x2_t hi = __builtin_bit_cast(f16x2_t, (uint32_t)(x[mt & 1][u][a] >> 32));
        v[4 * a] = __builtin_fmaf((float)lo[0], f[u], v[4 * a]);
        v[4 * a + 1] = __builtin_fmaf((float)lo[1], f[u], v[4 * a + 1]);
        v[4 * a + 2] = __builtin_fmaf((float)hi[0], f[u], v[4 * a + 2]);
        v[4 * a + 3] = __builtin_fmaf((float)hi[1], f[u], v[4 * a + 3]);
      }
    put_block(reg, lane, mt, v);
  }
  flush_rows(p, reg, t, hbase, lane);
}

__global__ void __launch_bounds__(256, 1) fwd_kernel(Params p) {
  extern __shared__ __attribute__((aligned(16))) uint8_t smem_generic[];
  SPMLA_LDS uint8_t* lds = (SPMLA_LDS uint8_t*)smem_generic;

  const int nwork = p.T * p.S * p.HG;
  const int f = remap_xcd(blockIdx.x, nwork);
  if (f < 0) return;
  const int hg = f % p.HG;
  const int ts = f / p.HG;
  const int s = ts % p.S;
  const int t = ts / p.S;

  const int tid = threadIdx.x, lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);   // wave-uniform: scalar control flow
  const int hh = lane >> 5, l32 = lane & 31;
  const int hbase = hg * HGW + w * HB;                      // first head of this wave
  const bool wact = hbase < p.H;                            // the wave has heads (uniform)
  const int h = hbase + l32;
  const bool hval = h < p.H;

  // ---- row range of this split
  const int kc = ((p.K + p.S - 1) / p.S + TR - 1) / TR * TR;
  const int kb = s * kc;
  int ke = kb + kc < p.K ? kb + kc : p.K;
  if (p.kcount) { const int cc = p.kcount[t]; ke = ke < cc ? ke : cc; }
  const int nrow = ke > kb ? ke - kb : 0;
  const int ntile = p.R > 0 ? (nrow + TR - 1) / TR : 0;     // no rows to read: o = 0, lse = -inf

  // ---- prologue: validated row ids -> LDS, query rope -> LDS, query latent -> VGPRs (B operands: lane holds head
  // l32, dims 32 (ks / 2) + 16 hh + 8 (ks % 2) .. + 7 of MFMA ks: the two MFMAs of a pair take the 16 codes of one
  // b128 read)
  const int* idxrow = p.idx + (long long)t * p.idx_st + kb;
  int xs[KMAX / 256];
#pragma unroll
  for (int k = 0; k < KMAX / 256; ++k) {
    const int i = tid + 256 * k;
    int x = -1;
    if (i < nrow) x = idxrow[i];
    xs[k] = (x >= 0 && (long long)x < p.R) ? x : -1;
  }
  const uint16_t* qrow = p.q + (long long)t * p.q_st + (long long)(hval ? h : 0) * p.q_sh;
  const uint32_t qmask = hval ? 0xffffffffu : 0u;          // heads past H: zero query
  u32x4 qraw[32];                                            // bf16, converted to f16 once the first copies are issued
#pragma unroll
  for (int ks = 0; ks < 32; ++ks) qraw[ks] = *(const u32x4*)(qrow + 32 * (ks >> 1) + 16 * hh + 8 * (ks & 1)) & qmask;
  u32x4 qrv[4];
#pragma unroll
  for (int k = 0; k < 4; ++k) {                              // rope: 32 heads x 8 chunks, 4 per lane
    const int cc = lane + 64 * k, qh = hbase + (cc >> 3);
    const bool ok = qh < p.H;
    const uint16_t* src = p.q + (long long)t * p.q_st + (long long)(ok ? qh : 0) * p.q_sh + D_LAT + 8 * (cc & 7);
    qrv[k] = *(const u32x4*)src & (ok ? 0xffffffffu : 0u);
  }
  wait_vm<0>();
  SPMLA_LDS int* ids = (SPMLA_LDS int*)(lds + L_IDS);
#pragma unroll
  for (int k = 0; k < KMAX / 256; ++k) {
    const int i = tid + 256 * k;
    if (i < ntile * TR) ids[i] = xs[k];
  }
  lds_barrier();

  // ---- copies of tiles 0 and 1
  const int r_dma0 = spos(lane & 31);                        // the row whose codes this lane copies
  const int r_dma1 = 8 * w + (lane >> 3);                    // the rope row this lane copies
  const int r_dma2 = zrow(lane & 31);                        // the row whose scale this lane copies
#pragma unroll
  for (int jj = 0; jj < 2; ++jj)
    if (jj < ntile)
      issue_tile(p, lds, jj, w, lane, ids[jj * TR + r_dma0], ids[jj * TR + r_dma1], ids[jj * TR + r_dma2]);
  // row ids of tile 2 (the first copies the loop issues)
  int nx0 = 2 < ntile ? ids[2 * TR + r_dma0] : -1, nx1 = 2 < ntile ? ids[2 * TR + r_dma1] : -1;
  int nx2 = 2 < ntile ? ids[2 * TR + r_dma2] : -1;

  // ---- query scaled per head by 2^kq, a power of two that puts its largest latent magnitude in [2^14, 2^15): the
  // latent then converts to f16 exactly wherever it matters (values below 2^-29 of the head's largest are the only
  // ones f16 cannot hold) and cannot overflow; the rope (bf16) takes the same exact factor, and the softmax the
  // inverse (ch). Magnitudes compare as the bf16 bit patterns without sign (packed 16-bit max).
  int kq;
  {
    typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));
    u16x2 mx2 = {0, 0};
#pragma unroll
    for (int ks = 0; ks < 32; ++ks)
#pragma unroll
      for (int e = 0; e < 4; ++e)
        mx2 = __builtin_elementwise_max(mx2, __builtin_bit_cast(u16x2, qraw[ks][e] & 0x7fff7fffu));
    uint32_t m = mx2[0] > mx2[1] ? mx2[0] : mx2[1];
    const uint32_t mo = __builtin_bit_cast(uint32_t, half_swap(__builtin_bit_cast(float, m)));
    m = m > mo ? m : mo;
    const int ebf = (int)(m >> 7) & 0xff;                   // bf16 exponent field of the head's largest |q|
    kq = ebf ? 141 - ebf : 0;
  }
  f16x8 qf[32];
#pragma unroll
  for (int ks = 0; ks < 32; ++ks) qf[ks] = bf16x8_to_f16(qraw[ks], kq);
  SPMLA_LDS uint8_t* qr = lds + L_QR + w * (HB * 128);      // this wave's query rope
  {
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const int cc = lane + 64 * k;
      const int kr = __shfl(kq, (cc >> 3) & 31);             // the factor of the chunk's head
      u32x4 r = qrv[k];
#pragma unroll
      for (int e = 0; e < 4; ++e)
        r[e] = pk_bf16(__builtin_ldexpf(__builtin_bit_cast(float, r[e] << 16), kr),
                       __builtin_ldexpf(__builtin_bit_cast(float, r[e] & 0xffff0000u), kr));
      *(SPMLA_LDS u32x4*)(qr + rp_off(cc >> 3, cc & 7)) = r;
    }
  }
  // QK operand of MFMA pair pp (MFMAs 2 pp, 2 pp + 1): row l32's codes of chunk 2 (pp % 4) + hh of group pp / 4 at
  // pp / 4 * 4096 + chunk * 512 + spos(l32) * 16 (eight rows per LDS cycle on eight bank groups)
  const int k_off = spos(l32) * 16 + hh * 512;
  // V^T conversion (wave w, chunk q = 0 .. 7 of its group): in 16-lane group G of the transposing read, source lane
  // 2 k + d reads codes 8 d .. 8 d + 7 of chunk q of row rho(G, k) = 16 (G / 2) + 8 (k / 4) + 4 (G % 2) + k % 4; lane
  // L then holds dim 16 q + L % 16 of the group for rows rho(G, 0 .. 7), which is block G of V^T (the row order of
  // the P' operand: k-slot e of lane half hh = row 16 ks + 8 (e / 4) + 4 hh + e % 4 for block 2 ks + hh)
  int t_off, v_dst;
  {
    const int G = lane >> 4, sl = lane & 15, k = sl >> 1, d = sl & 1;
    const int rho = 16 * (G >> 1) + 8 * (k >> 2) + 4 * (G & 1) + (k & 3);
    t_off = w * 4096 + spos(rho) * 16 + 8 * d;                       // + q * 512
    v_dst = (128 * w + sl) * 64 + 16 * (G ^ ((sl >> 1) & 3));        // + q * 1024 (dim 128 w + 16 q + sl)
  }
  // PV operand of block mt = 4 g + m4, k half ks: dim 32 mt + l32, block 2 ks + hh of V^T
  const int pv_off0 = l32 * 64 + 16 * (hh ^ ((l32 >> 1) & 3));         // + mt * 2048
  const int pv_off1 = l32 * 64 + 16 * ((2 + hh) ^ ((l32 >> 1) & 3));

  // V^T of tile 0 (this wave's group, once its copies have landed; tile 1's may stay in flight)
  if (ntile >= 2) wait_vm<VM_TILE>();
  else wait_vm<0>();
  if (ntile > 0) {
#pragma unroll
    for (int q = 0; q < 8; ++q) {
      const i32x2 tv = __builtin_amdgcn_ds_read_tr8_b64_v2i32((SPMLA_LDS i32x2*)(lds + L_STG + t_off + q * 512));
      *(SPMLA_LDS u32x4*)(lds + L_VT + v_dst + q * 1024) =
          u32x4{fp8lo_f16x2(tv[0]), fp8hi_f16x2(tv[0]), fp8lo_f16x2(tv[1]), fp8hi_f16x2(tv[1])};
    }
  }
  lds_barrier();                            // tile 0 landed for every wave, its V^T written, the query rope written


  const float ch = __builtin_ldexpf(p.c, -kq);   // sm_scale * kv_scale * log2(e) / 2^kq
  float m_run = -__builtin_inff();     // reference max of this lane's head (log2 units)
  float l_run = 0.f;                   // sum of p over this lane's 16 rows of every tile
  bool started = false;                // wave-uniform: O holds contributions
  int eps = 0;                         // P, O and l_run carry a factor 2^-eps (f16 range of P')
  float elim = 0.f;                    // 2^(9 + eps) once eps is set

  f32x16 O[16];
#pragma unroll
  for (int b = 0; b < 16; ++b) O[b] = f32x16{};

#pragma unroll 1
  for (int j = 0; j < ntile; ++j) {
    // tile j's codes, rope and scales have landed for every wave and its V^T is written (barrier at the end of the
    // previous step); the copies of tile j + 2 go out during the rope MFMAs (into tile j - 1's slots)
    SPMLA_LDS uint8_t* stg = lds + L_STG + (j % NRING) * STG_TILE;
    SPMLA_LDS uint8_t* rp = lds + L_RP + (j % NRING) * RP_TILE;
    SPMLA_LDS uint8_t* scb = lds + L_SC + (j % NRING) * SC_TILE;
    SPMLA_LDS uint8_t* vt = lds + L_VT + (j & 1) * VT_TILE;                  // V^T of tile j (PV)
    SPMLA_LDS uint8_t* vtn = lds + L_VT + ((j + 1) & 1) * VT_TILE;           // V^T of tile j + 1 (written here)
    SPMLA_LDS uint8_t* stn = lds + L_STG + ((j + 1) % NRING) * STG_TILE;     // codes of tile j + 1

    // ---- S^T of tile j: the rope chain (4 MFMAs) into S, then the latent MFMAs of groups 0 and 1 alternating (into
    // acc[0], acc[1]), then those of groups 2 and 3 (again acc[0], acc[1]): an MFMA that takes the previous one's
    // result waits for its write-back once VALU work sits between them, so consecutive MFMAs use different
    // accumulators. Each pair of groups is combined with its fp32 scales into S after its last MFMA (the accumulators
    // hold the next pair's partials from then on). With one wave per SIMD only a few VALU instructions hide behind each MFMA, so all side work is cut into
    // slices of that size, one slice per MFMA (a scheduling fence after every MFMA keeps the slices where they are):
    // the copies of tile j + 2, the code reads (4 MFMAs ahead) and their conversion (one MFMA ahead).
    // Waves without heads compute on a zero query.
    // Latent MFMA s (0 .. 31): group g = 2 (s / 16) + s % 2, k = (s / 2) % 8 (dims 128 g + 16 k .. of the group), the
    // k / 2-th code read of the group (read r = 8 (s / 16) + 2 (k / 2) + s % 2, half k % 2 of its 16 codes).
    auto kread = [&](int r) -> u32x4 {     // read r: group 2 (r / 8) + r % 2, chunk pair (r / 2) % 4
      const int g = 2 * (r >> 3) + (r & 1), pp = (r >> 1) & 3;
      return *(SPMLA_LDS u32x4*)(stg + g * 4096 + (2 * pp) * 512 + k_off);
    };
    auto rread = [&](int ks, bf16x8& ra, bf16x8& rb) {
      ra = __builtin_bit_cast(bf16x8, *(SPMLA_LDS u32x4*)(rp + rp_off(l32, 2 * ks + hh)));
      rb = __builtin_bit_cast(bf16x8, *(SPMLA_LDS u32x4*)(qr + rp_off(l32, 2 * ks + hh)));
    };
    bf16x8 ra[4], rb[4];
    rread(0, ra[0], rb[0]);
    // row scales of group g of tile j as DPP operands (see fmac4_dpp)
    auto zload = [&](int g) -> f32x4 { return *(SPMLA_LDS f32x4*)(scb + g * 128 + (4 * hh + (lane & 3)) * 16); };
    f32x4 zqa, zqb;
    float smx = 0.f;                       // largest row scale of the tile seen by this lane
    u32x4 kc[4];                           // code reads in flight (read r in kc[r % 4])
    f16x8 ka[2];                           // converted operands (MFMA parity)
    f32x16 S, acc[2];
    int idv = 0;                           // id of row l32 (the tile's valid-row mask)
    f32x4 z0;                              // scales of group 0 (the first P')
#pragma unroll
    for (int t = 0; t < 36; ++t) {
      if (t < 4) {                          // ---- rope chain
        if (t + 1 < 4) rread(t + 1, ra[t + 1], rb[t + 1]);
        if (t < 2) kc[t] = kread(t);
        if (t < 3 && j + 2 < ntile) {        // copies of tile j + 2: codes 0-1, codes 2-3, rope and scales
          // source offsets recomputed here from an opaque lane id (hoisted out of the loop they would be spilled)
          int ln = lane;
          asm volatile("" : "+v"(ln));
          if (t < 2) {
            const uint8_t* dsrc = (nx0 >= 0 ? p.pool + (long long)nx0 * ROW656 : zero_row) + 128 * w + 16 * (ln >> 5);
            SPMLA_LDS uint8_t* dst = lds + L_STG + ((j + 2) % NRING) * STG_TILE + w * 4096 + t * 2048;
            dma16(dsrc + 64 * t, dst);
            dma16(dsrc + 64 * t + 32, dst + 1024);
          } else {
            const uint8_t* rsrc = nx1 >= 0 ? p.pool + (long long)nx1 * ROW656 : zero_row;
            const int roff = ROPE_OFF + 16 * ((ln & 7) ^ (((8 * w + (ln >> 3)) >> 1) & 7));
            dma16(rsrc + roff, lds + L_RP + ((j + 2) % NRING) * RP_TILE + w * 1024);
            const uint8_t* zsrc = nx2 >= 0 ? p.pool + (long long)nx2 * ROW656 : zero_row;
            if (ln < 32) dma4(zsrc + SC_OFF + 4 * w, lds + L_SC + ((j + 2) % NRING) * SC_TILE + w * 128);
          }
        }
        if (t == 1) idv = ids[j * TR + l32];
        if (t == 3) {
          ka[0] = codes8_f16(kc[0][0], kc[0][1]);
          if (j + 2 < ntile) wait_vm<VM_TILE>();   // this wave's copies of tile j + 1 landed (tile j + 2's may not)
          else wait_vm<0>();
        }
        S = t == 0 ? qk_first(ra[0], rb[0]) : qk_next(ra[t], rb[t], S);
      } else {                              // ---- latent MFMA s
        const int sl = t - 4, half = sl >> 4, g = 2 * half + (sl & 1), k = (sl >> 1) & 7;
        // the read first used 4 MFMAs from now (reads 2 .. 15; 0 and 1 went out during the rope chain)
        if ((sl & 2) == 0) {
          const int s4 = sl + 4;
          if (s4 < 32 && ((s4 >> 1) & 1) == 0) {
            const int r = 8 * (s4 >> 4) + 2 * ((s4 >> 2) & 3) + (s4 & 1);
            kc[r & 3] = kread(r);
          }
        }
        if (sl == 12) zqa = zload(0);
        if (sl == 13) zqb = zload(1);
        if (sl == 16) {                     // groups 0 and 1 complete (qkh_last at MFMA 15): combine them into S
          smx = fmaxf(fmaxf(fmaxf(zqa[0], zqa[1]), fmaxf(zqa[2], zqa[3])),
                      fmaxf(fmaxf(zqb[0], zqb[1]), fmaxf(zqb[2], zqb[3])));
          fmac4_dpp<0>(S, zqa[0], acc[0]);
          fmac4_dpp<1>(S, zqa[1], acc[0]);
          fmac4_dpp<2>(S, zqa[2], acc[0]);
          fmac4_dpp<3>(S, zqa[3], acc[0]);
          fmac4_dpp<0>(S, zqb[0], acc[1]);
          fmac4_dpp<1>(S, zqb[1], acc[1]);
          fmac4_dpp<2>(S, zqb[2], acc[1]);
          fmac4_dpp<3>(S, zqb[3], acc[1]);
        }
        if (sl == 26) zqa = zload(2);
        if (sl == 27) zqb = zload(3);
        if (sl == 28) z0 = zload(0);
        if (sl == 29) {
          nx0 = j + 3 < ntile ? ids[(j + 3) * TR + r_dma0] : -1;   // ids of tile j + 3, used next step
          nx1 = j + 3 < ntile ? ids[(j + 3) * TR + r_dma1] : -1;
          nx2 = j + 3 < ntile ? ids[(j + 3) * TR + r_dma2] : -1;
        }
        const f16x8 kcur = ka[sl & 1];
        // the operand of MFMA s + 1
        if (sl + 1 < 32) {
          const int s1 = sl + 1, k1 = (s1 >> 1) & 7;
          const int r1 = 8 * (s1 >> 4) + 2 * (k1 >> 1) + (s1 & 1);
          const u32x4& c = kc[r1 & 3];
          ka[s1 & 1] = (k1 & 1) ? codes8_f16(c[2], c[3]) : codes8_f16(c[0], c[1]);
        }
        const f16x8 qop = qf[8 * g + k];
        if (k == 0) acc[g & 1] = qkh_first(kcur, qop);
        else if (sl == 15 || sl == 31) acc[g & 1] = qkh_last(kcur, qop, acc[g & 1]);
        else acc[g & 1] = qkh_next(kcur, qop, acc[g & 1]);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
    {                                        // combine of groups 2 and 3 (after qkh_last's wait states)
      smx = fmaxf(smx, fmaxf(fmaxf(fmaxf(zqa[0], zqa[1]), fmaxf(zqa[2], zqa[3])),
                             fmaxf(fmaxf(zqb[0], zqb[1]), fmaxf(zqb[2], zqb[3]))));
      fmac4_dpp<0>(S, zqa[0], acc[0]);
      fmac4_dpp<1>(S, zqa[1], acc[0]);
      fmac4_dpp<2>(S, zqa[2], acc[0]);
      fmac4_dpp<3>(S, zqa[3], acc[0]);
      fmac4_dpp<0>(S, zqb[0], acc[1]);
      fmac4_dpp<1>(S, zqb[1], acc[1]);
      fmac4_dpp<2>(S, zqb[2], acc[1]);
      fmac4_dpp<3>(S, zqb[3], acc[1]);
    }
    __builtin_amdgcn_sched_barrier(0);

    {
      // ---- rows that do not exist: -inf (C-layout row of value i: 8 (i / 4) + 4 hh + i % 4)
      const unsigned vmask = (unsigned)__ballot(idv >= 0);
      if (__builtin_expect(vmask != 0xffffffffu, 0)) {     // rare: keep it a branch, not 16 selects per tile
        asm volatile("" ::: "memory");
        const unsigned lm = vmask >> (4 * hh);
#pragma unroll
        for (int i = 0; i < 16; ++i)
          if (!((lm >> (8 * (i >> 2) + (i & 3))) & 1u)) S[i] = -__builtin_inff();
      }

      // ---- online softmax of this lane's head (tree reductions)
      float m8[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) m8[i] = fmaxf(S[i], S[i + 8]);
      float mx = fmaxf(fmaxf(fmaxf(m8[0], m8[4]), fmaxf(m8[1], m8[5])), fmaxf(fmaxf(m8[2], m8[6]), fmaxf(m8[3], m8[7])));
      mx = fmaxf(mx, half_swap(mx)) * ch;                      // ch > 0; -inf stays -inf
      const bool need = mx > m_run + TAU;                      // also true for the first finite tile
      if (__ballot(need)) {
        const float mn = need ? mx : m_run;
        const float alpha = need ? (m_run > -__builtin_inff() ? __builtin_amdgcn_exp2f(m_run - mn) : 0.f) : 1.f;
        l_run *= alpha;
        if (started) scale_acc(O, alpha);
        m_run = mn;
      }
      // ---- f16 range of P' = P * scale: P carries a factor 2^-eps (O and l_run too; the lse adds eps back), so that
      // P' < 2^TAU * 2^9 = 2^15 while every row scale of the tile is below 2^(9 + eps). eps is set by the first tile
      // with a positive scale and rises (exact power-of-two rescale of O and l_run) when a later tile's largest
      // scale passes 2^(9 + eps) -- rare: scales sit near amax / 448 of their rows.
      if (__ballot(smx > elim)) {
        float wm = fmaxf(smx, half_swap(smx));                // wave max (ds_swizzle xor within 32 lanes)
        wm = fmaxf(wm, __builtin_bit_cast(float, __builtin_amdgcn_ds_swizzle(__builtin_bit_cast(int, wm), 0x401F)));
        wm = fmaxf(wm, __builtin_bit_cast(float, __builtin_amdgcn_ds_swizzle(__builtin_bit_cast(int, wm), 0x201F)));
        wm = fmaxf(wm, __builtin_bit_cast(float, __builtin_amdgcn_ds_swizzle(__builtin_bit_cast(int, wm), 0x101F)));
        wm = fmaxf(wm, __builtin_bit_cast(float, __builtin_amdgcn_ds_swizzle(__builtin_bit_cast(int, wm), 0x081F)));
        wm = fmaxf(wm, __builtin_bit_cast(float, __builtin_amdgcn_ds_swizzle(__builtin_bit_cast(int, wm), 0x041F)));
        const int en = __builtin_amdgcn_readfirstlane(__builtin_amdgcn_frexp_expf(wm) - 9);   // wm * 2^-en < 2^9
        if (elim == 0.f || en > eps) {
          const float f = __builtin_ldexpf(1.f, eps - en);
          l_run *= f;
          if (started) scale_acc(O, f);
          eps = en;
          elim = __builtin_bit_cast(float, __builtin_amdgcn_readfirstlane(__builtin_bit_cast(int, __builtin_ldexpf(1.f, 9 + eps))));
        }
      }
      const float mref = (m_run > -__builtin_inff() ? m_run : 0.f) + (float)eps;
      float P[16];
#pragma unroll
      for (int i = 0; i < 16; ++i) P[i] = __builtin_amdgcn_exp2f(__builtin_fmaf(S[i], ch, -mref));  // exp2(-inf) = 0
      float s8[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) s8[i] = P[i] + P[i + 8];
      l_run += ((s8[0] + s8[4]) + (s8[1] + s8[5])) + ((s8[2] + s8[6]) + (s8[3] + s8[7]));
      started = true;

      // ---- PV: output dims of group g (MFMA blocks mt = 4g .. 4g + 3) use P' = P * scale(row, g) in f16. The V^T
      // reads run VD MFMAs ahead; group g + 1's P' is formed during group g, one quarter of its rows per MFMA (4
      // products, 2 packs), from scales read one MFMA earlier. Between them, the V^T conversion of this wave's group
      // of tile j + 1 (chunk q in MFMAs 4 q .. 4 q + 3; past the last tile it converts stale bytes into the unused
      // buffer).
      auto tread = [&](int q) -> i32x2 {
        return __builtin_amdgcn_ds_read_tr8_b64_v2i32((SPMLA_LDS i32x2*)(stn + t_off + q * 512));
      };
      i32x2 tv;                            // transposed codes of the current V^T chunk
      u32x4 tw;                            // ... converted
      constexpr int VD = 2;
      auto vread = [&](int v) -> f16x8 {          // MFMA v = (group g, k half ks, block m4): v = 8 g + 4 ks + m4
        const int mt = 4 * (v >> 3) + (v & 3);
        return __builtin_bit_cast(f16x8, *(SPMLA_LDS u32x4*)(vt + mt * 2048 + (((v >> 2) & 1) ? pv_off1 : pv_off0)));
      };
      u32x4 pbw[2], pbn[2];                  // P' of the current / next group, as packed f16 pairs
      {
        mul4_dpp_f16<0>(pbw[0], z0[0], P);
        mul4_dpp_f16<1>(pbw[0], z0[1], P);
        mul4_dpp_f16<2>(pbw[1], z0[2], P);
        mul4_dpp_f16<3>(pbw[1], z0[3], P);
      }
      f32x4 zp = zload(1);                   // scales of the P' formed during the group (group g + 1)
      f16x8 vr[4];
#pragma unroll
      for (int v = 0; v < VD; ++v) vr[v] = vread(v);
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int v = 0; v < 32; ++v) {
        const int g = v >> 3, v8 = v & 7, mt = 4 * g + (v & 3);      // consecutive MFMAs: different blocks
        if (v + VD < 32) vr[(v + VD) & 3] = vread(v + VD);
        if (g < 3) {                             // quarter v8 - 1 of group g + 1 at v8 = 1 .. 4
          if (v8 == 1) mul4_dpp_f16<0>(pbn[0], zp[0], P);
          if (v8 == 2) mul4_dpp_f16<1>(pbn[0], zp[1], P);
          if (v8 == 3) mul4_dpp_f16<2>(pbn[1], zp[2], P);
          if (v8 == 4) mul4_dpp_f16<3>(pbn[1], zp[3], P);
        }
        if (g < 2 && v8 == 6) zp = zload(g + 2);
        if ((v & 3) == 0) tv = tread(v >> 2);
        if ((v & 3) == 2) tw = u32x4{fp8lo_f16x2(tv[0]), fp8hi_f16x2(tv[0]), fp8lo_f16x2(tv[1]), fp8hi_f16x2(tv[1])};
        if ((v & 3) == 3) *(SPMLA_LDS u32x4*)(vtn + v_dst + (v >> 2) * 1024) = tw;
        O[mt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(vr[v & 3], __builtin_bit_cast(f16x8, pbw[v8 >> 2]), O[mt], 0, 0, 0);
        if (v8 == 7 && g < 3) { pbw[0] = pbn[0]; pbw[1] = pbn[1]; }
        __builtin_amdgcn_sched_barrier(0);
      }
    }
    lds_barrier();                          // tile j + 1's V^T written by every wave; tile j's slots free
  }

  // ---- epilogue: this wave's 32 heads are complete (no other wave holds them). C layout of O[mt]: lane holds head
  // l32, dims 32 mt + 8 a + 4 hh + b in value 4 a + b.
  l_run += half_swap(l_run);
  const float L = l_run;
  float lse_v = L > 0.f ? (m_run + (float)eps + log2f(L)) * 0.69314718055994531f : -__builtin_inff();
  if (p.ws_o) {                            // ---- split merge in the kernel (all waves reach the barriers)
    const long long blk = ((long long)s * p.T + t) * p.HG + hg;   // this split's partial
    if (wact) {
      // partial o / 2^(eps + 3) in f16: every row scale is <= 2^(9 + eps), so |o| < 448 * 2^(9 + eps) < 2^(18 + eps)
      const float f = L > 0.f ? __builtin_ldexpf(1.f, -(eps + 3)) / L : 0.f;
      // agent-scope stores (written through to the device's coherence point: the merging split may run on another
      // XCD, whose L2 does not see this one's) -- no L2 write-back fence needed
      uint64_t* po = (uint64_t*)(p.ws_o + (blk * NW + w) * (16 * 4 * 64 * 4)) + lane;
#pragma unroll
      for (int mt = 0; mt < 16; ++mt) {
#pragma unroll
        for (int a = 0; a < 4; ++a) {
          const uint64_t v = (uint64_t)pk_f16(O[mt][4 * a] * f, O[mt][4 * a + 1] * f) |
                             ((uint64_t)pk_f16(O[mt][4 * a + 2] * f, O[mt][4 * a + 3] * f) << 32);
          __hip_atomic_store(po + (mt * 4 + a) * 64, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        __builtin_amdgcn_sched_barrier(0);
      }
      if (hh == 0) {
        __hip_atomic_store((uint32_t*)p.ws_lse + blk * HGW + w * HB + l32, __builtin_bit_cast(uint32_t, lse_v),
                           __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_store((uint32_t*)p.ws_exp + blk * HGW + w * HB + l32, (uint32_t)(eps + 3), __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
      }
    }
    __builtin_amdgcn_s_waitcnt(0);         // every store of the partial has completed before it is counted
    __syncthreads();
    SPMLA_LDS int* flag = (SPMLA_LDS int*)(lds + L_IDS);
    if (tid == 0) {
      int* cnt = p.ws_cnt + (long long)t * p.HG + hg;
      const int old = __hip_atomic_fetch_add(cnt, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      const bool last = old == p.S - 1;
      if (last) __hip_atomic_store(cnt, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);   // ready for the next launch
      *flag = last;
    }
    __syncthreads();
    if (!*flag) return;                    // another split merges this token's heads
    if (!wact) return;                     // (the merge reads the partials with agent-scope loads)
    SPMLA_LDS uint8_t* reg = lds + w * HB * OROW;
    switch (p.S) {
      case 2: merge_splits<2>(p, reg, t, hg, hbase, w, lane); break;
      case 3: merge_splits<3>(p, reg, t, hg, hbase, w, lane); break;
      case 4: merge_splits<4>(p, reg, t, hg, hbase, w, lane); break;
      case 5: merge_splits<5>(p, reg, t, hg, hbase, w, lane); break;
      case 6: merge_splits<6>(p, reg, t, hg, hbase, w, lane); break;
      case 7: merge_splits<7>(p, reg, t, hg, hbase, w, lane); break;
      default: merge_splits<8>(p, reg, t, hg, hbase, w, lane); break;
    }
    return;
  }
  if (!wact) return;
  float inv = L > 0.f ? p.kv_scale / L : 0.f;
  float wp = 0.f;                           // weight of the prior partial (merge of two normalized partials)
  if (p.prior_o && hval) {
    const float lp = p.prior_lse[(long long)t * p.pl_st + h];
    const float mf = fmaxf(lse_v, lp);
    if (mf > -__builtin_inff()) {
      const float a = expf(lse_v - mf), b = expf(lp - mf);     // exp(-inf) = 0
      const float z = a + b;
      inv *= a / z;
      wp = b / z;
      lse_v = mf + logf(z);
    }
  }
  if (hh == 0 && hval) {
    if (p.opart) p.lsepart[((long long)s * p.T + t) * p.H + h] = lse_v;
    else p.lse[(long long)t * p.lse_st + h] = lse_v;
  }
  if (!p.opart && !p.prior_o) {            // bf16 rows through LDS (16-byte stores of whole head rows)
    SPMLA_LDS uint8_t* reg = lds + w * HB * OROW;
#pragma unroll
    for (int mt = 0; mt < 16; ++mt) {
      float v[16];
#pragma unroll
      for (int e = 0; e < 16; ++e) v[e] = O[mt][e] * inv;
      put_block(reg, lane, mt, v);
      __builtin_amdgcn_sched_barrier(0);
    }
    flush_rows(p, reg, t, hbase, lane);
    return;
  }
  if (!hval) return;
  // One block at a time (the fences keep the compiler from reading all 256 accumulators into VGPRs at once).
  const bool part = p.opart != nullptr;
  uint16_t* orow = part ? nullptr : p.out + (long long)t * p.o_st + (long long)h * p.o_sh;
  float* frow = part ? p.opart + (((long long)s * p.T + t) * p.H + h) * D_LAT : nullptr;
  const float* prow = p.prior_o ? p.prior_o + (long long)t * p.po_st + (long long)h * p.po_sh : nullptr;
#pragma unroll
  for (int mt = 0; mt < 16; ++mt) {
#pragma unroll
    for (int a = 0; a < 4; ++a) {
      const int col = 32 * mt + 8 * a + 4 * hh;
      f32x4 v = f32x4{O[mt][4 * a] * inv, O[mt][4 * a + 1] * inv, O[mt][4 * a + 2] * inv, O[mt][4 * a + 3] * inv};
      if (prow) {
        const f32x4 x = *(const f32x4*)(prow + col);
#pragma unroll
        for (int e = 0; e < 4; ++e) v[e] = __builtin_fmaf(x[e], wp, v[e]);
      }
      if (part) *(f32x4*)(frow + col) = v;
      else *(uint2*)(orow + col) = make_uint2(pk_bf16(v[0], v[1]), pk_bf16(v[2], v[3]));
    }
    __builtin_amdgcn_sched_barrier(0);
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

namespace spmla {
namespace pk {
// the head-group kernel's per-token launch (spmla_attn_hg.hip)
int launch_tokens(const void* q, long long q_st, long long q_sh, const void* pool, long long R, const int* idx,
                  long long idx_st, int K, const int* kcount, int T, int H, float sm_scale, float kv_scale, int S,
                  void* out, long long o_st, long long o_sh, float* lse, long long lse_st, float* opart,
                  float* lsepart, const float* prior_o, long long po_st, long long po_sh, const float* prior_lse,
                  long long pl_st, void* stream, bool r576);
}  // namespace pk
}  // namespace spmla

extern "C" {

static int attn_launch(const void* q, long long q_st, long long q_sh, const void* pool, long long R, const int* idx,
                       long long idx_st, int K, const int* kcount, int T, int H, float sm_scale, float kv_scale, int S,
                       void* out, long long o_st, long long o_sh, float* lse, long long lse_st, float* opart,
                       float* lsepart, const float* prior_o, long long po_st, long long po_sh, const float* prior_lse,
                       long long pl_st, void* ws, long long ws_bytes, void* stream) {
  if (T < 0 || H <= 0 || K < 0 || S <= 0 || R < 0) return SPMLA_EARG;
  if (T == 0) return SPMLA_OK;
  if (!q || !idx || (R > 0 && !pool)) return SPMLA_EARG;
  const bool f32part = opart != nullptr;   // fp32 partials (any S) instead of the bf16 output
  const bool fused = !f32part && S > 1;    // bf16 output of S splits merged in the kernel (workspace ws)
  if (f32part ? !lsepart : (!out || !lse)) return SPMLA_EARG;
  const int HG = (H + attn::HGW - 1) / attn::HGW;
  if (fused) {
    if (!ws || prior_o) return SPMLA_EARG;
    if (S > 8) return SPMLA_ELIMIT;
    if ((uintptr_t)ws & 255) return SPMLA_EALIGN;
    if (ws_bytes < attn::ws_cnt_bytes(T, HG) + 2 * attn::ws_lse_bytes(T, HG, S) + attn::ws_o_bytes(T, HG, S))
      return SPMLA_EARG;
  }
  if (((uintptr_t)q & 15) || (q_st & 7) || (q_sh & 7) || ((uintptr_t)pool & 15)) return SPMLA_EALIGN;
  if (out && (((uintptr_t)out & 7) || (o_st & 3) || (o_sh & 3))) return SPMLA_EALIGN;
  if (f32part && ((uintptr_t)opart & 15)) return SPMLA_EALIGN;
  const bool kfit = ((K + S - 1) / S + attn::TR - 1) / attn::TR * attn::TR <= attn::KMAX;
  if (!fused && (!kfit || (long long)T * S * ((H + 31) / 32) <= attn::HG_TOKENS_MAX))
    return pk::launch_tokens(q, q_st, q_sh, pool, R, idx, idx_st, K, kcount, T, H, sm_scale, kv_scale, S, out, o_st,
                             o_sh, lse, lse_st, opart, lsepart, prior_o, po_st, po_sh, prior_lse, pl_st, stream,
                             false);
  if (!kfit) return SPMLA_ELIMIT;
  attn::Params p;
  p.q = (const uint16_t*)q; p.q_st = q_st; p.q_sh = q_sh;
  p.pool = (const uint8_t*)pool; p.R = R;
  p.idx = idx; p.idx_st = idx_st; p.K = K; p.kcount = kcount;
  p.T = T; p.H = H; p.S = S; p.HG = (H + attn::HGW - 1) / attn::HGW;
  p.c = sm_scale * kv_scale * 1.4426950408889634f;
  p.kv_scale = kv_scale;
  p.out = (uint16_t*)out; p.o_st = o_st; p.o_sh = o_sh; p.lse = lse; p.lse_st = lse_st;
  p.opart = f32part ? opart : nullptr; p.lsepart = lsepart;
  p.prior_o = prior_o; p.po_st = po_st; p.po_sh = po_sh; p.prior_lse = prior_lse; p.pl_st = pl_st;
  p.ws_cnt = nullptr; p.ws_lse = nullptr; p.ws_exp = nullptr; p.ws_o = nullptr;
  if (fused) {
    uint8_t* b = (uint8_t*)ws;
    p.ws_cnt = (int*)b;
    b += attn::ws_cnt_bytes(T, HG);
    p.ws_lse = (float*)b;
    b += attn::ws_lse_bytes(T, HG, S);
    p.ws_exp = (float*)b;
    b += attn::ws_lse_bytes(T, HG, S);
    p.ws_o = (uint16_t*)b;
  }
  const long long nwork = (long long)T * S * p.HG;
  if (nwork > (1ll << 30)) return SPMLA_ELIMIT;
  const int grid = (int)((nwork + 7) / 8 * 8);
  static DynLds lds_attr;
  if (const int e = lds_attr.ensure((const void*)attn::fwd_kernel, attn::L_TOTAL)) return e;
  hipLaunchKernelGGL(attn::fwd_kernel, dim3(grid), dim3(256), attn::L_TOTAL, (hipStream_t)stream, p);
  return (int)hipGetLastError();
}

// See include/spmla.h for the contracts.
int spmla_attn_splitk(const void* q, long long q_st, long long q_sh, const void* pool, long long R,
                      const int* idx, long long idx_st, int K, const int* kcount, int T, int H, float sm_scale,
                      float kv_scale, int S, void* out, long long o_st, long long o_sh, float* lse,
                      long long lse_st, float* opart, float* lsepart, void* stream) {
  return attn_launch(q, q_st, q_sh, pool, R, idx, idx_st, K, kcount, T, H, sm_scale, kv_scale, S, out, o_st, o_sh, lse,
                     lse_st, opart, lsepart, nullptr, 0, 0, nullptr, 0, nullptr, 0, stream);
}

long long spmla_attn_ws_bytes(int T, int H, int S) {
  if (T < 0 || H <= 0 || S <= 0) return -1;
  if (S == 1) return 0;
  const int HG = (H + attn::HGW - 1) / attn::HGW;
  return attn::ws_cnt_bytes(T, HG) + 2 * attn::ws_lse_bytes(T, HG, S) + attn::ws_o_bytes(T, HG, S);
}

int spmla_attn(const void* q, long long q_st, long long q_sh, const void* pool, long long R, const int* idx,
               long long idx_st, int K, const int* kcount, int T, int H, float sm_scale, float kv_scale, int S,
               void* out, long long o_st, long long o_sh, float* lse, long long lse_st, void* ws, long long ws_bytes,
               void* stream) {
  return attn_launch(q, q_st, q_sh, pool, R, idx, idx_st, K, kcount, T, H, sm_scale, kv_scale, S, out, o_st, o_sh, lse,
                     lse_st, nullptr, nullptr, nullptr, 0, 0, nullptr, 0, S > 1 ? ws : nullptr, ws_bytes, stream);
}

int spmla_attn576(const void* q, long long q_st, long long q_sh, const void* pool, long long R, const int* idx,
                  long long idx_st, int K, const int* kcount, int T, int H, float sm_scale, float kv_scale, int S,
                  void* out, long long o_st, long long o_sh, float* lse, long long lse_st, float* opart,
                  float* lsepart, void* stream) {
  if (T < 0 || H <= 0 || K < 0 || S <= 0 || R < 0) return SPMLA_EARG;
  if (T == 0) return SPMLA_OK;
  if (!q || !idx || (R > 0 && !pool)) return SPMLA_EARG;
  const bool f32part = opart != nullptr;
  if (f32part ? !lsepart : (S != 1 || !out || !lse)) return SPMLA_EARG;
  if (((uintptr_t)q & 15) || (q_st & 7) || (q_sh & 7) || ((uintptr_t)pool & 15)) return SPMLA_EALIGN;
  if (out && (((uintptr_t)out & 7) || (o_st & 3) || (o_sh & 3))) return SPMLA_EALIGN;
  if (f32part && ((uintptr_t)opart & 15)) return SPMLA_EALIGN;
  return pk::launch_tokens(q, q_st, q_sh, pool, R, idx, idx_st, K, kcount, T, H, sm_scale, kv_scale, S, out, o_st,
                           o_sh, lse, lse_st, f32part ? opart : nullptr, lsepart, nullptr, 0, 0, nullptr, 0, stream,
                           true);
}

int spmla_attn_merge(const void* q, long long q_st, long long q_sh, const void* pool, long long R, const int* idx,
                     long long idx_st, int K, const int* kcount, int T, int H, float sm_scale, float kv_scale,
                     const float* prior_o, long long po_st, long long po_sh, const float* prior_lse, long long pl_st,
                     void* out, long long o_st, long long o_sh, float* lse, long long lse_st, void* stream) {
  if (T > 0 && (!prior_o || !prior_lse)) return SPMLA_EARG;
  if (((uintptr_t)prior_o & 15) || (po_st & 3) || (po_sh & 3)) return SPMLA_EALIGN;
  return attn_launch(q, q_st, q_sh, pool, R, idx, idx_st, K, kcount, T, H, sm_scale, kv_scale, 1, out, o_st, o_sh, lse,
                     lse_st, nullptr, nullptr, prior_o, po_st, po_sh, prior_lse, pl_st, nullptr, 0, stream);
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
