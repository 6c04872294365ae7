// KV-cache write (quantize + pack) and indexer-key write.
//
// Row656 (per token): per 128 latent values s = max(amax / 448, 1e-12) (fp32, correctly rounded),
//   code = e4m3fn_rne(x / s); layout [512 codes | 4 x fp32 s | 64 x bf16 rope (bit copy)].
//   Closed form of the reference's per-128 FP8 activation quantizer: dotsnote/training/finetune/student.py:80-87;
//   656-byte layout: dotsnote/engine/vllm_patch/vllm/v1/hisparse/runtime.py:35-36.
// Row576 (the reference's deployed offload row, dotsnote/engine/arcstats_pkg/arcstats/sparse_offload.py:252-270):
//   code = e4m3fn_rne(clamp(x * inv_scale, -448, 448)) for the 512 latent and the 64 rope values.
// Row400 (the reference's compact e2m2b32 host row, dotsnote/engine/arcstats_pkg/arcstats/offload_rowfmt.py:81-129,
//   torch statement ref_quant / ref_pack :336-388): x = clamp(v * inv_scale, +-448); per 32 values
//   k = smallest integer with 2^k >= amax / 7 (fp32 amax / 7; zero or subnormal quotients give k = -126), y = |x| 2^-k,
//   mag = floor(4y + 0.5) for y < 1, else ((e2 + 1) << 2) + floor(y / 2^(e2 - 2) + 0.5) - 4 with e2 = [y >= 2] +
//   [y >= 4], capped at 15; the sign bit is set for x < 0 with mag > 0. Rope as in Row576.
// Index key (dotsnote/engine/arcstats_pkg/arcstats/shard_indexer.py:42-60): s = max(amax, 1e-4) / 448 (optionally
//   rounded up to a power of two, UE8M0), code = e4m3fn_rne(k / s); 132-byte row [128 codes | fp32 s].
//
// One wave per token, 4 tokens per 256-thread block; slot < 0 (padding) and slot >= R are skipped.
#include "spmla_common.h"

namespace spmla {
namespace wr {

__device__ inline float wave_max16(float v) {   // max over aligned groups of 16 lanes
  v = fmaxf(v, __shfl_xor(v, 1, 64));
  v = fmaxf(v, __shfl_xor(v, 2, 64));
  v = fmaxf(v, __shfl_xor(v, 4, 64));
  v = fmaxf(v, __shfl_xor(v, 8, 64));
  return v;
}

// e2m2 magnitude index of y = |x| 2^-k >= 0 (offload_rowfmt.py:93-101 with M = 2). The products are exact
// (powers of two), so the one rounding is the fp32 add of 0.5, as in the reference.
__device__ inline uint32_t e2m2_mag(float y) {
  if (y < 1.0f) return (uint32_t)floorf(y * 4.0f + 0.5f);       // 0 .. 4
  const int e2 = (y >= 2.0f) + (y >= 4.0f);
  const float inv_stp = u2f((uint32_t)(127 + 2 - e2) << 23);     // 2^(2 - e2)
  const uint32_t nrm = ((uint32_t)(e2 + 1) << 2) + (uint32_t)floorf(y * inv_stp + 0.5f) - 4u;
  return nrm < 15u ? nrm : 15u;
}

struct WriteParams {
  const uint16_t* kv; long long kv_st;      // kv_c_normed[n][512] bf16
  const uint16_t* pe; long long pe_st;      // k_pe[n][64] bf16
  const long long* slots; int n;
  uint8_t* cache; long long R; int bs; long long blk_stride;   // row of slot: (slot / bs) * blk_stride + (slot % bs) * row
  int fmt;                                  // 0: Row656, 1: Row576, 2: Row400
  float inv_scale;                          // Row576 / Row400
};

__global__ void __launch_bounds__(256) cache_write_kernel(WriteParams p) {
  const int tok = blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (tok >= p.n) return;
  const long long slot = p.slots[tok];
  if (slot < 0 || slot >= p.R) return;
  const int rowb = p.fmt == 0 ? ROW656 : (p.fmt == 1 ? ROW576 : ROW400);
  uint8_t* row = p.cache + (slot / p.bs) * p.blk_stride + (slot % p.bs) * rowb;
  const uint16_t* src = p.kv + (long long)tok * p.kv_st + lane * 8;
  const u32x4 raw = *(const u32x4*)src;
  float x[8];
#pragma unroll
  for (int e = 0; e < 4; ++e) { x[2 * e] = u2f(raw[e] << 16); x[2 * e + 1] = u2f(raw[e] & 0xffff0000u); }
  uint32_t lo = 0, hi = 0;
  if (p.fmt == 0) {
    float am = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) am = fmaxf(am, fabsf(x[e]));
    am = wave_max16(am);
    const float s = fmaxf(am / 448.0f, 1e-12f);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      lo |= (uint32_t)e4m3_rne(x[e] / s) << (8 * e);
      hi |= (uint32_t)e4m3_rne(x[4 + e] / s) << (8 * e);
    }
    *(uint2*)(row + lane * 8) = make_uint2(lo, hi);
    if ((lane & 15) == 0) *(float*)(row + SC_OFF + (lane >> 4) * 4) = s;
    if (lane < 16) {   // rope: 64 bf16 = 16 x 8 bytes
      const uint2 r = *(const uint2*)(p.pe + (long long)tok * p.pe_st + lane * 4);
      *(uint2*)(row + ROPE_OFF + lane * 8) = r;
    }
  } else if (p.fmt == 2) {
    // Row400: lane l holds values 8l .. 8l + 7; the 4 lanes 4b .. 4b + 3 form exponent block b
    float am = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      x[e] = fminf(fmaxf(x[e] * p.inv_scale, -448.f), 448.f);
      am = fmaxf(am, fabsf(x[e]));
    }
    am = fmaxf(am, __shfl_xor(am, 1, 64));
    am = fmaxf(am, __shfl_xor(am, 2, 64));
    const uint32_t rb = f2u(am / 7.0f);
    const int ex = (int)((rb >> 23) & 255u) - 127;
    int k = ex + ((rb & 0x7fffffu) != 0u);
    k = ex < -126 ? -126 : (k < 127 ? k : 127);
    const float inv = u2f((uint32_t)(127 - k) << 23);                // 2^-k
    uint32_t nib = 0, sgn = 0;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const uint32_t mag = e2m2_mag(fabsf(x[e]) * inv);
      nib |= mag << (4 * e);
      sgn |= (x[e] < 0.f && mag > 0u ? 1u : 0u) << e;
    }
    *(uint32_t*)(row + 4 * lane) = nib;
    row[R4_SIGN + lane] = (uint8_t)sgn;
    if ((lane & 3) == 0) row[R4_K + (lane >> 2)] = (uint8_t)(int8_t)k;
    if (lane < 16) {   // rope: 64 values -> 64 e4m3 codes, 4 per lane
      const uint2 r = *(const uint2*)(p.pe + (long long)tok * p.pe_st + lane * 4);
      const float y[4] = {u2f(r.x << 16), u2f(r.x & 0xffff0000u), u2f(r.y << 16), u2f(r.y & 0xffff0000u)};
      uint32_t c = 0;
#pragma unroll
      for (int e = 0; e < 4; ++e) c |= (uint32_t)e4m3_rne(fminf(fmaxf(y[e] * p.inv_scale, -448.f), 448.f)) << (8 * e);
      *(uint32_t*)(row + R4_ROPE + lane * 4) = c;
    }
  } else {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      lo |= (uint32_t)e4m3_rne(fminf(fmaxf(x[e] * p.inv_scale, -448.f), 448.f)) << (8 * e);
      hi |= (uint32_t)e4m3_rne(fminf(fmaxf(x[4 + e] * p.inv_scale, -448.f), 448.f)) << (8 * e);
    }
    *(uint2*)(row + lane * 8) = make_uint2(lo, hi);
    if (lane < 16) {   // rope: 64 values -> 64 codes, 4 per lane
      const uint2 r = *(const uint2*)(p.pe + (long long)tok * p.pe_st + lane * 4);
      const float y[4] = {u2f(r.x << 16), u2f(r.x & 0xffff0000u), u2f(r.y << 16), u2f(r.y & 0xffff0000u)};
      uint32_t c = 0;
#pragma unroll
      for (int e = 0; e < 4; ++e) c |= (uint32_t)e4m3_rne(fminf(fmaxf(y[e] * p.inv_scale, -448.f), 448.f)) << (8 * e);
      *(uint32_t*)(row + D_LAT + lane * 4) = c;
    }
  }
}

struct KeyParams {
  const uint16_t* k; long long k_st;       // k[n][128] bf16
  const long long* slots; int n;
  uint8_t* store; long long R_local;       // local rows
  int P, rank, rpb; long long blk_stride;  // row r at (r / rpb) * blk_stride + (r % rpb) * 132
  int ue8m0;
  int shuf;                                // vLLM's paged SHUFFLE layout (P = 1): key t of a block of rpb keys has
                                           // its 16-byte chunk c at (t / 16) * 2048 + (t % 16) * 16 + 256 c and its
                                           // scale at rpb * 128 + 4 t
};

__global__ void __launch_bounds__(256) key_write_kernel(KeyParams p) {
  const int tok = blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (tok >= p.n) return;
  const long long slot = p.slots[tok];
  if (slot < 0 || slot % p.P != p.rank) return;
  const long long r = slot / p.P;
  if (r >= p.R_local) return;
  uint8_t* blk = p.store + (r / p.rpb) * p.blk_stride;
  const int t = (int)(r % p.rpb);
  uint8_t* row = blk + t * 132;                                        // 132-byte rows
  uint8_t* code = p.shuf ? blk + (t >> 4) * 2048 + (t & 15) * 16 + (lane >> 3) * 256 + (lane & 7) * 2
                         : row + lane * 2;
  float* scale = (float*)(p.shuf ? blk + p.rpb * 128 + 4 * t : row + 128);
  const uint32_t raw = *(const uint32_t*)(p.k + (long long)tok * p.k_st + lane * 2);
  const float x0 = u2f(raw << 16), x1 = u2f(raw & 0xffff0000u);
  float am = fmaxf(fabsf(x0), fabsf(x1));
  am = wave_max16(am);
  am = fmaxf(am, __shfl_xor(am, 16, 64));
  am = fmaxf(am, __shfl_xor(am, 32, 64));
  float s = fmaxf(am, 1e-4f) / 448.0f;
  if (p.ue8m0) {   // next power of two >= s (s is positive and normal here)
    uint32_t u = f2u(s);
    if (u & 0x7fffffu) u = (u & 0xff800000u) + 0x800000u;
    s = u2f(u);
  }
  const uint32_t c = (uint32_t)e4m3_rne(x0 / s) | ((uint32_t)e4m3_rne(x1 / s) << 8);
  *(uint16_t*)code = (uint16_t)c;
  if (lane == 0) *scale = s;
}

}  // namespace wr
}  // namespace spmla

using namespace spmla;

extern "C" {

int spmla_cache_write(const void* kv_c, long long kv_st, const void* k_pe, long long pe_st, const long long* slots,
                      int n, void* cache, long long R, int block_size, long long block_stride, int fmt,
                      float kv_scale, void* stream) {
  if (n < 0 || R < 0 || fmt < 0 || fmt > 2 || block_size <= 0) return SPMLA_EARG;
  if (n == 0) return SPMLA_OK;
  if (!kv_c || !k_pe || !slots || !cache) return SPMLA_EARG;
  if (((uintptr_t)kv_c & 15) || (kv_st & 7) || ((uintptr_t)k_pe & 7) || (pe_st & 3)) return SPMLA_EALIGN;
  const int rowb = fmt == 0 ? ROW656 : (fmt == 1 ? ROW576 : ROW400);
  if (((uintptr_t)cache & 7) || (block_stride & 7) || block_stride < (long long)block_size * rowb) return SPMLA_EALIGN;
  if (fmt != 0 && !(kv_scale > 0.f)) return SPMLA_EARG;
  wr::WriteParams p;
  p.kv = (const uint16_t*)kv_c; p.kv_st = kv_st; p.pe = (const uint16_t*)k_pe; p.pe_st = pe_st;
  p.slots = slots; p.n = n; p.cache = (uint8_t*)cache; p.R = R; p.bs = block_size; p.blk_stride = block_stride;
  p.fmt = fmt; p.inv_scale = fmt != 0 ? 1.0f / kv_scale : 1.0f;
  hipLaunchKernelGGL(wr::cache_write_kernel, dim3((n + 3) / 4), dim3(256), 0, (hipStream_t)stream, p);
  return (int)hipGetLastError();
}

int spmla_index_key_write(const void* k, long long k_st, const long long* slots, int n, void* store,
                          long long R_local, int P, int rank, int rows_per_block, long long block_stride, int ue8m0,
                          void* stream) {
  if (n < 0 || P <= 0 || rank < 0 || rank >= P || rows_per_block <= 0 || R_local < 0) return SPMLA_EARG;
  if (n == 0) return SPMLA_OK;
  if (!k || !slots || !store) return SPMLA_EARG;
  if (((uintptr_t)k & 3) || (k_st & 1) || ((uintptr_t)store & 3) || (block_stride & 3) ||
      block_stride < (long long)rows_per_block * 132)
    return SPMLA_EALIGN;
  wr::KeyParams p;
  p.k = (const uint16_t*)k; p.k_st = k_st; p.slots = slots; p.n = n; p.store = (uint8_t*)store;
  p.R_local = R_local; p.P = P; p.rank = rank; p.rpb = rows_per_block; p.blk_stride = block_stride; p.ue8m0 = ue8m0;
  p.shuf = 0;
  hipLaunchKernelGGL(wr::key_write_kernel, dim3((n + 3) / 4), dim3(256), 0, (hipStream_t)stream, p);
  return (int)hipGetLastError();
}

int spmla_index_key_write_shuffle(const void* k, long long k_st, const long long* slots, int n, void* cache,
                                  long long num_blocks, int block_size, long long block_stride, int ue8m0,
                                  void* stream) {
  if (n < 0 || num_blocks < 0 || block_size <= 0 || (block_size & 15)) return SPMLA_EARG;
  if (n == 0) return SPMLA_OK;
  if (!k || !slots || !cache) return SPMLA_EARG;
  if (((uintptr_t)k & 3) || (k_st & 1) || ((uintptr_t)cache & 3) || (block_stride & 3) ||
      block_stride < (long long)block_size * 132)
    return SPMLA_EALIGN;
  wr::KeyParams p;
  p.k = (const uint16_t*)k; p.k_st = k_st; p.slots = slots; p.n = n; p.store = (uint8_t*)cache;
  p.R_local = num_blocks * block_size; p.P = 1; p.rank = 0; p.rpb = block_size; p.blk_stride = block_stride;
  p.ue8m0 = ue8m0; p.shuf = 1;
  hipLaunchKernelGGL(wr::key_write_kernel, dim3((n + 3) / 4), dim3(256), 0, (hipStream_t)stream, p);
  return (int)hipGetLastError();
}

}  // extern "C"
