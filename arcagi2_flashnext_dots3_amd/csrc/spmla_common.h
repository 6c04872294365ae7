// Shared device helpers for the gfx950 sparse-MLA kernels: the 656-byte KV row layout, the OCP e4m3fn
// codec, bf16 bit helpers, MFMA vector types and the XCD-aware workgroup order.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <atomic>
#include <mutex>

namespace spmla {

// ---- KV row formats -------------------------------------------------------------------------------------
// Row656: [512 B e4m3fn latent codes | 4 x fp32 scale (one per 128 latent values) | 64 x bf16 rope].
// Row576: [512 B e4m3fn latent | 64 B e4m3fn rope], one per-tensor kv_scale (the reference's deployed row).
constexpr int D_LAT = 512, D_ROPE = 64, D_QK = D_LAT + D_ROPE;
constexpr int ROW656 = 656, SC_OFF = 512, ROPE_OFF = 528;
constexpr int ROW576 = 576;
constexpr int QGROUP = 128;           // latent values per fp32 scale

// ---- vector types ---------------------------------------------------------------------------------------
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef int i32x8 __attribute__((ext_vector_type(8)));
typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef int i32x2 __attribute__((ext_vector_type(2)));
typedef unsigned u32x4 __attribute__((ext_vector_type(4)));

#define SPMLA_LDS __attribute__((address_space(3)))

// ---- bit helpers ----------------------------------------------------------------------------------------
__host__ __device__ inline uint32_t f2u(float f) { return __builtin_bit_cast(uint32_t, f); }
__host__ __device__ inline float u2f(uint32_t u) { return __builtin_bit_cast(float, u); }
__host__ __device__ inline float bf2f(uint16_t b) { return u2f((uint32_t)b << 16); }

// fp32 -> bf16, round to nearest even (NaN kept quiet).
__host__ __device__ inline uint16_t f2bf_rne(float f) {
  const uint32_t u = f2u(f);
  const uint32_t r = (u + 0x7fffu + ((u >> 16) & 1u)) >> 16;
  return (uint16_t)(((u & 0x7fffffffu) > 0x7f800000u) ? ((u >> 16) | 0x40u) : r);   // a select, not a branch
}

// OCP e4m3fn encoder, round to nearest even, from the format definition: bias 7, 3 mantissa bits,
// subnormals m * 2^-9, largest finite 448 (0x7e), 0x7f = NaN, no infinities. Values whose rounded
// magnitude does not fit (>= 464 rounds past 448) and inf/NaN inputs give NaN (0x7f | sign).
__host__ __device__ inline uint8_t e4m3_rne(float f) {
  const uint32_t u = f2u(f);
  const uint32_t sign = (u >> 24) & 0x80u;
  const uint32_t a = u & 0x7fffffffu;
  if (a >= 0x7f800000u) return (uint8_t)(sign | 0x7fu);
  const int e = (int)(a >> 23) - 127;               // unbiased exponent (fp32 subnormals: e = -127)
  uint32_t code;
  if (e >= -6) {
    // normal e4m3 range: keep 3 of 23 mantissa bits
    uint32_t q = a >> 20;                            // exponent and top 3 mantissa bits
    const uint32_t r = a & 0xfffffu;
    if (r > 0x80000u || (r == 0x80000u && (q & 1u))) ++q;
    code = q - ((uint32_t)(127 - 7) << 3);          // rebias exponent 127 -> 7 (carry may bump it)
    if (code > 0x7eu) code = 0x7fu;
  } else {
    // subnormal e4m3 range: integer multiple of 2^-9, value = M * 2^(e-23) with M the 24-bit significand
    if (e < -127 + 1) return (uint8_t)sign;         // fp32 zero / subnormal inputs round to zero
    const uint32_t M = (a & 0x7fffffu) | 0x800000u;
    const int s = 14 - e;                            // M >> s = floor(value * 2^9); s >= 21
    if (s > 25) return (uint8_t)sign;                // value < 2^-11: rounds to 0
    uint32_t q = M >> s;
    const uint32_t r = M & ((1u << s) - 1u), half = 1u << (s - 1);
    if (r > half || (r == half && (q & 1u))) ++q;
    code = q;                                        // q == 8 is the smallest normal (0x08): consistent
  }
  return (uint8_t)(sign | code);
}

// e4m3fn code -> fp32 (exact), from the format definition.
__host__ __device__ inline float e4m3_to_f32(uint8_t c) {
  const uint32_t s = (uint32_t)(c & 0x80u) << 24;
  const uint32_t e = (c >> 3) & 0xfu, m = c & 7u;
  if (e == 0xfu && m == 7u) return u2f(s | 0x7fc00000u);
  if (e == 0) return u2f(s | f2u((float)m * 0.001953125f));   // m * 2^-9
  return u2f(s | ((e + 120u) << 23) | (m << 20));
}

// ---- Row400: the reference's compact e2m2b32 host row (dotsnote/engine/arcstats_pkg/arcstats/offload_rowfmt.py:1-22)
// [256 B low nibbles | 64 B sign bits | 16 x int8 block exponent k | 64 B e4m3fn rope]. Latent value e (0..511) has the
// 5-bit code (sign << 4) | mag, mag = nibble e % 2 of byte e / 2, sign = bit e % 8 of byte 256 + e / 8; the 32
// values of block b = e / 32 share k = byte 320 + b. mag = (e2 << 2) | m: value = (e2 ? 4 + m : m) *
// 2^(max(e2, 1) - 3 + k) (exponent clamped to [-126, 127]), clamped to +-448; the row's GPU form is the e4m3 code
// of that value (offload_rowfmt.py:131-160), exact whenever it lies in e4m3's range.
constexpr int ROW400 = 400, R4_SIGN = 256, R4_K = 320, R4_ROPE = 336;

// e2m2 code (5 bits) and block exponent -> e4m3fn code of the dequantized value (offload_rowfmt.py:149-158).
__host__ __device__ inline uint8_t e2m2_to_e4m3(uint32_t code, int k) {
  const uint32_t mag = code & 15u, e2 = mag >> 2, mm = mag & 3u;
  const uint32_t mant = e2 ? mm + 4u : mm;
  int ex = (e2 > 1u ? (int)e2 : 1) - 3 + k;
  ex = ex < -126 ? -126 : (ex > 127 ? 127 : ex);
  float v = (float)mant * u2f((uint32_t)(ex + 127) << 23);
  v = v > 448.f ? 448.f : v;                       // v >= 0 (or +inf, which the clamp also catches)
  const uint8_t c = e4m3_rne(v);
  return (uint8_t)(c | ((code & 16u) << 3));     // the sign survives rounding to zero (-0 -> 0x80)
}

// ---- XCD-aware workgroup order ---------------------------------------------------------------------------
// The dispatcher hands workgroup i to XCD (i % 8). remap_xcd(i, n) gives the logical work index so that
// each XCD receives a contiguous block of ceil(n / 8) logical items: consecutive logical items (e.g. the
// head groups of one token, which gather the same rows) then share one XCD's L2. Returns -1 for the padding
// workgroups of the last, partial block (the launch uses 8 * ceil(n / 8) workgroups).
__device__ inline int remap_xcd(int i, int n) {
  const int per = (n + 7) >> 3;
  const int f = (i & 7) * per + (i >> 3);
  return f < n ? f : -1;
}

// ---- launch error codes ----------------------------------------------------------------------------------
enum : int {
  SPMLA_OK = 0,
  SPMLA_EARG = -2,      // bad sizes / strides / null pointers
  SPMLA_EALIGN = -3,    // misaligned pointer or stride
  SPMLA_ELIMIT = -5,    // size beyond what the kernel supports
};

// ---- LDS DMA and hand-counted waits (shared by the attention and indexer kernels) ----------------------------
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"   // m0 is reserved; nothing else in these kernels uses it
// Direct global->LDS copy (lane l's 16 bytes land at lds + 16 * l). Issued through inline asm so that the
// compiler does not track it: it would otherwise drain every outstanding copy (vmcnt(0)) at the first
// s_waitcnt it places for its own loads. Completion is tracked by hand with wait_vm<>(). The LDS destination is
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

// Workgroup barrier for data exchanged through LDS only (no vector-memory drain).
__device__ inline void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

// vmcnt-only wait (expcnt and lgkmcnt left at their maxima), gfx9 encoding. Also a compiler memory barrier, so
// that reads of LDS filled by the copies are not moved above the wait.
template <int N>
__device__ inline void wait_vm() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
  asm volatile("" ::: "memory");
}

// ---- host: the dynamic-LDS limit of a kernel, raised once per device ---------------------------------------
// hipFuncSetAttribute applies to the current device, so each kernel keeps one bit per device (ids 0..63) of where
// it is set; the first launch on a device sets it under a mutex, later launches only read the bit. Safe to call
// from several host threads.
struct DynLds {
  std::atomic<uint64_t> done{0};
  std::mutex m;
  int ensure(const void* fn, int bytes) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return (int)e;
    const uint64_t bit = dev >= 0 && dev < 64 ? 1ull << dev : 0;
    if (bit && (done.load(std::memory_order_acquire) & bit)) return SPMLA_OK;
    std::lock_guard<std::mutex> g(m);
    if (bit && (done.load(std::memory_order_relaxed) & bit)) return SPMLA_OK;
    e = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, bytes);
    if (e != hipSuccess) return (int)e;
    done.fetch_or(bit, std::memory_order_release);
    return SPMLA_OK;
  }
};

}  // namespace spmla
