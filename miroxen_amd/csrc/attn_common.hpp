// Shared device/host helpers for the gfx950 attention kernels.
#pragma once
#include <hip/hip_runtime.h>

#include <type_traits>
#include <utility>
#include <stdint.h>

#include "miroxen_attn.h"

namespace mxa {

using bf16x8 = __attribute__((ext_vector_type(8))) __bf16;
using bf16x4 = __attribute__((ext_vector_type(4))) __bf16;
using f32x16 = __attribute__((ext_vector_type(16))) float;
using f32x4 = __attribute__((ext_vector_type(4))) float;
using f32x2 = __attribute__((ext_vector_type(2))) float;
using i32x16 = __attribute__((ext_vector_type(16))) int;
using i32x8 = __attribute__((ext_vector_type(8))) int;
using i32x4 = __attribute__((ext_vector_type(4))) int;
using i32x32 = __attribute__((ext_vector_type(32))) int;
using u32x4 = __attribute__((ext_vector_type(4))) unsigned;
using u32x2 = __attribute__((ext_vector_type(2))) unsigned;

#define MXA_LDS __attribute__((address_space(3)))

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLog2_448 = 8.807354922057604f;  // log2(448): FP8 P is stored as 448*p
constexpr int kStatTok = 256;                     // tokens per kv_stats partial (reference kStatTok)
constexpr int kSqPad = 256;                       // Sage Q rows are padded to this multiple
constexpr int kKvPad = 64;                        // Sage key tile / K-scale group

__device__ __forceinline__ float bf2f(uint16_t h) { return __uint_as_float(uint32_t(h) << 16); }

// float -> bf16 bits, round to nearest even (v_cvt_pk_bf16_f32 on gfx950).
__device__ __forceinline__ uint16_t f2bf(float f) { return __builtin_bit_cast(uint16_t, (__bf16)f); }

__device__ __forceinline__ uint32_t pack_bf16x2(float a, float b) {
  using bf16x2 = __attribute__((ext_vector_type(2))) __bf16;
  return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2){a, b}, bf16x2));
}

// Value of `x` from lane (lane ^ 32): v_permlane32_swap exchanges the upper half
// of its first operand with the lower half of its second.
__device__ __forceinline__ float other_half(float x) {
  auto r = __builtin_amdgcn_permlane32_swap(__float_as_int(x), __float_as_int(x), false, false);
  return __int_as_float((threadIdx.x & 32) ? r[0] : r[1]);
}
__device__ __forceinline__ int other_half_i(int x) {
  auto r = __builtin_amdgcn_permlane32_swap(x, x, false, false);
  return (threadIdx.x & 32) ? r[0] : r[1];
}

// 16-byte global -> LDS copy: lane i of the wave writes lds_wave_base + 16*i.
__device__ __forceinline__ void g2lds16(const void* g, MXA_LDS void* lds_wave_base) {
  __builtin_amdgcn_global_load_lds(g, lds_wave_base, 16, 0, 0);
}

// f(std::integral_constant<int, 0>{}) ... f(std::integral_constant<int, N-1>{}).
template <typename F, int... J>
__device__ __forceinline__ void static_for_impl(F&& f, std::integer_sequence<int, J...>) {
  (f(std::integral_constant<int, J>{}), ...);
}
template <int N, typename F>
__device__ __forceinline__ void static_for(F&& f) {
  static_for_impl(f, std::make_integer_sequence<int, N>{});
}

// Raw buffer resource over `bytes` bytes from `base` (gfx9 dword3: 32-bit data,
// no swizzle). Loads at offsets >= bytes return zeros.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buf_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, int(bytes), 0x00020000);
}

// 16 bytes per lane from rsrc + voff + soff into LDS at lds_wave_base + 16 * lane.
// Constant offsets go in soff: an instruction offset would also move the LDS
// destination of a buffer-to-LDS load.
__device__ __forceinline__ void buf2lds16(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff,
                                          MXA_LDS void* lds_wave_base) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, lds_wave_base, 16, voff, soff, 0, 0);
}

__device__ __forceinline__ void wait_vm() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }

// 16-byte device-scope (sc1) buffer store, then two wait states. A VALU write to the
// data registers of a store of more than 8 bytes must not follow it directly (the
// store may read its data after that write); the compiler for gfx950 schedules such
// writes right after the store (seen: the next 16-byte group converted into the same
// registers, with values of that group stored in some lanes), so this store carries
// its own wait states.
__device__ __forceinline__ void store_b128_sc1(u32x4 d, __amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
  asm volatile("buffer_store_dwordx4 %0, %1, %2, %3 offen sc1\n\ts_nop 1" ::"v"(d), "v"(voff), "s"(r), "s"(soff)
               : "memory");
}

// Work-group barrier without __syncthreads()'s memory fence: the fence drains
// every outstanding global load (vmcnt(0)), which would serialize a multi-stage
// prefetch. Callers order LDS-DMA completion themselves with counted vmcnt waits;
// LDS reads issued before the barrier have been consumed (their lgkmcnt waited)
// before the barrier by construction.
__device__ __forceinline__ void block_sync() { asm volatile("s_barrier" ::: "memory"); }

// Key-liveness of one key per lane for a later tile: the in-range flag needs no
// memory, the mask byte is loaded from a clamped index and only combined (in
// key_live) when the tile is consumed, so the load never forces an early wait on
// the tile prefetch issued next to it.
struct KeyLive {
  int in_range, byte;
};
__device__ __forceinline__ KeyLive key_live_load(const mx_attn_params& p, int key) {
  KeyLive r;
  r.in_range = key < p.Skv;
  r.byte = 1;
  if (p.kv_valid) r.byte = p.kv_valid[key < p.Skv ? key : p.Skv - 1];
  return r;
}
__device__ __forceinline__ uint64_t key_live_ballot(const KeyLive& k) { return __ballot(k.in_range && k.byte); }

template <int N>
__device__ __forceinline__ void wait_vm_n() {
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

// Liveness bitmaps of 64-key tiles (bit j = key t*64+j exists and is not
// padding). With a key-padding mask they are built once per work-group into LDS
// (table of kMaxLiveTiles entries, so masked calls need Skv <= 65536), so the
// tile loop issues no per-tile mask loads; without a mask they are arithmetic.
// Wave w handles tiles w, w+NW, ...; all of a wave's mask bytes are requested
// before any is used.
constexpr int kMaxLiveTiles = 1024;
template <int NW, int KT>
__device__ __forceinline__ void build_live(uint64_t* live, const mx_attn_params& p, int nt, int wave, int lane) {
  if (!p.kv_valid) return;
  constexpr int B = 8;  // tiles per batch per wave
  for (int t0 = wave; t0 < nt; t0 += NW * B) {
    int byte[B];
#pragma unroll
    for (int j = 0; j < B; ++j) {
      const int t = t0 + j * NW, key = t * KT + lane;
      byte[j] = t < nt && key < p.Skv ? int(p.kv_valid[key]) : 0;
    }
#pragma unroll
    for (int j = 0; j < B; ++j) {
      const int t = t0 + j * NW;
      const uint64_t bits = __ballot(byte[j] != 0);
      if (t < nt && lane == 0) live[t] = bits;
    }
  }
}
// The same bitmaps from 16-byte loads when the mask is 16-byte aligned: lane i of a
// wave loads keys 16i..16i+15 of a 1024-key chunk (16 tiles) through a buffer
// resource ending at Skv (keys past it read as 0: dead), folds each byte to one bit
// and stores the 16 bits as entry 64c + i of the table viewed as uint16, so the
// table's uint64 t holds tile t's 64 keys in order. Wave w loads chunks w and w + NW
// first (live16_issue, before the caller's other loads, so their latencies overlap)
// and folds them, then any further chunks (live16_finish).
struct Live16 {
  u32x4 w[2];
};
__device__ __forceinline__ u32x4 live16_load(const mx_attn_params& p, int c, int lane) {
  const __amdgpu_buffer_rsrc_t r = buf_rsrc(p.kv_valid, uint32_t(p.Skv));
  return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, uint32_t(c * 1024 + lane * 16), 0, 0));
}
__device__ __forceinline__ void live16_store(uint64_t* live, u32x4 w, int c, int lane) {
  uint32_t bits = 0;
#pragma unroll
  for (int d = 0; d < 4; ++d) {
    const uint32_t x = w[d];
    const uint32_t hi = ((x & 0x7f7f7f7fu) + 0x7f7f7f7fu) | x;  // byte's top bit set iff the byte is nonzero
    bits |= ((((hi >> 7) & 0x01010101u) * 0x01020408u) >> 24) << (4 * d);
  }
  if (c * 16 + (lane >> 2) < kMaxLiveTiles) reinterpret_cast<uint16_t*>(live)[c * 64 + lane] = uint16_t(bits);
}
template <int NW>
__device__ __forceinline__ Live16 live16_issue(const mx_attn_params& p, int nt, int wave, int lane) {
  const int nch = (nt + 15) / 16;
  Live16 L;
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int c = wave + j * NW;
    L.w[j] = c < nch ? live16_load(p, c, lane) : u32x4{0, 0, 0, 0};
  }
  return L;
}
template <int NW>
__device__ __forceinline__ void live16_finish(uint64_t* live, const Live16& L, const mx_attn_params& p, int nt,
                                              int wave, int lane) {
  const int nch = (nt + 15) / 16;
#pragma unroll
  for (int j = 0; j < 2; ++j)
    if (wave + j * NW < nch) live16_store(live, L.w[j], wave + j * NW, lane);
  for (int c = wave + 2 * NW; c < nch; c += NW) live16_store(live, live16_load(p, c, lane), c, lane);
}

template <int KT>
__device__ __forceinline__ uint64_t tile_live(const uint64_t* live, const mx_attn_params& p, int t) {
  if (p.kv_valid) return live[t];
  const int left = p.Skv - t * KT;
  return left >= 64 ? ~0ull : (1ull << left) - 1;
}

// Logical work-group index for a grid of n blocks such that consecutive logical
// indices land on the same XCD (blocks are dispatched round-robin over 8 XCDs):
// work items that share K/V (same head) then share one XCD's L2.
__device__ __forceinline__ int xcd_remap(int b, int n) {
  const int q = n / 8, r = n % 8, x = b % 8, local = b / 8;
  return x * q + (x < r ? x : r) + local;
}

#ifdef MX_STAMPS
// Timing probe (debug builds only, one array per translation unit): per work-group,
// slots 0-3 take the 100 MHz chip clock at points the kernel chooses, slot 6 HW_ID
// and XCC_ID.
static __device__ uint64_t g_stamps[1 << 20];
__device__ __forceinline__ void stamp(int slot) {
  if (threadIdx.x == 0) {
    uint64_t* d = g_stamps + size_t(blockIdx.x) * 8;
    d[slot] = __builtin_amdgcn_s_memrealtime();
    if (slot == 0) d[6] = (uint64_t(__builtin_amdgcn_s_getreg(0xF814)) << 32) | __builtin_amdgcn_s_getreg(0xF804);
  }
}
#define MX_STAMP(i) stamp(i)
#else
#define MX_STAMP(i)
#endif

}  // namespace mxa
