// Device-side building blocks shared by the attention kernels (gfx950 only).
//
// MFMA operand layout used throughout (v_mfma_f32_16x16x4_f32, wave64):
//   A (16x4):  lane l supplies A[m = l%16][k = l/16]
//   B (4x16):  lane l supplies B[k = l/16][n = l%16]
//   D (16x16): lane l holds    D[m = 4*(l/16) + i][n = l%16], i = 0..3
// The contraction index k can be mapped to any physical index as long as A and
// B agree.  For contractions over the head dimension, lane group g = l/16 owns
// the d-range [g*DP/4, (g+1)*DP/4) and MFMA step s uses d = g*DP/4 + s, so a
// lane reads its A operand for four consecutive steps with one 128-bit LDS
// load.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

// LDS row padding (floats) of the staged [rows][head_dim] tiles; a multiple of
// 4 keeps 128-bit LDS accesses aligned.
#ifndef WHA_LDS_PAD
#define WHA_LDS_PAD 4
#endif
// Waves per block of the forward and query-stationary backward kernels
// (16 queries per wave).
#ifndef WHA_FWD_NW
#define WHA_FWD_NW 4
#endif
#ifndef WHA_DQ_NW
#define WHA_DQ_NW 4
#endif
#ifndef WHA_LDS_SWZ
#define WHA_LDS_SWZ 1
#endif
#ifndef WHA_DKV_DMA
#define WHA_DKV_DMA 1
#endif
// Scheduling fence between the phases of a loop body: keeps the machine
// scheduler from hoisting every LDS operand read of an iteration to its top,
// which costs registers (and occupancy) for no gain.
#ifndef WHA_PRIO
#define WHA_PRIO 1
#endif
#ifndef WHA_FENCE
#define WHA_FENCE() __builtin_amdgcn_sched_barrier(0)
#endif

namespace wha {

typedef float floatx4 __attribute__((ext_vector_type(4)));

constexpr float kLog2e = 1.4426950408889634f;
// The MFMA accumulates a chain of fused multiply-adds, so scores are formed
// from accumulators started near the row's running maximum (partial sums stay
// small).  A tile or chunk whose scores pass the maximum it started from by
// more than this (log2 units) is formed again from the new maximum (the
// register-staged and small-problem forwards; the direct-to-LDS forward does
// so in its rescale branch, whose threshold is the same).
constexpr float kRedoMax = 8.f;
constexpr float kLn2 = 0.69314718055994531f;

// Strided [B,H,T,D] view (unit stride on d), shared by every [T][D] tensor of a call.
struct View {
  int B, H, T, D;
  int64_t sb, sh, st;
};

__device__ __forceinline__ floatx4 mfma4(float a, float b, floatx4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

// exp2 on the transcendental unit (v_exp_f32).  Arguments here are <= 0
// (scores minus a running max or minus the row LSE), so results lie in [0, 1];
// results below 2^-126 flush to zero, which changes no sum at fp32 precision.
__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

__device__ __forceinline__ float xor_shfl(float x, int mask) { return __shfl_xor(x, mask, 64); }

// phi = atan2(s, r) of the wave attention (src/common/attn.rs:121-128),
// evaluated in double and rounded once to f32: the correctly rounded phase
// (but for double-rounding cases of probability ~2^-29).  The reference's
// f32::atan2 calls the host libm's atan2f; glibc 2.35's agrees with the
// correctly rounded value on ~84% of inputs and is 1 ulp off otherwise, while
// the device's f32 atan2f is up to 3 ulp off it -- and the phase decides a
// discrete bucket, so the closer rounding keeps bucket flips rarer.
__device__ __forceinline__ float wave_phase(float s, float r) { return (float)atan2((double)s, (double)r); }

// phase_to_bucket (src/common/kv_cache.rs:66-70) in f32, operation for operation:
// fmod is exact and + and / are correctly rounded, so equal inputs give the
// reference's bucket bit for bit.
__device__ __forceinline__ int wave_phase_bucket(float phi) {
  const float tau = 6.28318548f;  // std::f32::consts::TAU
  const float width = tau / 8.f;
  const float nrm = fmodf(fmodf(phi, tau) + tau, tau);
  const float q = nrm / width;
  const int b = (q >= 0.f) ? (q < 8.f ? (int)q : 8) : 0;
  return b < 7 ? b : 7;
}

// The wave attention's bucket relation (src/common/attn.rs:189-224): key
// bucket kb and query bucket qb within one of each other mod 8, i.e.
// (kb - qb) mod 8 in {7, 0, 1}.  Symmetric in its arguments.
__device__ __forceinline__ bool wave_bucket_near(int kb, int qb) { return ((kb - qb + 1) & 7) <= 2; }

// Reductions over lane pairs (l, l^16) and (l, l^32) with the gfx950 VALU lane
// swaps instead of an LDS permute.  With both operands = x,
// v_permlane16_swap leaves lane l holding {x[l], x[l^16]} (in some order) and
// v_permlane32_swap {x[l], x[l^32]}; max and + are commutative, so both lanes of
// a pair get bit-identical results.
// max(a, b, c) and max(a, b) as compiler-visible operations (v_max3_f32 /
// v_max_f32, with an operand quieted where IEEE mode needs it).  These read
// MFMA results, and the compiler only inserts the wait states an MFMA result
// needs before a VALU read when it sees the read: an inline-asm v_max3_f32
// here once read a score chain's last accumulators with no wait at all and got
// stale values (a wrong running maximum, whole waves' rows shifted into
// underflow), and an asm output could also land on a register an MFMA still
// reads.  A NaN operand yields the other operand, as fmaxf does; a NaN score
// only ever comes from a NaN input, which the exp of the scores propagates.
__device__ __forceinline__ float vmax3(float a, float b, float c) { return fmaxf(fmaxf(a, b), c); }
__device__ __forceinline__ float vmax2(float a, float b) { return fmaxf(a, b); }
__device__ __forceinline__ float pair_max16(float x) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return vmax2(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float pair_max32(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return vmax2(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float pair_sum16(float x) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float pair_sum32(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// LDS layout of a staged [rows][DP] operand tile, addressed by 16-byte quads
// (four consecutive head-dim entries).  The kernels read such tiles in two
// patterns: lane (lq, g) reads quad c(g, j) of row r0 + lq (the A operand of
// contractions over the head dimension), or quad lq of row r0 + 4g + i (the A
// operand of contractions over rows); TileStage writes quad lane%16 of row
// r0 + lane/16.  A gfx950 ds_read_b128 runs in 4 cycles when the 16 lanes the
// LDS serves together hit 16 different 4-bank groups (measured with an LDS
// probe: a padded pitch such as DP+4 leaves both read patterns 2-way
// conflicted).  For DP = 64 rows are unpadded and quad c of row r is stored at
// quad c ^ (r & 11), which keeps all three patterns conflict-free for every
// lane grouping consistent with the probe; DP = 128 uses the XOR in swz().
// DP = 48 rows (12 quads) are unpadded too: the three 16-float groups of a
// row are stored in the order 1, 2, 0 and quad c within its group at
// c ^ ((r >> 2) & 3).  Its kernels pair it with a different assignment
// (dma48_row, dma48_quad): the A operand row m of an MFMA is tile row tr16(m)
// (rows transposed in 4 x 4 blocks), rows-by-lane reads take quads 4j + g, and
// the contractions over rows read d = 2lq, 2lq+1 (one 64-bit read) and
// d = 32 + lq (one 32-bit read) of rows tr16(4g + i) (lds_read_seg).  Then
// every ds_read_b128 is conflict-free for every lane grouping consistent with
// the probe, each 32-lane half of a ds_read_b64 (the halves the LDS serves
// together, measured with a probe) and all 64 lanes of a 32-bit read hit
// different banks.  Kernels opt in (ALLOW_SWZ):
// the permutation costs per-lane address registers, which only pays where LDS
// traffic matters more than VGPRs.  Other DP, and kernels that do not opt in,
// keep a 4-float pad.
template <int DP, bool ALLOW_SWZ = false>
struct Lds {
  static constexpr bool SWZ = WHA_LDS_SWZ && ALLOW_SWZ && (DP == 48 || DP == 64 || DP == 128);
  static constexpr int PITCH = SWZ ? DP : DP + WHA_LDS_PAD;
  // XOR applied to the quad index of row r (128-float rows: rows by lane read
  // quads 8g + j, and the contractions over rows read quads lq and lq + 16 --
  // see lds_read_seg -- which r & 11 does not keep apart)
  __device__ __forceinline__ static int swz(int r) { return DP == 64 ? (r & 11) : ((r & 3) | ((r >> 1) & 4)); }
  // stored position of quad c in row r, and the quad stored at position p
  __device__ __forceinline__ static int pq(int r, int c) {
    if constexpr (DP == 48) return 4 * (c < 4 ? 2 : (c >> 2) - 1) + ((c & 3) ^ ((r >> 2) & 3));
    else return c ^ swz(r);
  }
  __device__ __forceinline__ static int pq_inv(int r, int p) {
    if constexpr (DP == 48) return 4 * (p < 8 ? (p >> 2) + 1 : 0) + ((p & 3) ^ ((r >> 2) & 3));
    else return p ^ swz(r);
  }
  // float offset of quad c of row r
  __device__ __forceinline__ static int at(int r, int c) { return r * PITCH + 4 * (SWZ ? pq(r, c) : c); }
  // float offset of head-dim entry d of row r (a quad-aligned group of N <= 4
  // entries starting at d stays contiguous)
  __device__ __forceinline__ static int at_d(int r, int d) { return SWZ ? at(r, d >> 2) + (d & 3) : r * PITCH + d; }
};

// Cooperative global -> register -> LDS staging of a ROWS x DP tile of one
// (b,h) matrix, rows [row0, row0+ROWS), zero-filled past T and past D.
// VEC: 128-bit global loads (requires D, all strides and the base 16-byte
// aligned in floats, checked on the host); otherwise 32-bit loads.
template <int DP, int ROWS, int NT, bool VEC>
struct TileStage {
  static constexpr int C4 = DP / 4;             // float4 per row
  static constexpr int NF4 = ROWS * C4;         // float4 per tile
  static constexpr int PER = (NF4 + NT - 1) / NT;
  float4 r[PER];

  __device__ __forceinline__ void load(const float* __restrict__ base, int row0, int T, int D,
                                       int64_t st, int tid) {
    if (VEC && row0 + ROWS <= T && D == DP) {
      // whole tile in bounds (block-uniform): unpredicated 128-bit loads
#pragma unroll
      for (int p = 0; p < PER; ++p) {
        const int idx = tid + p * NT;
        if (NF4 % NT == 0 || idx < NF4) {
          const int row = idx / C4;
          const int c = (idx % C4) * 4;
          r[p] = *reinterpret_cast<const float4*>(base + (int64_t)(row0 + row) * st + c);
        }
      }
      return;
    }
#pragma unroll
    for (int p = 0; p < PER; ++p) {
      const int idx = tid + p * NT;
      const int row = idx / C4;
      const int c = (idx % C4) * 4;
      float4 val = make_float4(0.f, 0.f, 0.f, 0.f);
      if ((NF4 % NT == 0 || idx < NF4) && row0 + row < T) {
        const float* src = base + (int64_t)(row0 + row) * st + c;
        if (VEC) {
          if (c < D) val = *reinterpret_cast<const float4*>(src);
        } else {
          if (c + 0 < D) val.x = src[0];
          if (c + 1 < D) val.y = src[1];
          if (c + 2 < D) val.z = src[2];
          if (c + 3 < D) val.w = src[3];
        }
      }
      r[p] = val;
    }
  }

  template <int LD>
  __device__ __forceinline__ void store(float* lds, int tid) const {
#pragma unroll
    for (int p = 0; p < PER; ++p) {
      const int idx = tid + p * NT;
      if (NF4 % NT == 0 || idx < NF4) {
        const int row = idx / C4;
        const int c = (idx % C4) * 4;
        *reinterpret_cast<float4*>(lds + row * LD + c) = r[p];
      }
    }
  }

  // store in the Lds<DP, SW> layout
  template <bool SW = false>
  __device__ __forceinline__ void store_tile(float* lds, int tid) const {
#pragma unroll
    for (int p = 0; p < PER; ++p) {
      const int idx = tid + p * NT;
      if (NF4 % NT == 0 || idx < NF4) *reinterpret_cast<float4*>(lds + Lds<DP, SW>::at(idx / C4, idx % C4)) = r[p];
    }
  }
};

// Reads N head-dim entries of row r of an Lds<DP, SW> tile for lane lq: the
// entries [N*lq, N*lq + N) (padded tiles, and swizzled 64-wide tiles where
// N = 4), for swizzled 128-wide tiles quads lq and lq + 16 (d = 4lq..4lq+3
// and 64+4lq..64+4lq+3), or for swizzled 48-wide tiles d = 2lq, 2lq+1 and
// 32+lq (a 64-bit and a 32-bit read): the split layouts store_row_frag_split
// writes back.
template <int DP, int N, bool SW = false>
__device__ __forceinline__ void lds_read_seg(const float* tile, int r, int lq, float* out) {
  using LT = Lds<DP, SW>;
  if constexpr (LT::SWZ && N == 4) {
    const float4 v = *reinterpret_cast<const float4*>(tile + LT::at(r, lq));
    out[0] = v.x;
    out[1] = v.y;
    out[2] = v.z;
    out[3] = v.w;
  } else if constexpr (LT::SWZ && N == 8) {
    const float4 v = *reinterpret_cast<const float4*>(tile + LT::at(r, lq));
    const float4 w = *reinterpret_cast<const float4*>(tile + LT::at(r, lq + 16));
    out[0] = v.x;
    out[1] = v.y;
    out[2] = v.z;
    out[3] = v.w;
    out[4] = w.x;
    out[5] = w.y;
    out[6] = w.z;
    out[7] = w.w;
  } else if constexpr (LT::SWZ && DP == 48 && N == 3) {
    const float2 v = *reinterpret_cast<const float2*>(tile + LT::at_d(r, 2 * lq));
    out[0] = v.x;
    out[1] = v.y;
    out[2] = tile[LT::at_d(r, 32 + lq)];
  } else {
    static_assert(!LT::SWZ, "swizzled tiles are read in whole quads, or as d = 2lq, 2lq+1, 32+lq at DP = 48");
    const float* p = tile + r * LT::PITCH + N * lq;
    if (N % 4 == 0) {
#pragma unroll
      for (int c = 0; c < N / 4; ++c) {
        const float4 v = *reinterpret_cast<const float4*>(p + 4 * c);
        out[4 * c + 0] = v.x;
        out[4 * c + 1] = v.y;
        out[4 * c + 2] = v.z;
        out[4 * c + 3] = v.w;
      }
    } else {
#pragma unroll
      for (int c = 0; c < N; ++c) out[c] = p[c];
    }
  }
}

// gfx950 direct global -> LDS loads (global_load_lds_dword / _dwordx4): every
// lane supplies its own global address and its data lands at
// lds_base + lane * bytes (lds_base wave-uniform; checked on the box with a
// probe).  They count in vmcnt like other vector-memory loads.
__device__ __forceinline__ void dma_quad(const float* gsrc, float* lds_base) {
  __builtin_amdgcn_global_load_lds((const void __attribute__((address_space(1)))*)gsrc,
                                   (void __attribute__((address_space(3)))*)lds_base, 16, 0, 0);
}
__device__ __forceinline__ void dma_dword(const float* gsrc, float* lds_base) {
  __builtin_amdgcn_global_load_lds((const void __attribute__((address_space(1)))*)gsrc,
                                   (void __attribute__((address_space(3)))*)lds_base, 4, 0, 0);
}
// Wave priority from the share of a block's work still ahead of it
// (remaining / total in quarters -> s_setprio 3 .. 0).  The instruction
// arbiter otherwise favours the oldest waves, so of the blocks sharing a CU the
// first-dispatched one races ahead and the last one finishes alone, with the
// MFMA pipe mostly idle; ranking by remaining work keeps blocks of equal work
// finishing together.
__device__ __forceinline__ void prio_by_remaining(int remaining, int total) {
#if WHA_PRIO
  const int q = 4 * remaining;
  if (q > 3 * total) __builtin_amdgcn_s_setprio(3);
  else if (q > 2 * total) __builtin_amdgcn_s_setprio(2);
  else if (q > total) __builtin_amdgcn_s_setprio(1);
  else __builtin_amdgcn_s_setprio(0);
#endif
}

// 16 zero bytes in device memory: the DMA source of LDS quads past the head
// dimension when a head dim below 64 runs on the 64-wide kernels (the pad
// must hold exact zeros: a finite operand times a zero pad, never times data)
static __device__ __align__(16) float g_zero_quad[4];

// Raw buffer descriptors (gfx9 family: word 3 = 32-bit data format, no
// swizzle; loads are range-checked against the record count in bytes).  A
// buffer load takes a wave-uniform descriptor and offset from scalar registers
// and only a 32-bit offset per lane, so a fixed per-lane offset plus a moving
// uniform one costs no per-lane address arithmetic.
constexpr int kRawBufferWord3 = 0x00020000;
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buffer_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, kRawBufferWord3);
}
__device__ __forceinline__ float4 buffer_load_quad(__amdgpu_buffer_rsrc_t r, int voff, int soff) {
  const floatx4 v = __builtin_bit_cast(floatx4, __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, 0));
  return make_float4(v[0], v[1], v[2], v[3]);
}
__device__ __forceinline__ float buffer_load_float(__amdgpu_buffer_rsrc_t r, int voff, int soff) {
  return __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(r, voff, soff, 0));
}
// x by value: __builtin_bit_cast of a vector element (v[i]) miscompiles here
// (it reads element 0), so callers pass plain floats
__device__ __forceinline__ void buffer_store_float(__amdgpu_buffer_rsrc_t r, float x, int voff, int soff) {
  __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(x), r, voff, soff, 0);
}
// Four floats as two 64-bit stores.  A store of more than 8 bytes reads its
// data VGPRs after it issues and needs a wait state before a VALU instruction
// overwrites them, which this compiler does not always leave: a 128-bit store
// here came out followed directly by a v_max3_f32 into one of its data
// registers (the 128-wide kept-scores forward), and the stored scores were
// wrong in that element.  Stores of 8 bytes have no such hazard.
__device__ __forceinline__ void buffer_store_quad(__amdgpu_buffer_rsrc_t r, floatx4 v, int voff, int soff) {
  typedef unsigned uintx2 __attribute__((ext_vector_type(2)));
  typedef float floatx2 __attribute__((ext_vector_type(2)));
  const floatx2 lo = v.xy, hi = v.zw;
  __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(uintx2, lo), r, voff, soff, 0);
  __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(uintx2, hi), r, voff + 8, soff, 0);
}

// s_waitcnt vmcnt(0) (expcnt and lgkmcnt left at their maxima)
__device__ __forceinline__ void wait_vmem() { __builtin_amdgcn_s_waitcnt(0x0F70); }

// Index m = 4a + b of a 16-row group -> 4b + a (an involution).
__host__ __device__ __forceinline__ int tr16(int m) { return ((m & 3) << 2) | ((m >> 2) & 3) | (m & ~15); }
// Tile row of MFMA A-operand row m in the swizzled direct-to-LDS kernels:
// transposed in 4 x 4 blocks at DP = 48, else m itself.
template <int DP>
__device__ __forceinline__ int dma48_row(int m) { return DP == 48 ? tr16(m) : m; }
// Quad of k-step group j read by lane group g in a contraction over the head
// dimension (DG/4 groups of four k-steps): quads 4j + g at DP = 48, else the
// lane group's own contiguous range (DG/4) g + j.
template <int DP>
__device__ __forceinline__ int dma48_quad(int g, int j) { return DP == 48 ? 4 * j + g : (DP / 16) * g + j; }

// Reads quad c of row r of an Lds<DP, SW> tile.
template <int DP, bool SW = false>
__device__ __forceinline__ float4 lds_read_quad(const float* tile, int r, int c) {
  return *reinterpret_cast<const float4*>(tile + Lds<DP, SW>::at(r, c));
}

// Per-lane operand fragment of one row: lane group g = lane/16 holds
// x[row][g*DP/4 + s], s = 0 .. DP/4-1, multiplied by mul; zero past T and D.
template <int DP, bool VEC>
__device__ __forceinline__ void load_row_frag(const float* __restrict__ base, int row, int T, int D,
                                              int64_t st, int g, float mul, float* frag) {
  constexpr int DG = DP / 4;
  const int c0 = g * DG;
  if (row < T) {
    const float* src = base + (int64_t)row * st + c0;
    if (VEC) {
#pragma unroll
      for (int j = 0; j < DG / 4; ++j) {
        float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
        if (c0 + 4 * j < D) v = *reinterpret_cast<const float4*>(src + 4 * j);
        frag[4 * j + 0] = v.x * mul;
        frag[4 * j + 1] = v.y * mul;
        frag[4 * j + 2] = v.z * mul;
        frag[4 * j + 3] = v.w * mul;
      }
    } else {
#pragma unroll
      for (int s = 0; s < DG; ++s) frag[s] = (c0 + s < D) ? src[s] * mul : 0.f;
    }
  } else {
#pragma unroll
    for (int s = 0; s < DG; ++s) frag[s] = 0.f;
  }
}

// The row fragment matching dma48_quad: lane group g holds quads
// dma48_quad<DP>(g, j), j < DP/16, of row `row` in order (x[row][16j + 4g ..
// +3] at DP = 48; load_row_frag's contiguous range otherwise), times mul; zero
// past T and D.  128-bit loads.
template <int DP>
__device__ __forceinline__ void load_row_frag_dma(const float* __restrict__ base, int row, int T, int D,
                                                  int64_t st, int g, float mul, float* frag) {
  if constexpr (DP != 48) {
    load_row_frag<DP, true>(base, row, T, D, st, g, mul, frag);
  } else {
    const float* src = base + (int64_t)min(row, T - 1) * st;
#pragma unroll
    for (int j = 0; j < 3; ++j) {
      const int c = 4 * dma48_quad<DP>(g, j);
      float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
      if (row < T && c < D) v = *reinterpret_cast<const float4*>(src + c);
      frag[4 * j + 0] = v.x * mul;
      frag[4 * j + 1] = v.y * mul;
      frag[4 * j + 2] = v.z * mul;
      frag[4 * j + 3] = v.w * mul;
    }
  }
}

// Reads N consecutive floats from LDS (128-bit reads when N is a multiple of 4
// and the address is 16-byte aligned, which holds for every call site with
// N = 4 or 8).
template <int N>
__device__ __forceinline__ void lds_read_vec(const float* p, float* out) {
  if (N % 4 == 0) {
#pragma unroll
    for (int c = 0; c < N / 4; ++c) {
      const float4 v = *reinterpret_cast<const float4*>(p + 4 * c);
      out[4 * c + 0] = v.x;
      out[4 * c + 1] = v.y;
      out[4 * c + 2] = v.z;
      out[4 * c + 3] = v.w;
    }
  } else {
#pragma unroll
    for (int c = 0; c < N; ++c) out[c] = p[c];
  }
}

// Accumulators of a contraction X^T[d][r] += A^T[d][k] B[k][r] whose MFMA row m
// of d-tile dt stands for d = NDT*m + dt (NDT = DP/16).  With that
// permutation lane (lq, g) reads its A operands for all NDT d-tiles as NDT
// consecutive floats A[k][NDT*lq ...], and holds X[r][NDT*(4g+i) + dt] in
// acc[dt][i]: the contiguous d-range [g*DP/4, (g+1)*DP/4) of row r, the same
// range load_row_frag gives that lane.  Writes it scaled by mul.
template <int DP, bool VEC>
__device__ __forceinline__ void store_row_frag(float* __restrict__ base, int row, int T, int D, int64_t st,
                                               int g, const floatx4* acc, float mul) {
  constexpr int NDT = DP / 16;
  if (row >= T) return;
  float* dst = base + (int64_t)row * st;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int c0 = NDT * (4 * g + i);
    if (VEC && NDT % 4 == 0) {
#pragma unroll
      for (int c4 = 0; c4 < NDT / 4; ++c4) {
        const int c = c0 + 4 * c4;
        if (c < D)
          *reinterpret_cast<float4*>(dst + c) = make_float4(acc[4 * c4 + 0][i] * mul, acc[4 * c4 + 1][i] * mul,
                                                            acc[4 * c4 + 2][i] * mul, acc[4 * c4 + 3][i] * mul);
      }
    } else {
#pragma unroll
      for (int dt = 0; dt < NDT; ++dt)
        if (c0 + dt < D) dst[c0 + dt] = acc[dt][i] * mul;
    }
  }
}

// The contraction-over-rows accumulators of a kernel that reads its A operand
// with lds_read_seg<DP, NDT, true> (swizzled tiles): for DP = 64 the layout of
// store_row_frag; for DP = 128 d-tile dt < 4 holds d = 4m + dt and dt >= 4
// holds d = 64 + 4m + dt - 4 (m = MFMA row), so lane (lq, g) stores quads
// 4g+i and 16+4g+i of row `row`; for DP = 48 d-tiles 0 and 1 hold d = 2m and
// 2m + 1, d-tile 2 holds d = 32 + m, so the lane stores quads 2g, 2g+1 and
// 8+g.  128-bit stores, columns >= D skipped.
template <int DP>
__device__ __forceinline__ void store_row_frag_split(float* __restrict__ base, int row, int T, int D, int64_t st,
                                                     int g, const floatx4* acc, float mul) {
  if (DP == 64) {
    store_row_frag<DP, true>(base, row, T, D, st, g, acc, mul);
    return;
  }
  if (row >= T) return;
  float* dst = base + (int64_t)row * st;
  if (DP == 48) {
#pragma unroll
    for (int h = 0; h < 2; ++h)  // d = 8g + 4h + e <- d-tile e & 1 of row 4g + 2h + (e >> 1)
      *reinterpret_cast<float4*>(dst + 8 * g + 4 * h) =
          make_float4(acc[0][2 * h] * mul, acc[1][2 * h] * mul, acc[0][2 * h + 1] * mul, acc[1][2 * h + 1] * mul);
    if (32 + 4 * g < D)
      *reinterpret_cast<float4*>(dst + 32 + 4 * g) =
          make_float4(acc[2][0] * mul, acc[2][1] * mul, acc[2][2] * mul, acc[2][3] * mul);
    return;
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) {
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int c = 64 * h + 4 * (4 * g + i);
      if (c < D)
        *reinterpret_cast<float4*>(dst + c) = make_float4(acc[4 * h + 0][i] * mul, acc[4 * h + 1][i] * mul,
                                                          acc[4 * h + 2][i] * mul, acc[4 * h + 3][i] * mul);
    }
  }
}

// dS workspace of the backward, per (b,h), with Tp = T rounded up to 64:
// column block kt (keys 64kt..64kt+63) holds rows q = 64kt..Tp-1, 64 floats
// each, blocks back to back.  Rows past T exist so that a 64-query tile is
// written without a bounds check per row; they are never read.
// First row of column block kt: sum_{j<kt} (Tp - 64 j).
__host__ __device__ __forceinline__ int64_t ds_block_row(int kt, int T) {
  const int64_t Tp = ((int64_t)T + 63) / 64 * 64;
  return (int64_t)kt * Tp - (int64_t)32 * kt * (kt - 1);
}
// Rows of dS per (b,h).
__host__ __device__ __forceinline__ int64_t ds_rows(int T) { return ds_block_row((T + 63) / 64, T); }

}  // namespace wha
