// FP8 (e4m3fn) gate/up GEMM + SwiGLU on fragment-packed weights, for gfx950.
//
// Same arithmetic as ff_gemm_fp8_swiglu (one v_mfma_f32_16x16x128_f8f6f4 per
// 128-byte k step into the same fp32 accumulator, k steps in order, then
// bf16((acc * sa) * sw) and bf16(bf16(silu(g)) * u)), so the two produce
// identical bits. What differs is how the operands reach the matrix cores:
//
// * Weights are repacked once at setup (ff_pack_weight_fp8) so that the MFMA
//   operand of one 16-row x 128-byte fragment is 2 KB contiguous: lane l's 32
//   bytes are split into two 1 KB planes, the first 16 at 16 l and the last 16
//   at 1024 + 16 l. Each wave loads its weight fragments with buffer loads
//   straight into the operand registers: each of the two load instructions of
//   a fragment moves one contiguous 1 KB plane (whole cache lines, every byte
//   used; interleaving a lane's 32 bytes would make each instruction touch 2 KB
//   of lines for 1 KB of data), and no LDS traffic or barrier is spent on the
//   weights.
// * A workgroup of 4 waves owns BM tokens x BN = 4 CW weight rows; wave w owns
//   all BM tokens x CW rows, so each A fragment read from LDS feeds CW/16 MFMAs
//   (0.33 KB of LDS reads per MFMA at 144 x 96, a third of a 64 x 64 wave tile).
//   For the SwiGLU pairing each wave takes CW/2 gate channels and the matching
//   CW/2 up channels, alternating 16-channel fragments (gate, up, gate, ..).
// * The weight fragment is the MFMA's first operand and the activation fragment
//   its second, so the accumulator holds the transposed tile: lane 16 g + r of
//   fragment (i, j) holds tokens 16 i + r, channels 16 j + 4 g .. + 3. Each lane
//   thus owns 4 consecutive channels of one token, and the epilogues (SwiGLU,
//   scaling, bf16 rounding) run in registers and store 8-byte row pieces
//   without an LDS round trip. The products and their order are those of the
//   untransposed form, so the bits are the same.
// * Activations go global -> registers -> LDS (D steps of register staging,
//   2G LDS stages, one barrier per G steps). Every load is an ordinary
//   compiler-visible buffer load, so the compiler's wait counts are exact
//   partial waits; the prologue issues its loads in the loop's own order so the
//   loop entry needs no full drain.
// * Inside a k step the MFMAs run weight fragment by weight fragment, and each
//   weight fragment is refilled for step k + P as soon as its last MFMA has
//   been issued.
// * The MFMA is issued from inline asm with the accumulator tied ("+a"): the
//   compiler otherwise gives this gfx950 instruction distinct source and
//   destination AGPRs in an unrolled loop and copies every accumulator back at
//   the loop edge. The hazards the compiler no longer sees are covered by
//   s_nop: after the accumulators are zeroed, and after the last MFMA before
//   the epilogue reads them (ACC_NOPS).
//
// Packed layout (ff_pack_weight_fp8): fragment (f, kt) of rows [16 f, 16 f + 16)
// and k bytes [128 kt, 128 kt + 128) is the 2048 bytes at (kt * N/16 + f) * 2048
// (k-step major: the fragments every workgroup reads at one k step are
// contiguous; with the rows' k steps contiguous instead, the loads in flight
// together sat 64 KB apart and streamed weights from HBM 0.5-2 us slower per
// GEMM); lane l = 16 g + r holds row 16 f + r, k bytes [128 kt + 32 g, +16) at
// 16 l and [128 kt + 32 g + 16, +16) at 1024 + 16 l.
// That is the operand layout of the MFMA for both A and B (the row-major
// kernels feed the same k range to the same lane).
#include <stdio.h>
#include <type_traits>

#include "ff_common.h"
#include "ff_rope.h"

using namespace ff;

namespace {

constexpr int kThreads = 256;
constexpr int kXcds = 8;

constexpr int lcm3(int a, int b, int c) {
  int l = a;
  while (l % b || l % c) l += a;
  return l;
}

// acc += A . B^T for one 16 x 16 x 128 e4m3 tile (A rows index the result's
// rows, held as 4 consecutive rows per lane), accumulator tied in place.
__device__ __forceinline__ void mfma_acc(f32x4& acc, const i32x8& a, const i32x8& b) {
  asm volatile("v_mfma_f32_16x16x128_f8f6f4 %0, %1, %2, %0" : "+a"(acc) : "v"(a), "v"(b));
}

__global__ __launch_bounds__(kThreads) void pack_fp8_kernel(const uint8_t* __restrict__ w, uint8_t* __restrict__ p,
                                                            int64_t n, int64_t k) {
  const int64_t kt_n = k / 128;
  const int64_t lanes = (n / 16) * kt_n * 64;
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < lanes; i += (int64_t)gridDim.x * blockDim.x) {
    const int l = (int)(i & 63);
    const int64_t f = i >> 6;  // fragment index f16 * kt_n + kt
    const int64_t kt = f % kt_n, f16 = f / kt_n;
    const int64_t nf = n / 16;
    const int64_t row = f16 * 16 + (l & 15);
    const u32x4* src = reinterpret_cast<const u32x4*>(w + row * k + kt * 128 + 32 * (l >> 4));
    uint8_t* dst = p + (kt * nf + f16) * 2048 + 16 * l;
    *reinterpret_cast<u32x4*>(dst) = src[0];
    *reinterpret_cast<u32x4*>(dst + 1024) = src[1];
  }
}

// Main loop shared by the kernels below: acc (BM x 4 CW tile of this
// workgroup, wave w owning all BM rows x CW weight rows, transposed: acc[i][j]
// of lane 16 g + r is tokens 16 i + r, weight rows 16 j + 4 g .. + 3) = sum over k steps
// [kt0, kt0 + nk) of A . B^T. sB[j] is the byte offset of this wave's weight
// fragment row j at k step 0. P = weight register stages, D = activation
// register stages, G = k steps per barrier; nk % lcm(P, D, 2G) == 0. pre()
// runs once the first activation loads are issued, while they are in flight
// (VALU work of the epilogue that does not depend on the product).
template <int BM, int CW, int P, int D, int G, typename Pre>
__device__ __forceinline__ void pk_mainloop(f32x4 (&acc)[BM / 16][CW / 16], uint8_t* smem,
                                            const uint8_t* __restrict__ qa, int M, int K, int m0,
                                            const uint8_t* __restrict__ qwp, uint32_t wbytes,
                                            const uint32_t (&sB)[CW / 16], int kt0, int nk, Pre&& pre) {
  constexpr int RA = BM / 16, TJ = CW / 16;
  constexpr int A_CHUNKS = BM * 8;  // 16-byte chunks of one A stage
  constexpr int FULL = A_CHUNKS / kThreads, REM = A_CHUNKS % kThreads;
  constexpr int NA = FULL + (REM ? 1 : 0);
  constexpr int STAGE = BM * 128;
  constexpr int NB = 2 * G;
  constexpr int U = lcm3(P, D, NB);  // k steps per unrolled loop iteration
  static_assert(A_CHUNKS >= kThreads, "at least one full activation round");
  const int tid = threadIdx.x, lane = tid & 63;
  const int r16 = lane & 15, g = lane >> 4;
  const int kend = kt0 + nk;

  // Activations: chunk c = tid + 256 i is row c / 8, 16-byte chunk c % 8; a
  // partial last round is moved back over the last 256 chunks (the overlap is
  // loaded and stored twice with the same bytes), so nothing is predicated.
  // LDS stage layout: 1 KB blocks of 8 rows x 128 B, chunk c of row r at slot
  // c ^ (r % 8) ^ ((r / 8) % 2). A fragment read (16 rows, two chunks per row)
  // then puts every 8 lanes of a ds_read_b128 on 8 distinct slots of their 1 KB
  // blocks and every 16 lanes on 16 distinct 16-byte bank groups (c ^ ((r % 16) / 2),
  // the row-major kernels' slot rule, measured 10 % below this one in LDS read
  // throughput, 120 against 133 B per clock per CU).
  const __amdgpu_buffer_rsrc_t rA = make_rsrc(qa, (uint32_t)M * (uint32_t)K);
  uint32_t voffA[NA];
  int dstA[NA];
#pragma unroll
  for (int i = 0; i < NA; ++i) {
    const int c = i < FULL ? tid + kThreads * i : A_CHUNKS - kThreads + tid;
    const int row = c >> 3, ch = c & 7;
    voffA[i] = (uint32_t)min(m0 + row, M - 1) * (uint32_t)K + 16 * ch;
    dstA[i] = (row >> 3) * 1024 + 128 * (row & 7) + 16 * (ch ^ (row & 7) ^ ((row >> 3) & 1));
  }
  i32x4v ast[D][NA];  // ext-vector elements: an array of structs would be kept in scratch
  auto loadA = [&](int kt, auto SLOT) {
    constexpr int slot = decltype(SLOT)::value;
    static_for<0, NA>([&](auto I_) {
      constexpr int i = decltype(I_)::value;
      ast[slot][i] = bload16(rA, voffA[i], (uint32_t)kt * 128);
    });
  };
  auto writeA = [&](auto SLOT, auto BUF) {
    constexpr int slot = decltype(SLOT)::value, buf = decltype(BUF)::value;
    static_for<0, NA>([&](auto I_) {
      constexpr int i = decltype(I_)::value;
      *reinterpret_cast<i32x4v*>(smem + buf * STAGE + dstA[i]) = ast[slot][i];
    });
  };

  const __amdgpu_buffer_rsrc_t rB = make_rsrc(qwp, wbytes);
  const uint32_t kstride = wbytes / (uint32_t)(K / 128);
  const uint32_t voffB = 16u * (uint32_t)lane;
  i32x8 bq[P][TJ];
  auto loadB = [&](int kt, auto SLOT) {
    constexpr int slot = decltype(SLOT)::value;
#pragma unroll
    for (int j = 0; j < TJ; ++j) {
      const i32x4v lo = bload16(rB, voffB, sB[j] + (uint32_t)kt * kstride);
      const i32x4v hi = bload16(rB, voffB + 1024u, sB[j] + (uint32_t)kt * kstride);
      bq[slot][j] = i32x8{lo.x, lo.y, lo.z, lo.w, hi.x, hi.y, hi.z, hi.w};
    }
  };

#pragma unroll
  for (int i = 0; i < RA; ++i)
#pragma unroll
    for (int j = 0; j < TJ; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
  // ACC_PIN: every accumulator through an asm barrier (each is zeroed before it).
  // ACC_NOPS: wait states between VALU writes / MFMA results and their readers.
#define ACC_PIN()                                     \
  do {                                                \
    _Pragma("unroll") for (int i_ = 0; i_ < RA; ++i_) \
    _Pragma("unroll") for (int j_ = 0; j_ < TJ; ++j_) \
      asm volatile("" : "+a"(acc[i_][j_]));           \
  } while (0)
#define ACC_NOPS() asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7" : "+a"(acc[RA - 1][TJ - 1]))
  ACC_PIN();
  ACC_NOPS();

  // Prologue: LDS stages 0..G-1 = steps kt0..kt0+G-1, staging slots = the next D
  // steps, weight stages = steps kt0..kt0+P-1, issued in the loop's order (A,
  // then B) so that the loop entry needs no full drain.
  using I0 = std::integral_constant<int, 0>;
  static_for<0, G>([&](auto S_) {
    constexpr int s = decltype(S_)::value;
    loadA(min(kt0 + s, kend - 1), I0{});
    if constexpr (s == 0) {
      __builtin_amdgcn_sched_barrier(0);
      pre();
      __builtin_amdgcn_sched_barrier(0);
    }
    writeA(I0{}, std::integral_constant<int, s>{});
  });
  static_for<0, (D > P ? D : P)>([&](auto S_) {
    constexpr int s = decltype(S_)::value;
    if constexpr (s < D) loadA(min(kt0 + G + s, kend - 1), std::integral_constant<int, (G + s) % D>{});
    __builtin_amdgcn_sched_barrier(0);
    if constexpr (s < P) loadB(min(kt0 + s, kend - 1), std::integral_constant<int, s>{});
    __builtin_amdgcn_sched_barrier(0);
  });

  const int frag = 128 * (r16 & 7) + 1024 * (r16 >> 3);
  const int sw = (r16 & 7) ^ (r16 >> 3);
  const int c0 = 16 * ((2 * g) ^ sw), c1 = 16 * ((2 * g + 1) ^ sw);
  for (int kb = kt0; kb < kend; kb += U) {
    static_for<0, U>([&](auto U_) {
      constexpr int u = decltype(U_)::value;
      const int kt = kb + u;
      // One barrier per G steps: this group's stages (written during the previous
      // group) are visible, and the previous group's stages, overwritten below
      // with steps kt + G.., are no longer read.
      if constexpr (u % G == 0) __syncthreads();
      writeA(std::integral_constant<int, (u + G) % D>{}, std::integral_constant<int, (u + G) % NB>{});
      loadA(min(kt + G + D, kend - 1), std::integral_constant<int, (u + G) % D>{});
      const uint8_t* st = smem + (u % NB) * STAGE + frag;
      i32x8 af[RA];
#pragma unroll
      for (int i = 0; i < RA; ++i) {
        const i32x4v lo = *reinterpret_cast<const i32x4v*>(st + 2 * i * 1024 + c0);
        const i32x4v hi = *reinterpret_cast<const i32x4v*>(st + 2 * i * 1024 + c1);
        af[i] = i32x8{lo.x, lo.y, lo.z, lo.w, hi.x, hi.y, hi.z, hi.w};
      }
      const uint32_t ktn = (uint32_t)min(kt + P, kend - 1);
      static_for<0, TJ>([&](auto J_) {
        constexpr int j = decltype(J_)::value;
#pragma unroll
        for (int i = 0; i < RA; ++i) mfma_acc(acc[i][j], bq[u % P][j], af[i]);
        const i32x4v lo = bload16(rB, voffB, sB[j] + ktn * kstride);
        const i32x4v hi = bload16(rB, voffB + 1024u, sB[j] + ktn * kstride);
        bq[u % P][j] = i32x8{lo.x, lo.y, lo.z, lo.w, hi.x, hi.y, hi.z, hi.w};
      });
    });
  }
  ACC_NOPS();
  ACC_PIN();
#undef ACC_PIN
#undef ACC_NOPS
}

// LDS of the main loop's activation stages.
template <int BM, int G>
constexpr int pk_smem() {
  return 2 * G * BM * 128;
}

// The main loop with the next step's activation fragments read under this
// step's last MFMAs (same operands, same k order per accumulator as
// pk_mainloop, so the same bits). In pk_mainloop a step's fragment reads issue
// only once the previous step's last MFMA has: the four waves then wait together
// for the whole LDS delivery while their first MFMAs of the step trail it. Here
// two LDS stages; each step writes the next step's stage from registers first,
// runs its MFMAs weight fragment by weight fragment (each weight fragment
// refilled for step k + P right after its MFMAs, as in pk_mainloop), and takes
// its one barrier before the last weight fragment's MFMAs, each of which is
// followed by the read of the same activation fragment for the next step. The
// stage a step writes last held step k - 1, whose fragments every wave read
// before the previous step's barrier.
template <int BM, int CW, int P, int D, typename Pre>
__device__ __forceinline__ void pk_mainloop_pf(f32x4 (&acc)[BM / 16][CW / 16], uint8_t* smem,
                                               const uint8_t* __restrict__ qa, int M, int K, int m0,
                                               const uint8_t* __restrict__ qwp, uint32_t wbytes,
                                               const uint32_t (&sB)[CW / 16], int kt0, int nk, Pre&& pre) {
  constexpr int RA = BM / 16, TJ = CW / 16;
  constexpr int A_CHUNKS = BM * 8;
  constexpr int FULL = A_CHUNKS / kThreads, REM = A_CHUNKS % kThreads;
  constexpr int NA = FULL + (REM ? 1 : 0);
  constexpr int STAGE = BM * 128;
  constexpr int U = lcm3(P, D, 2);  // k steps per unrolled loop iteration
  static_assert(A_CHUNKS >= kThreads, "at least one full activation round");
  const int tid = threadIdx.x, lane = tid & 63;
  const int r16 = lane & 15, g = lane >> 4;
  const int kend = kt0 + nk;

  const __amdgpu_buffer_rsrc_t rA = make_rsrc(qa, (uint32_t)M * (uint32_t)K);
  uint32_t voffA[NA];
  int dstA[NA];
#pragma unroll
  for (int i = 0; i < NA; ++i) {
    const int c = i < FULL ? tid + kThreads * i : A_CHUNKS - kThreads + tid;
    const int row = c >> 3, ch = c & 7;
    voffA[i] = (uint32_t)min(m0 + row, M - 1) * (uint32_t)K + 16 * ch;
    dstA[i] = (row >> 3) * 1024 + 128 * (row & 7) + 16 * (ch ^ (row & 7) ^ ((row >> 3) & 1));
  }
  i32x4v ast[D][NA];
  auto loadA = [&](int kt, auto SLOT) {
    constexpr int slot = decltype(SLOT)::value;
    static_for<0, NA>([&](auto I_) {
      constexpr int i = decltype(I_)::value;
      ast[slot][i] = bload16(rA, voffA[i], (uint32_t)kt * 128);
    });
  };
  auto writeA = [&](auto SLOT, auto BUF) {
    constexpr int slot = decltype(SLOT)::value, buf = decltype(BUF)::value;
    static_for<0, NA>([&](auto I_) {
      constexpr int i = decltype(I_)::value;
      *reinterpret_cast<i32x4v*>(smem + buf * STAGE + dstA[i]) = ast[slot][i];
    });
  };

  const __amdgpu_buffer_rsrc_t rB = make_rsrc(qwp, wbytes);
  const uint32_t kstride = wbytes / (uint32_t)(K / 128);
  const uint32_t voffB = 16u * (uint32_t)lane;
  i32x8 bq[P][TJ];
  auto loadB = [&](int kt, auto SLOT) {
    constexpr int slot = decltype(SLOT)::value;
#pragma unroll
    for (int j = 0; j < TJ; ++j) {
      const i32x4v lo = bload16(rB, voffB, sB[j] + (uint32_t)kt * kstride);
      const i32x4v hi = bload16(rB, voffB + 1024u, sB[j] + (uint32_t)kt * kstride);
      bq[slot][j] = i32x8{lo.x, lo.y, lo.z, lo.w, hi.x, hi.y, hi.z, hi.w};
    }
  };
  const int frag = 128 * (r16 & 7) + 1024 * (r16 >> 3);
  const int sw = (r16 & 7) ^ (r16 >> 3);
  const int c0 = 16 * ((2 * g) ^ sw), c1 = 16 * ((2 * g + 1) ^ sw);
  i32x8 af[RA];
  auto readA = [&](int buf, int i) {
    const uint8_t* st = smem + buf * STAGE + frag + 2 * i * 1024;
    const i32x4v lo = *reinterpret_cast<const i32x4v*>(st + c0);
    const i32x4v hi = *reinterpret_cast<const i32x4v*>(st + c1);
    af[i] = i32x8{lo.x, lo.y, lo.z, lo.w, hi.x, hi.y, hi.z, hi.w};
  };

#pragma unroll
  for (int i = 0; i < RA; ++i)
#pragma unroll
    for (int j = 0; j < TJ; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
#define ACC_PIN()                                     \
  do {                                                \
    _Pragma("unroll") for (int i_ = 0; i_ < RA; ++i_) \
    _Pragma("unroll") for (int j_ = 0; j_ < TJ; ++j_) \
      asm volatile("" : "+a"(acc[i_][j_]));           \
  } while (0)
#define ACC_NOPS() asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7" : "+a"(acc[RA - 1][TJ - 1]))
  ACC_PIN();
  ACC_NOPS();

  // Prologue: stage 0 = step kt0; staging slots (s) % D = steps kt0 + s for
  // s = 1..D; weight stages = steps kt0..kt0+P-1; then step kt0's fragments.
  using I0 = std::integral_constant<int, 0>;
  loadA(kt0, I0{});
  __builtin_amdgcn_sched_barrier(0);
  pre();
  __builtin_amdgcn_sched_barrier(0);
  writeA(I0{}, I0{});
  static_for<0, (D > P ? D : P)>([&](auto S_) {
    constexpr int s = decltype(S_)::value;
    if constexpr (s < D) loadA(min(kt0 + 1 + s, kend - 1), std::integral_constant<int, (1 + s) % D>{});
    __builtin_amdgcn_sched_barrier(0);
    if constexpr (s < P) loadB(min(kt0 + s, kend - 1), std::integral_constant<int, s>{});
    __builtin_amdgcn_sched_barrier(0);
  });
  __syncthreads();
#pragma unroll
  for (int i = 0; i < RA; ++i) readA(0, i);

  for (int kb = kt0; kb < kend; kb += U) {
    static_for<0, U>([&](auto U_) {
      constexpr int u = decltype(U_)::value;
      const int kt = kb + u;
      // step kt + 1's stage (its buffer last held step kt - 1, whose fragments
      // every wave read before the previous step's barrier)
      writeA(std::integral_constant<int, (u + 1) % D>{}, std::integral_constant<int, (u + 1) % 2>{});
      loadA(min(kt + 1 + D, kend - 1), std::integral_constant<int, (u + 1) % D>{});
      const uint32_t ktn = (uint32_t)min(kt + P, kend - 1);
      static_for<0, TJ - 1>([&](auto J_) {
        constexpr int j = decltype(J_)::value;
#pragma unroll
        for (int i = 0; i < RA; ++i) mfma_acc(acc[i][j], bq[u % P][j], af[i]);
        const i32x4v lo = bload16(rB, voffB, sB[j] + ktn * kstride);
        const i32x4v hi = bload16(rB, voffB + 1024u, sB[j] + ktn * kstride);
        bq[u % P][j] = i32x8{lo.x, lo.y, lo.z, lo.w, hi.x, hi.y, hi.z, hi.w};
      });
      __syncthreads();
#pragma unroll
      for (int i = 0; i < RA; ++i) {
        mfma_acc(acc[i][TJ - 1], bq[u % P][TJ - 1], af[i]);
        readA((u + 1) % 2, i);
      }
      const i32x4v lo = bload16(rB, voffB, sB[TJ - 1] + ktn * kstride);
      const i32x4v hi = bload16(rB, voffB + 1024u, sB[TJ - 1] + ktn * kstride);
      bq[u % P][TJ - 1] = i32x8{lo.x, lo.y, lo.z, lo.w, hi.x, hi.y, hi.z, hi.w};
    });
  }
  ACC_NOPS();
  ACC_PIN();
#undef ACC_PIN
#undef ACC_NOPS
}


// Gate/up: BM tokens x (BN/2 gate + BN/2 up channels), BN = 4 CW; wave w takes
// gate channels [w CW/2, (w + 1) CW/2) of the tile and the matching up
// channels, as fragments j = 2 t (gate, channels 16 t ..) and j = 2 t + 1 (up,
// the same channels).
// SQ (static quantisation of the output): sa[0] and sw[0] are per-tensor
// scales and h is written as e4m3(clamp(h * qinv, +-448)) into hq (ldh bytes
// per row), without row maxima.
template <int BM, int CW, int P, int D, int G, bool SQ = false, bool PF = false>
__global__ __launch_bounds__(kThreads, 1) void gemm_fp8_swiglu_packed_kernel(
    const uint8_t* __restrict__ qa, const float* __restrict__ sa, const uint8_t* __restrict__ qwp,
    const float* __restrict__ sw, bf16_t* __restrict__ h, int64_t ldh, float* __restrict__ pmax, int M, int half,
    int K, int tiles_m, int tiles_n, uint8_t* __restrict__ hq, float qinv) {
  constexpr int BN = 4 * CW, CH = BN / 2, WCH = CW / 2;
  constexpr int RA = BM / 16, TJ = CW / 16, TT = TJ / 2;
  constexpr int SMEM = pk_smem<BM, G>();
  constexpr int Q16 = CH / 16;  // 16-channel blocks per tile row
  static_assert(SMEM <= 160 * 1024, "LDS budget");
  static_assert(TJ % 2 == 0 && CH % 64 == 0, "gate/up fragment pairs; whole 64-channel row-max blocks");
  __shared__ __align__(1024) uint8_t smem[SMEM];
  __shared__ float pm16[BM][Q16];  // max |h| per token and 16-channel block of the tile
  __shared__ uint16_t silu_tab[kSiluEntries];
  // sw of the tile's gate then up channels, sa of its tokens: copied in the
  // prologue (behind the table fill), so the epilogue reads them from LDS
  // instead of starting with their memory latency (no registers are left to
  // hold them through the main loop)
  __shared__ float sc_w[2 * CH], sc_a[BM];

  const int nblk = tiles_m * tiles_n;
  const int b = blockIdx.x;
  int logical = b;
  if (nblk % kXcds == 0) logical = (b % kXcds) * (nblk / kXcds) + b / kXcds;  // one XCD walks a tile range
  const int tm = logical % tiles_m, tn = logical / tiles_m;                    // M fastest: L2 shares weights
  const int m0 = tm * BM;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int r16 = lane & 15, g = lane >> 4;
  const int KT = K / 128;

  // Weights: fragment j of this wave is the 16-row group of gate (j even) or
  // up (j odd) rows of channels tn CH + wave WCH + 16 (j / 2) ..
  const int wave_s = __builtin_amdgcn_readfirstlane(wave);
  uint32_t sB[TJ];
#pragma unroll
  for (int j = 0; j < TJ; ++j) {
    const int row = (j & 1 ? half : 0) + tn * CH + wave_s * WCH + 16 * (j >> 1);
    sB[j] = (uint32_t)(row / 16) * 2048u;
  }
  f32x4 acc[RA][TJ];
  auto pre = [&] {
    constexpr int NSC = (2 * CH + BM + kThreads - 1) / kThreads;
    float v[NSC];
#pragma unroll
    for (int c = 0; c < NSC; ++c) {  // the loads first: the table fill runs under them
      const int e = tid + c * kThreads;
      if (e < 2 * CH) v[c] = sw[SQ ? 0 : (e < CH ? 0 : half - CH) + tn * CH + e];
      else if (e < 2 * CH + BM) v[c] = sa[SQ ? 0 : min(m0 + e - 2 * CH, M - 1)];
    }
    silu_table_fill<kThreads>(silu_tab, tid);
#pragma unroll
    for (int c = 0; c < NSC; ++c) {
      const int e = tid + c * kThreads;
      if (e < 2 * CH) sc_w[e] = v[c];
      else if (e < 2 * CH + BM) sc_a[e - 2 * CH] = v[c];
    }
  };
  if constexpr (PF)
    pk_mainloop_pf<BM, CW, P, D>(acc, smem, qa, M, K, m0, qwp, (uint32_t)(2 * half) * (uint32_t)K, sB, 0, KT, pre);
  else
    pk_mainloop<BM, CW, P, D, G>(acc, smem, qa, M, K, m0, qwp, (uint32_t)(2 * half) * (uint32_t)K, sB, 0, KT, pre);

  // g, u = bf16((acc * sa) * sw); h = bf16(bf16(silu(g)) * u), in registers:
  // lane 16 g + r holds token 16 i + r, channels c + 4 g .. + 3 of block t.
  // bf16(silu(g)) comes from the table filled in the prologue (written before
  // the main loop's first barrier). The row maximum is taken over |h| before
  // the rounding: bf16 rounding is monotonic and odd, so rounding the maximum
  // gives the maximum of the rounded values.
  const int c_base = tn * CH + wave * WCH + 4 * g;
  float swg[TT][4], swu[TT][4];
#pragma unroll
  for (int t = 0; t < TT; ++t)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      swg[t][r] = sc_w[wave * WCH + 4 * g + 16 * t + r];
      swu[t][r] = sc_w[CH + wave * WCH + 4 * g + 16 * t + r];
    }
  // First every g of the tile and its table read (the reads are all in flight
  // before the first result is needed), then h.
  uint32_t gp[RA][TT][2], tv[RA][TT][4];
  float sav[RA];
#pragma unroll
  for (int i = 0; i < RA; ++i) {
    sav[i] = sc_a[16 * i + r16];
#pragma unroll
    for (int t = 0; t < TT; ++t)
#pragma unroll
      for (int r = 0; r < 4; r += 2) {
        const uint32_t p = pack_bf16x2((acc[i][2 * t][r] * sav[i]) * swg[t][r],
                                       (acc[i][2 * t][r + 1] * sav[i]) * swg[t][r + 1]);
        gp[i][t][r / 2] = p;
        tv[i][t][r] = silu_bf16_read(p & 0xFFFFu, silu_tab);
        tv[i][t][r + 1] = silu_bf16_read(p >> 16, silu_tab);
      }
  }
#pragma unroll
  for (int i = 0; i < RA; ++i) {
    const int tl = 16 * i + r16, m = m0 + tl;
#pragma unroll
    for (int t = 0; t < TT; ++t) {
      float hv[4], mx = 0.f;
      uint32_t up[2];
#pragma unroll
      for (int r = 0; r < 4; r += 2)
        up[r / 2] = pack_bf16x2((acc[i][2 * t + 1][r] * sav[i]) * swu[t][r],
                                (acc[i][2 * t + 1][r + 1] * sav[i]) * swu[t][r + 1]);
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const uint32_t gb = r & 1 ? gp[i][t][r / 2] >> 16 : gp[i][t][r / 2] & 0xFFFFu;
        const float uv = r & 1 ? __uint_as_float(up[r / 2] & 0xFFFF0000u) : __uint_as_float(up[r / 2] << 16);
        hv[r] = silu_bf16_finish(gb, tv[i][t][r]) * uv;
        mx = fmaxf(mx, fabsf(hv[r]));
      }
      if constexpr (SQ) {
        if (m < M)
          *reinterpret_cast<uint32_t*>(hq + (int64_t)m * ldh + c_base + 16 * t) = quant4_static(
              round_bf16(hv[0]), round_bf16(hv[1]), round_bf16(hv[2]), round_bf16(hv[3]), qinv);
        continue;
      }
      if (m < M)
        *reinterpret_cast<u32x2*>(h + (int64_t)m * ldh + c_base + 16 * t) = pack4_bf16(hv[0], hv[1], hv[2], hv[3]);
      mx = max_rows(round_bf16(mx));  // over the 4 lanes of this token: 16 channels
      if (g == 0) pm16[tl][wave * TT + t] = mx;
    }
  }
  if constexpr (SQ) return;
  __syncthreads();
  // Row maxima per 64 channels (4 consecutive 16-channel blocks) for ff_quant_rows_pmax.
  const int64_t npart = half / 64;
  for (int c = tid; c < BM * (CH / 64); c += kThreads) {
    const int tl = c / (CH / 64), q = c % (CH / 64);
    const int m = m0 + tl;
    if (m < M)
      pmax[(int64_t)m * npart + tn * (CH / 64) + q] =
          fmaxf(fmaxf(pm16[tl][4 * q], pm16[tl][4 * q + 1]), fmaxf(pm16[tl][4 * q + 2], pm16[tl][4 * q + 3]));
  }
}

// y = bf16((acc * sa) * sw) for one BM x 4 CW tile held in the (transposed)
// accumulator layout of the main loop, stored as 8-byte row pieces: lane
// 16 g + r of fragment (i, j) writes token m0 + 16 i + r, columns
// n0 + wave CW + 16 j + 4 g .. + 3. sa per row if sa_rows else one value; sw
// per column if sw_cols else one value.
// The scales of this lane's outputs of a BM x 4 CW tile in the transposed
// accumulator layout: sa of tokens m0 + 16 i + r16, sw of columns c0 + 16 j +
// 4 g .. + 3 (c0 = the wave's first column). Loaded before the main loop, so
// the epilogue does not start with their memory latency.
template <int RA, int TJ>
struct PkScales {
  float sav[RA];
  float swv[TJ][4];
  __device__ __forceinline__ void load(const float* __restrict__ sa, int sa_rows, const float* __restrict__ sw,
                                       int sw_cols, int M, int m0, int c0) {
    const int lane = threadIdx.x & 63, r16 = lane & 15, g = lane >> 4;
#pragma unroll
    for (int i = 0; i < RA; ++i) sav[i] = sa[sa_rows ? min(m0 + 16 * i + r16, M - 1) : 0];
#pragma unroll
    for (int j = 0; j < TJ; ++j)
#pragma unroll
      for (int r = 0; r < 4; ++r) swv[j][r] = sw[sw_cols ? c0 + 16 * j + 4 * g + r : 0];
  }
};

template <int BM, int CW>
__device__ __forceinline__ void pk_store_tile(const f32x4 (&acc)[BM / 16][CW / 16],
                                              const PkScales<BM / 16, CW / 16>& sc, bf16_t* __restrict__ y,
                                              int64_t ldy, int M, int m0, int n0) {
  constexpr int RA = BM / 16, TJ = CW / 16;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int r16 = lane & 15, g = lane >> 4;
  const float(&sav)[RA] = sc.sav;
#pragma unroll
  for (int j = 0; j < TJ; ++j) {
    const int col = n0 + wave * CW + 16 * j + 4 * g;
    const float(&swv)[4] = sc.swv[j];
#pragma unroll
    for (int i = 0; i < RA; ++i) {
      const int m = m0 + 16 * i + r16;
      if (m < M)
        *reinterpret_cast<u32x2*>(y + (int64_t)m * ldy + col) =
            pack4_bf16((acc[i][j][0] * sav[i]) * swv[0], (acc[i][j][1] * sav[i]) * swv[1],
                       (acc[i][j][2] * sav[i]) * swv[2], (acc[i][j][3] * sav[i]) * swv[3]);
    }
  }
}

// Plain y = bf16((A . W^T * sa) * sw) with k split S ways: workgroup (tile,
// split) runs k steps [split KT/S, (split + 1) KT/S). With S == 1 it stores y;
// with S > 1 it stores its fp32 partial tile row-major over the rows padded to
// whole tiles, part[(split Mp + row) N + col] (Mp = tiles_m BM), and the next
// launch adds the partials: split_reduce_kernel, or the add_rms row kernel
// that takes them in place of its bf16 addend.
template <int BM, int CW, int P, int D, int G, int S, bool PF = false>
__global__ __launch_bounds__(kThreads, BM <= 96 && !PF ? 2 : 1) void gemm_fp8_split_packed_kernel(
    const uint8_t* __restrict__ qa, const float* __restrict__ sa, int sa_rows, const uint8_t* __restrict__ qwp,
    const float* __restrict__ sw, int sw_cols, bf16_t* __restrict__ y, int64_t ldy, int M, int N, int K,
    int tiles_m, int tiles_n, float* __restrict__ part) {
  constexpr int BN = 4 * CW;
  constexpr int RA = BM / 16, TJ = CW / 16;
  constexpr int SMEM = pk_smem<BM, G>();  // pk_mainloop_pf uses the first two stages
  static_assert(SMEM <= 160 * 1024, "LDS budget");
  __shared__ __align__(1024) uint8_t smem[SMEM];

  const int nblk = tiles_m * tiles_n * S;
  const int b = blockIdx.x;
  int logical = b;
  if (nblk % kXcds == 0) logical = (b % kXcds) * (nblk / kXcds) + b / kXcds;
  const int tm = logical % tiles_m, rest = logical / tiles_m;  // M fastest: L2 shares weights
  const int split = rest % S, tn = rest / S;
  const int m0 = tm * BM, n0 = tn * BN;
  const int tid = threadIdx.x, wave = tid >> 6;
  // this split's k steps: the kt / U blocks of U steps (U = the main loop's
  // unrolled steps) dealt out as evenly as whole blocks allow, so k need not
  // divide by S U (32B down, 200 steps: 3 splits of 68, 68 and 64)
  constexpr int U = PF ? lcm3(P, D, 2) : lcm3(P, D, 2 * G);
  const int nbk = K / (128 * U);
  const int kt0 = split * nbk / S * U, nk = (split + 1) * nbk / S * U - kt0;

  const int wave_s = __builtin_amdgcn_readfirstlane(wave);
  uint32_t sB[TJ];
#pragma unroll
  for (int j = 0; j < TJ; ++j) sB[j] = (uint32_t)((n0 + wave_s * CW + 16 * j) / 16) * 2048u;
  f32x4 acc[RA][TJ];
  PkScales<RA, TJ> sc;
  if constexpr (S == 1) sc.load(sa, sa_rows, sw, sw_cols, M, m0, n0 + wave_s * CW);
  if constexpr (PF)
    pk_mainloop_pf<BM, CW, P, D>(acc, smem, qa, M, K, m0, qwp, (uint32_t)N * (uint32_t)K, sB, kt0, nk, [] {});
  else
    pk_mainloop<BM, CW, P, D, G>(acc, smem, qa, M, K, m0, qwp, (uint32_t)N * (uint32_t)K, sB, kt0, nk, [] {});
  if constexpr (S > 1) {
    // the fp32 partial tile, row-major over the rows padded to whole tiles
    store_tile_rows_lds<BM, CW, SMEM>(acc, smem, part + ((int64_t)split * tiles_m * BM + m0) * N + n0, N, tid);
  } else {
    pk_store_tile<BM, CW>(acc, sc, y, ldy, M, m0, n0);
  }
}

// y = bf16((sum_s part_s * sa) * sw) for the rows < M of a split launch's
// row-major partials, added in split order 0, 1, .., S-1 (the unsplit
// kernel's arithmetic on the same sums); one thread per 8 columns.
template <int S>
__global__ __launch_bounds__(kThreads) void split_reduce_kernel(const float* __restrict__ part, int64_t mp,
                                                                const float* __restrict__ sa, int sa_rows,
                                                                const float* __restrict__ sw, int sw_cols,
                                                                bf16_t* __restrict__ y, int64_t ldy, int M, int N) {
  const int nc = N / 8;
  const int64_t e = (int64_t)blockIdx.x * kThreads + threadIdx.x;
  const int m = (int)(e / nc), col = (int)(e % nc) * 8;
  if (m >= M) return;
  f32x4 v[S][2], vs[2];
#pragma unroll
  for (int s2 = 0; s2 < S; ++s2) {
    const float* src = part + ((int64_t)s2 * mp + m) * N + col;
    v[s2][0] = *reinterpret_cast<const f32x4*>(src);
    v[s2][1] = *reinterpret_cast<const f32x4*>(src + 4);
  }
  if (sw_cols && ((uintptr_t)sw & 15) == 0) {
    vs[0] = *reinterpret_cast<const f32x4*>(sw + col);
    vs[1] = *reinterpret_cast<const f32x4*>(sw + col + 4);
  } else if (sw_cols) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      vs[0][r] = sw[col + r];
      vs[1][r] = sw[col + 4 + r];
    }
  } else {
    vs[0] = vs[1] = f32x4{sw[0], sw[0], sw[0], sw[0]};
  }
  const float sav = sa[sa_rows ? m : 0];
  float f[8];
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    f32x4 t = v[0][h];
#pragma unroll
    for (int s2 = 1; s2 < S; ++s2) t = t + v[s2][h];
#pragma unroll
    for (int r = 0; r < 4; ++r) f[4 * h + r] = (t[r] * sav) * vs[h][r];
  }
  *reinterpret_cast<u32x4*>(y + (int64_t)m * ldy + col) = pack8(f);
}

// The configuration measured for the 8B gate/up shape (576 x 4096 x 2 x 12288):
// 144 x 384 tiles, one workgroup per CU (4 x 64 = 256 workgroups).
constexpr int kPkBM = 144, kPkCW = 96, kPkP = 2, kPkD = 2, kPkG = 2;
constexpr int kPkKAlign = 128 * lcm3(kPkP, kPkD, 2 * kPkG);  // k multiple of the unrolled k steps

// Wave width CW of the packed gate/up tile (CW / 2 gate + CW / 2 up channels
// per wave, 2 CW channels of h per workgroup) for MLP width i: 96 (192-channel
// tiles) where i allows it, else 64 (128-channel tiles: the 32B shape's 25600
// and the 4B shape's 9728 channels); 0 when neither divides i (the row-major
// kernel runs then).
// Row tiles of the 64-channel tile (CW = 32) for short m: one row tile of the
// smallest height that holds m.
constexpr int kSwNarrowBM[5] = {64, 80, 112, 144, 176};

int swiglu_cw(int64_t m, int64_t i) {
  const int forced = ff_tuning(FF_TUNE_SWIGLU_PK_TILE) % 1000;
  if (forced == 32 || forced == 64 || forced == 96) return i % (2 * forced) == 0 ? forced : 0;
  // Short m with at least 192 channel tiles of 64: one row tile of 64
  // channels x up to 176 tokens per workgroup, so each weight is read by one
  // workgroup (176 tokens, 8B: 192 workgroups; the 4.47 ms step takes 4.18
  // ms, against 80 x 384 tiles).
  if (m > 4 && m <= kSwNarrowBM[4] && i % 64 == 0 && i / 64 >= 192) return 32;
  return i % 192 == 0 ? 96 : (i % 128 == 0 ? 64 : 0);
}

// Row-tile height of the packed gate/up GEMM for m tokens and tiles_n column
// tiles: the candidate whose grid takes the fewest row steps per CU, counted as
// rounds of 256 workgroups (one per CU) x (BM + 16) rows (the 16 stand for the
// per-tile prologue and the lower operand reuse of shorter tiles), ties to the
// taller tile; 0 when no candidate gives 192 or more workgroups (the row-major
// kernel runs then). 8B gate/up (64 column tiles): 576 tokens 144 x 384 tiles
// in one round; 640 tokens 80 (two rounds of 80 against two of 144); 176 and
// 320 tokens 80; 2048 tokens 128.
int swiglu_bm(int64_t m, int64_t tiles_n, int cw) {
  // ff_set_tuning(FF_TUNE_SWIGLU_PK_TILE, 1000 bm + cw) forces the tile for measurement sweeps
  const int forced = ff_tuning(FF_TUNE_SWIGLU_PK_TILE) / 1000;
  if (forced) return forced;
  if (cw == 32) {
    for (const int bm : kSwNarrowBM)
      if (bm >= m) return bm;
    return 0;
  }
  constexpr int cand[5] = {144, 128, 112, 96, 80};
  int best = 0;
  int64_t best_cost = 0;
  for (const int bm : cand) {
    const int64_t tiles = (m + bm - 1) / bm * tiles_n;
    if (tiles < 192) continue;
    const int64_t cost = (tiles + 255) / 256 * (bm + 16);
    if (best == 0 || cost < best_cost) {
      best = bm;
      best_cost = cost;
    }
  }
  return best;
}

// Gate/up tile for callers without the row-major weight (every m > 4 must run
// on the packed copy): where the library's plan declines (too few workgroups),
// the instantiated tile with the most workgroups, ties to the taller tile.
void swiglu_any_tile(int64_t m, int64_t i, int* cw_out, int* bm_out) {
  constexpr int cands[15][2] = {{144, 96}, {128, 96}, {112, 96}, {96, 96}, {80, 96},
                                {144, 64}, {128, 64}, {112, 64}, {96, 64}, {80, 64},
                                {176, 32}, {144, 32}, {112, 32}, {80, 32}, {64, 32}};
  int64_t most = 0;
  *cw_out = *bm_out = 0;
  for (const auto& c : cands) {
    if (i % (2 * c[1])) continue;
    const int64_t wg = (m + c[0] - 1) / c[0] * (i / (2 * c[1]));
    if (wg > most) {
      most = wg;
      *bm_out = c[0];
      *cw_out = c[1];
    }
  }
}

// Plain GEMM: 144 x 256 tiles, k split so that about 256 workgroups run (the
// 8B o and down projections: 4 x 16 tiles, 4 splits).
constexpr int kSpBM = 144, kSpCW = 64, kSpP = 2, kSpD = 2, kSpG = 2;
constexpr int kSpBN = 4 * kSpCW;
constexpr int kSpU = lcm3(kSpP, kSpD, 2 * kSpG);

// The plain packed GEMM's plan for an m x n x k product: row tile bm (x 256
// weight rows) and k splits s (1: unsplit, 0: the kernel does not take it).
// One launch when 144-row tiles fill the GPU, else 144-row tiles with k split
// when k is long enough that the extra reduction pays off (the 8B down
// projection, 576 x 4096 x 12288); shorter k takes small_plan's tiles (below)
// or the row-major kernels. ff_set_tuning(FF_TUNE_FP8_PK_SPLIT, 100 bm + s)
// forces bm in {64, 144} and s in {1, ..., 6, 8} for measurement sweeps.
// (80-row tiles at two workgroups per CU with half the k splits, fewer fp32
// partials on the same grid, measured slower: the 8B FP8 step 6.35 -> 6.85 ms
// with the down projection on 80 x 256 tiles split 2 ways instead of 144 x 256
// split 4 ways.)
// cw: the wave width (weight rows per wave; 4 cw per tile): kSpCW, or 32 for
// one-head-wide (128-column) tiles.
struct SplitPlan {
  int bm = 0, s = 0, cw = kSpCW;
};
SplitPlan split_plan(int64_t m, int64_t n, int64_t k) {
  SplitPlan p;
  if (m <= 4 || n % 128 || k % 128 || m * k >= (int64_t(1) << 31) || n * k >= (int64_t(1) << 31)) return p;
  const int64_t kt = k / 128;
  const int forced_short = k <= 4096 ? ff_tuning(FF_TUNE_FP8_PK_SPLIT_SHORT_K) : 0;
  const int forced = forced_short ? forced_short : ff_tuning(FF_TUNE_FP8_PK_SPLIT);
  if (forced) {
    // 100 bm + s: 256-column tiles, bm 64 or 144; 100000 + 100 bm + s: 128-column tiles, bm 64, 80, 96, 128 or 144
    const int cw = forced >= 100000 ? 32 : kSpCW, f = forced % 100000;
    const int bm = f / 100, sp = f % 100;
    const bool bm_ok =
        cw == 32 ? (bm == 64 || bm == 80 || bm == 96 || bm == 128 || bm == kSpBM) : (bm == 64 || bm == kSpBM);
    if (bm_ok && n % (4 * cw) == 0 && (sp >= 1 && sp <= 6 || sp == 8) && kt % kSpU == 0 &&
        kt / kSpU >= sp) {
      p.bm = bm;
      p.s = sp;
      p.cw = cw;
    }
    return p;
  }
  if (n % kSpBN) return p;
  const int64_t tiles = (m + kSpBM - 1) / kSpBM * (n / kSpBN);
  if (tiles >= 192) {
    if (kt % kSpU == 0) p = SplitPlan{kSpBM, 1};
    return p;
  }
  if (m <= 256) {
    // Short m (up to four 64-row tiles): 64 x 256 tiles, k split the most ways
    // among 8, 6, 5, 4 and 2 that keeps the grid within 256 workgroups (8, 4
    // and 2 where they divide k into whole unrolled blocks; 6 and 5, whose
    // split kernels run pk_mainloop_pf and deal out 2-step blocks, where every
    // split gets at least two of them): 176 tokens of the 8B shape, o and down
    // 48 tiles x 5 splits, 240 workgroups (4 splits, 192 workgroups, took the
    // 4.47 ms step to 4.31 ms against small_plan's 64 x 128 tiles for o and
    // 144 x 256 tiles split 8 ways for down).
    const int64_t t64 = (m + 63) / 64 * (n / kSpBN);
    for (const int sp : {8, 6, 5, 4, 2}) {
      const bool even = sp == 8 || sp == 4 || sp == 2;
      if (t64 * sp <= 256 && (even ? kt % (sp * kSpU) == 0 : kt >= 4 * sp)) return SplitPlan{64, sp};
    }
  }
  if (kt < 64) return p;
  // 64 k steps (the 32B o projection, 1024 x 8192 x 5120): where an unsplit
  // small tile (small_plan) fills the GPU on its own, no split: 8 splits of
  // 144 x 256 tiles wrote and read back 168 MB of fp32 partials (32B step
  // 47.40 -> 43.97 ms on unsplit 64 x 256 tiles; 44.57 ms split 2 ways).
  if (kt == 64) {
    constexpr int cand[3][2] = {{64, 64}, {96, 32}, {64, 32}};
    for (const auto& c : cand) {
      const int64_t t = (m + c[0] - 1) / c[0] * (n / (4 * c[1]));
      if (n % (4 * c[1]) == 0 && t >= 192 && t <= 512) return p;
    }
  }
  // The split count (2, 3, 4 or 8) with the fewest k steps per CU: rounds of
  // 256 workgroups (one per CU) x the longest split's steps (whole blocks of
  // kSpU steps, dealt out as evenly as they go), ties to fewer splits (less
  // partial traffic). 8B down (k = 12288): 576 tokens 4 in one round, 640
  // tokens 3 in one round (4 would take two), 1152 tokens 2; 32B down (1024 x
  // 25600 x 5120, 160 tiles) 3 in two rounds of 68 steps, where 2 splits took
  // two rounds of 100.
  if (kt % kSpU) return p;
  const int64_t nbk = kt / kSpU;
  int64_t best_steps = 0;
  for (int sp = 2; sp <= 8; sp += sp < 4 ? 1 : 4) {
    if (nbk < sp) continue;
    const int64_t steps = (tiles * sp + 255) / 256 * ((nbk + sp - 1) / sp * kSpU);
    if (p.s == 0 || steps < best_steps) {
      p = SplitPlan{kSpBM, sp};
      best_steps = steps;
    }
  }
  return p;
}

// Unsplit plain GEMMs whose 144 x 256 tiles are too few and whose k is too
// short to split (the 8B o projection, 576 x 4096 x 4096; a QKV-shaped plain
// GEMM): smaller packed tiles at two workgroups per CU. BM x 4 CW with BM =
// 64, CW = 64, else BM = 80, CW = 32 where that grid fits one round of one
// workgroup per CU, else BM = 96, CW = 32, else BM = 64, CW = 32, the first
// whose grid has 192 .. 512 workgroups (8B o projection: 80 x 128 tiles, 256
// workgroups, 20.4 / 19.3 -> 19.3 / 17.8 us per launch against 96 x 128
// tiles at 192 workgroups; 64 x 128 at 288 workgroups 20.9 us). A wave still owns all BM rows of its CW
// weight rows, so each weight fragment feeds BM / 16 MFMAs and the
// activations alone go through LDS (the row-major kernels' 2 x 2 waves at 64
// x 128 read both operands from LDS: 1.8-2.5 us slower at these shapes).
struct SmallTile {
  int bm = 0, cw = 0;
};
SmallTile small_plan(int64_t m, int64_t n, int64_t k, bool any_count = false) {
  SmallTile t;
  if (m <= 4 || k % (128 * kSpU) || m * k >= (int64_t(1) << 31) || n * k >= (int64_t(1) << 31)) return t;
  constexpr int cand[4][2] = {{64, 64}, {80, 32}, {96, 32}, {64, 32}};
  for (const auto& c : cand) {
    if (n % (4 * c[1])) continue;
    const int64_t tiles = (m + c[0] - 1) / c[0] * (n / (4 * c[1]));
    if (tiles >= 192 && tiles <= (c[0] == 80 ? 256 : 512)) {
      t.bm = c[0];
      t.cw = c[1];
      return t;
    }
  }
  // Short m (no candidate reaches 192 workgroups): the candidate with the
  // most workgroups, if it has at least 64 (the row-major kernel's 64 x 128
  // tiles give no more) or there is no row-major weight (any_count).
  int64_t most = any_count ? 0 : 63;
  for (const auto& c : cand) {
    if (n % (4 * c[1]) || c[0] == 80) continue;
    const int64_t tiles = (m + c[0] - 1) / c[0] * (n / (4 * c[1]));
    if (tiles > most && tiles <= 512) {
      most = tiles;
      t.bm = c[0];
      t.cw = c[1];
    }
  }
  return t;
}

template <int BM, int CW>
void launch_small(const void* qa, const float* sa, int sa_rows, const void* qw_packed, const float* sw, int sw_cols,
                  void* y, int64_t ldy, int64_t m, int64_t n, int64_t k, hipStream_t st) {
  const int64_t tm = (m + BM - 1) / BM, tn = n / (4 * CW);
  // The 80 x 128 tile (the 8B o projection at 576 tokens) on pk_mainloop_pf.
  constexpr bool pf = BM == 80 && CW == 32;
  hipLaunchKernelGGL((gemm_fp8_split_packed_kernel<BM, CW, kSpP, kSpD, kSpG, 1, pf>), dim3((unsigned)(tm * tn)),
                     dim3(kThreads), 0, st, (const uint8_t*)qa, sa, sa_rows, (const uint8_t*)qw_packed, sw, sw_cols,
                     (bf16_t*)y, ldy, (int)m, (int)n, (int)k, (int)tm, (int)tn, (float*)nullptr);
}

int64_t split_workspace(int64_t m, int64_t n, int64_t k) {
  const SplitPlan p = split_plan(m, n, k);
  if (p.s <= 1) return 0;
  return (m + p.bm - 1) / p.bm * (n / (4 * p.cw)) * p.s * p.bm * (4 * p.cw) * 4;
}

// The plain packed kernel at row tile BM x 4 CW with S k splits (S == 1: y directly).
template <int BM, int S, int CW = kSpCW>
void launch_split(const void* qa, const float* sa, int sa_rows, const void* qw_packed, const float* sw, int sw_cols,
                  void* y, int64_t ldy, int64_t m, int64_t n, int64_t k, void* part, hipStream_t st) {
  const int64_t tiles_m = (m + BM - 1) / BM, tiles_n = n / (4 * CW);
  // pk_mainloop_pf for 144 x 256 tiles split 4 ways (the 8B down projection at
  // 576 tokens) and 64 x 256 tiles split 4, 5 or 6 ways (o and down at 176
  // tokens; 5 and 6 deal their k steps out in pk_mainloop_pf's 2-step blocks).
  constexpr bool pf = (BM == 144 && CW == 64 && S == 4) || (BM == 64 && CW == 64 && S >= 4 && S <= 6);
  hipLaunchKernelGGL((gemm_fp8_split_packed_kernel<BM, CW, kSpP, kSpD, kSpG, S, pf>),
                     dim3((unsigned)(tiles_m * tiles_n * S)), dim3(kThreads), 0, st, (const uint8_t*)qa, sa, sa_rows,
                     (const uint8_t*)qw_packed, sw, sw_cols, (bf16_t*)y, ldy, (int)m, (int)n, (int)k, (int)tiles_m,
                     (int)tiles_n, (float*)part);
}

template <int BM, int CW = kSpCW>
void launch_splits(int s, const void* qa, const float* sa, int sa_rows, const void* qw_packed, const float* sw,
                   int sw_cols, void* y, int64_t ldy, int64_t m, int64_t n, int64_t k, void* part, hipStream_t st) {
  switch (s) {
    case 1: launch_split<BM, 1, CW>(qa, sa, sa_rows, qw_packed, sw, sw_cols, y, ldy, m, n, k, part, st); break;
    case 2: launch_split<BM, 2, CW>(qa, sa, sa_rows, qw_packed, sw, sw_cols, y, ldy, m, n, k, part, st); break;
    case 3: launch_split<BM, 3, CW>(qa, sa, sa_rows, qw_packed, sw, sw_cols, y, ldy, m, n, k, part, st); break;
    case 4: launch_split<BM, 4, CW>(qa, sa, sa_rows, qw_packed, sw, sw_cols, y, ldy, m, n, k, part, st); break;
    case 5: launch_split<BM, 5, CW>(qa, sa, sa_rows, qw_packed, sw, sw_cols, y, ldy, m, n, k, part, st); break;
    case 6: launch_split<BM, 6, CW>(qa, sa, sa_rows, qw_packed, sw, sw_cols, y, ldy, m, n, k, part, st); break;
    case 8: launch_split<BM, 8, CW>(qa, sa, sa_rows, qw_packed, sw, sw_cols, y, ldy, m, n, k, part, st); break;
    default: break;
  }
}

// The plan's tile: bm x 4 cw (bm 64 or 144 at cw = kSpCW; 64, 80, 96, 128 or 144 at cw = 32).
void launch_plan(const SplitPlan& p, int s, const void* qa, const float* sa, int sa_rows, const void* qw_packed,
                 const float* sw, int sw_cols, void* y, int64_t ldy, int64_t m, int64_t n, int64_t k, void* part,
                 hipStream_t st) {
  if (p.cw == 32) {
    if (p.bm == 64)
      launch_splits<64, 32>(s, qa, sa, sa_rows, qw_packed, sw, sw_cols, y, ldy, m, n, k, part, st);
    else if (p.bm == 80)
      launch_splits<80, 32>(s, qa, sa, sa_rows, qw_packed, sw, sw_cols, y, ldy, m, n, k, part, st);
    else if (p.bm == 96)
      launch_splits<96, 32>(s, qa, sa, sa_rows, qw_packed, sw, sw_cols, y, ldy, m, n, k, part, st);
    else if (p.bm == 128)
      launch_splits<128, 32>(s, qa, sa, sa_rows, qw_packed, sw, sw_cols, y, ldy, m, n, k, part, st);
    else
      launch_splits<kSpBM, 32>(s, qa, sa, sa_rows, qw_packed, sw, sw_cols, y, ldy, m, n, k, part, st);
  } else if (p.bm == 64) {
    launch_splits<64>(s, qa, sa, sa_rows, qw_packed, sw, sw_cols, y, ldy, m, n, k, part, st);
  } else {
    launch_splits<kSpBM>(s, qa, sa, sa_rows, qw_packed, sw, sw_cols, y, ldy, m, n, k, part, st);
  }
}

// Fused QKV on fragment-packed weights: BM tokens x BN = 4 CW channels (BN /
// 128 whole heads) per workgroup, the packed main loop at two workgroups per
// CU up to 96 rows (one above: 128 and 144 rows need the registers). The tile y = bf16((acc * sa) * sw) is written to LDS as a row-major
// bf16 tile (lane 16 g + r of fragment (i, j) holds token 16 i + r, columns
// wave CW + 16 j + 4 g .. + 3: one 8-byte store), then each head of the tile
// gets the epilogue of the row-major QKV kernel, the same code on the same
// bits: q/k heads the per-head RMSNorm + rotary (rope_row_pre, 16 lanes per
// token row) stored head-major, v heads stored transposed with zeros for the
// tokens in [M, t_pad).
struct PkQkv {
  const bf16_t* qn;  // q_norm weight (128)
  const bf16_t* kn;  // k_norm weight (128)
  float eps_q, eps_k;
  const bf16_t* cos;  // (M, 128)
  const bf16_t* sin;
  bf16_t* yq;  // (hq, M, 128)
  bf16_t* yk;  // (hk, M, 128)
  bf16_t* vt;  // (hk, 128, t_pad)
  int hq, hk, t_pad;
};

template <int BM, int CW, int P, int D, int G, bool PF = false>
__global__ __launch_bounds__(kThreads, BM <= 96 && !PF ? 2 : 1) void gemm_fp8_qkv_packed_kernel(
    const uint8_t* __restrict__ qa, const float* __restrict__ sa, int sa_rows, const uint8_t* __restrict__ qwp,
    const float* __restrict__ sw, int sw_cols, int M, int N, int K, int tiles_m, int tiles_n, PkQkv qe) {
  constexpr int BN = 4 * CW, RA = BM / 16, TJ = CW / 16;
  static_assert(BN % kHeadDim == 0, "whole heads per tile");
  constexpr int HPT = BN / kHeadDim;         // heads per tile
  constexpr int LD = BN + 8;                 // bf16 row pitch of the LDS tile
  constexpr int ROWS = BM / (kThreads / 16);  // token rows per 16-lane group
  constexpr int SMEM_LOOP = PF ? 2 * BM * 128 : pk_smem<BM, G>(), SMEM_TILE = BM * LD * 2;
  constexpr int SMEM = SMEM_LOOP > SMEM_TILE ? SMEM_LOOP : SMEM_TILE;
  static_assert(SMEM <= (BM <= 96 ? 80 : 160) * 1024, "two workgroups per CU up to 96 rows");
  __shared__ __align__(1024) uint8_t smem[SMEM];

  const int nblk = tiles_m * tiles_n;
  const int b = blockIdx.x;
  int logical = b;
  if (nblk % kXcds == 0) logical = (b % kXcds) * (nblk / kXcds) + b / kXcds;
  const int tm = logical % tiles_m, tn = logical / tiles_m;  // M fastest: L2 shares weights
  const int m0 = tm * BM, n0 = tn * BN;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int r16 = lane & 15, g = lane >> 4;
  const int KT = K / 128;

  const int wave_s = __builtin_amdgcn_readfirstlane(wave);
  uint32_t sB[TJ];
#pragma unroll
  for (int j = 0; j < TJ; ++j) sB[j] = (uint32_t)((n0 + wave_s * CW + 16 * j) / 16) * 2048u;
  f32x4 acc[RA][TJ];
  PkScales<RA, TJ> sc;
  sc.load(sa, sa_rows, sw, sw_cols, M, m0, n0 + wave_s * CW);
  if constexpr (PF)
    pk_mainloop_pf<BM, CW, P, D>(acc, smem, qa, M, K, m0, qwp, (uint32_t)N * (uint32_t)K, sB, 0, KT, [] {});
  else
    pk_mainloop<BM, CW, P, D, G>(acc, smem, qa, M, K, m0, qwp, (uint32_t)N * (uint32_t)K, sB, 0, KT, [] {});

  // The epilogue's global loads (norm weights, this thread's cos / sin rows)
  // are issued before the tile is staged.
  const int jr = tid & 15, grp = tid >> 4;
  float rope_w[HPT][8];
  u32x4 rope_c[ROWS], rope_s[ROWS];
#pragma unroll
  for (int hh = 0; hh < HPT; ++hh) {
    const int head = tn * HPT + hh;
    if (head < qe.hq + qe.hk) unpack8(*reinterpret_cast<const u32x4*>((head < qe.hq ? qe.qn : qe.kn) + 8 * jr), rope_w[hh]);
  }
#pragma unroll
  for (int p = 0; p < ROWS; ++p) {
    const int mm = min(m0 + grp + p * (kThreads / 16), M - 1);
    rope_c[p] = *reinterpret_cast<const u32x4*>(qe.cos + (size_t)mm * kHeadDim + 8 * jr);
    rope_s[p] = *reinterpret_cast<const u32x4*>(qe.sin + (size_t)mm * kHeadDim + 8 * jr);
  }

  __syncthreads();  // every wave's last activation-stage reads are done before the tile overwrites them
  bf16_t* tile = reinterpret_cast<bf16_t*>(smem);
  const float(&sav)[RA] = sc.sav;
#pragma unroll
  for (int j = 0; j < TJ; ++j) {
    const int col = wave * CW + 16 * j + 4 * g;
    const float(&swv)[4] = sc.swv[j];
#pragma unroll
    for (int i = 0; i < RA; ++i)
      *reinterpret_cast<u32x2*>(tile + (16 * i + r16) * LD + col) =
          pack4_bf16((acc[i][j][0] * sav[i]) * swv[0], (acc[i][j][1] * sav[i]) * swv[1],
                     (acc[i][j][2] * sav[i]) * swv[2], (acc[i][j][3] * sav[i]) * swv[3]);
  }
  __syncthreads();
#pragma unroll
  for (int hh = 0; hh < HPT; ++hh) {
    const int head = tn * HPT + hh;
    if (head < qe.hq + qe.hk) {
      const bool isq = head < qe.hq;
      const int hx = isq ? head : head - qe.hq;
      const float eps = isq ? qe.eps_q : qe.eps_k;
      bf16_t* dst = (isq ? qe.yq : qe.yk) + (size_t)hx * M * kHeadDim;
#pragma unroll
      for (int p = 0; p < ROWS; ++p) {
        const int rl = grp + p * (kThreads / 16);
        const int m = m0 + rl;
        const bool valid = m < M;
        const int mm = valid ? m : M - 1;
        rope_row_pre(tile + rl * LD + hh * kHeadDim, rope_w[hh], eps, rope_c[p], rope_s[p],
                     dst + (size_t)mm * kHeadDim, jr, valid);
      }
    } else {
      const int hv = head - qe.hq - qe.hk;
      for (int c = tid; c < kHeadDim * (BM / 8); c += kThreads) {
        const int d = c % kHeadDim, t0 = (c / kHeadDim) * 8;
        const int tok = m0 + t0;
        if (tok >= qe.t_pad) continue;
        float f[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) f[e] = (tok + e < M) ? bf16_to_f32(tile[(t0 + e) * LD + hh * kHeadDim + d]) : 0.f;
        *reinterpret_cast<u32x4*>(qe.vt + ((size_t)hv * kHeadDim + d) * qe.t_pad + tok) = pack8(f);
      }
    }
  }
}

// Fused QKV tile: 64 tokens x 256 channels (two heads).
constexpr int kQkBM = 64, kQkCW = 64;

// ---------------------------------------------------------------- unpacking
// The row-major (N, K) codes back from the fragment copy (the inverse of
// pack_fp8_kernel), for callers that read the codes themselves.
__global__ __launch_bounds__(kThreads) void unpack_fp8_kernel(const uint8_t* __restrict__ p, uint8_t* __restrict__ w,
                                                              int64_t n, int64_t k) {
  const int64_t kt_n = k / 128;
  const int64_t lanes = (n / 16) * kt_n * 64;
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < lanes; i += (int64_t)gridDim.x * blockDim.x) {
    const int l = (int)(i & 63);
    const int64_t f = i >> 6;
    const int64_t kt = f % kt_n, f16 = f / kt_n;
    const int64_t nf = n / 16;
    const int64_t row = f16 * 16 + (l & 15);
    const uint8_t* src = p + (kt * nf + f16) * 2048 + 16 * l;
    u32x4* dst = reinterpret_cast<u32x4*>(w + row * k + kt * 128 + 32 * (l >> 4));
    dst[0] = *reinterpret_cast<const u32x4*>(src);
    dst[1] = *reinterpret_cast<const u32x4*>(src + 1024);
  }
}

// ---------------------------------------------------------------- rows <= 4 on packed weights
//
// The pick-only tail's products (m <= 4 rows) straight from the fragment copy.
// Lane 16 g + r of a wave holds, for each k step kt, the 32 k bytes [128 kt +
// 32 g, +32) of row r of a 16-row fragment group (its two 16-byte pieces): it
// decodes them with v_cvt_pk_f32_fp8 and adds the exact products with the
// activations in fp32 FMAs; the four lane groups of a row are then added with
// row swaps. Plain product: one workgroup per 16-row group, its 4 waves taking
// every 4th k step and their sums added in wave order through LDS. SwiGLU: one
// workgroup per 64 channels, wave w the gate and up rows of channels 16 w ..
// + 15 over all k steps. The plain product issues a wave's loads of eight k
// steps before their products (each wave still adds its k steps in order, so
// the batch size does not change the sums).
constexpr int kGemvPkMaxM = 4;
constexpr int kGemvPkU = 8;  // k steps whose loads are in flight together

__device__ __forceinline__ void e4m3x16_to_f32(const u32x4 v, float* f) {
  const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const auto lo = __builtin_amdgcn_cvt_pk_f32_fp8((int)w[q], false);
    const auto hi = __builtin_amdgcn_cvt_pk_f32_fp8((int)w[q], true);
    f[4 * q + 0] = lo[0];
    f[4 * q + 1] = lo[1];
    f[4 * q + 2] = hi[0];
    f[4 * q + 3] = hi[1];
  }
}

// acc[m] += the products of this lane's 32 k bytes of step kt with rows m of qa,
// k in order, one 16-byte piece at a time.
template <int MM>
__device__ __forceinline__ void gemv_pk_step(const uint8_t* __restrict__ qa, int K, int kt, int g, const u32x4& wlo,
                                             const u32x4& whi, float (&acc)[MM]) {
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    float wf[16];
    e4m3x16_to_f32(h ? whi : wlo, wf);
#pragma unroll
    for (int m = 0; m < MM; ++m) {
      float af[16];
      e4m3x16_to_f32(*reinterpret_cast<const u32x4*>(qa + (size_t)m * K + 128 * kt + 32 * g + 16 * h), af);
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[m] = __builtin_fmaf(af[e], wf[e], acc[m]);
    }
  }
}

template <int MM>
__global__ __launch_bounds__(kThreads) void gemv_fp8_packed_kernel(const uint8_t* __restrict__ qa,
                                                                   const float* __restrict__ sa, int sa_rows,
                                                                   const uint8_t* __restrict__ qwp,
                                                                   const float* __restrict__ sw, int sw_cols,
                                                                   bf16_t* __restrict__ y, int64_t ldy, int N, int K) {
  __shared__ float red[4][MM][16];
  const int f = blockIdx.x, lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int r = lane & 15, g = lane >> 4;
  const int KT = K / 128, nf = N / 16;
  float acc[MM];
#pragma unroll
  for (int m = 0; m < MM; ++m) acc[m] = 0.f;
  for (int kb = wave; kb < KT; kb += 4 * kGemvPkU) {
    u32x4 lo[kGemvPkU], hi[kGemvPkU];
#pragma unroll
    for (int u = 0; u < kGemvPkU; ++u) {
      const int kt = min(kb + 4 * u, KT - 1);
      const uint8_t* src = qwp + ((size_t)kt * nf + f) * 2048 + 16 * lane;
      lo[u] = *reinterpret_cast<const u32x4*>(src);
      hi[u] = *reinterpret_cast<const u32x4*>(src + 1024);
    }
#pragma unroll
    for (int u = 0; u < kGemvPkU; ++u)
      if (kb + 4 * u < KT) gemv_pk_step<MM>(qa, K, kb + 4 * u, g, lo[u], hi[u], acc);
  }
#pragma unroll
  for (int m = 0; m < MM; ++m) {
    const float v = sum_rows(acc[m]);
    if (g == 0) red[wave][m][r] = v;
  }
  __syncthreads();
  if (wave == 0 && g == 0) {
    const int n = 16 * f + r;
    const float swv = sw[sw_cols ? n : 0];
#pragma unroll
    for (int m = 0; m < MM; ++m) {
      const float tot = ((red[0][m][r] + red[1][m][r]) + red[2][m][r]) + red[3][m][r];
      y[(size_t)m * ldy + n] = (bf16_t)f32_to_bf16((tot * sa[sa_rows ? m : 0]) * swv);
    }
  }
}

// SwiGLU: h = bf16(bf16(silu(g)) * u) for the 64 channels of workgroup
// blockIdx.x, g and u = bf16((dot * sa) * sw) of gate row c and up row half + c,
// and the workgroup's max |h| into pmax[m, blockIdx.x] (the 64-channel row
// maxima of the tile kernels); SQ: h written as e4m3(clamp(h * qinv, +-448))
// into hq instead, without maxima. 16 waves: wave 4 j + w takes channels
// 16 j .. + 15 over the k steps kt = w mod 4, and the four k phases are added in
// order through LDS, so g and u are the bits of the plain kernel above on the
// same rows.
template <int MM, bool SQ>
__global__ __launch_bounds__(1024) void gemv_fp8_swiglu_packed_kernel(
    const uint8_t* __restrict__ qa, const float* __restrict__ sa, int sa_rows, const uint8_t* __restrict__ qwp,
    const float* __restrict__ sw, int sw_cols, bf16_t* __restrict__ h, int64_t ldh, float* __restrict__ pmax,
    uint8_t* __restrict__ hq, float qinv, int half, int K) {
  __shared__ float red[2][4][4][MM][16];  // [gate / up][channel group][k phase][row][channel]
  __shared__ float hmax[4][MM];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int r = lane & 15, g = lane >> 4;
  const int grp = wave >> 2, ph = wave & 3;
  const int KT = K / 128, nf = 2 * half / 16;
  const int c0 = 64 * (int)blockIdx.x + 16 * grp;  // first channel of this wave's group
  const int fg = c0 / 16, fu = (half + c0) / 16;
  float ag[MM], au[MM];
#pragma unroll
  for (int m = 0; m < MM; ++m) ag[m] = au[m] = 0.f;
  constexpr int U = 2;  // 16 waves per workgroup: 128 registers each
  for (int kb = ph; kb < KT; kb += 4 * U) {
    u32x4 glo[U], ghi[U], ulo[U], uhi[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int kt = min(kb + 4 * u, KT - 1);
      const uint8_t* sg = qwp + ((size_t)kt * nf + fg) * 2048 + 16 * lane;
      const uint8_t* su = qwp + ((size_t)kt * nf + fu) * 2048 + 16 * lane;
      glo[u] = *reinterpret_cast<const u32x4*>(sg);
      ghi[u] = *reinterpret_cast<const u32x4*>(sg + 1024);
      ulo[u] = *reinterpret_cast<const u32x4*>(su);
      uhi[u] = *reinterpret_cast<const u32x4*>(su + 1024);
    }
#pragma unroll
    for (int u = 0; u < U; ++u)
      if (kb + 4 * u < KT) {
        gemv_pk_step<MM>(qa, K, kb + 4 * u, g, glo[u], ghi[u], ag);
        gemv_pk_step<MM>(qa, K, kb + 4 * u, g, ulo[u], uhi[u], au);
      }
  }
#pragma unroll
  for (int m = 0; m < MM; ++m) {
    const float vg = sum_rows(ag[m]), vu = sum_rows(au[m]);
    if (g == 0) {
      red[0][grp][ph][m][r] = vg;
      red[1][grp][ph][m][r] = vu;
    }
  }
  __syncthreads();
  if (ph == 0) {  // waves 0, 4, 8, 12: one channel group each
    const int c = c0 + r;
    const float swg = sw[sw_cols ? c : 0], swu = sw[sw_cols ? half + c : 0];
#pragma unroll
    for (int m = 0; m < MM; ++m) {
      const float sav = sa[sa_rows ? m : 0];
      const float tg = ((red[0][grp][0][m][r] + red[0][grp][1][m][r]) + red[0][grp][2][m][r]) + red[0][grp][3][m][r];
      const float tu = ((red[1][grp][0][m][r] + red[1][grp][1][m][r]) + red[1][grp][2][m][r]) + red[1][grp][3][m][r];
      const float gv = round_bf16((tg * sav) * swg);
      const float uv = round_bf16((tu * sav) * swu);
      const float hv = round_bf16(round_bf16(silu(gv)) * uv);
      if constexpr (SQ) {
        if (g == 0) hq[(size_t)m * ldh + c] = (uint8_t)(e4m3x4(clamp448(hv * qinv), 0.f, 0.f, 0.f) & 0xFFu);
      } else {
        if (g == 0) h[(size_t)m * ldh + c] = (bf16_t)f32_to_bf16(hv);
        float mx = fabsf(hv);
        mx = fmaxf(mx, dpp<kDppXor1>(mx));
        mx = fmaxf(mx, dpp<kDppXor2>(mx));
        mx = fmaxf(mx, dpp<kDppHalfMirror>(mx));
        mx = fmaxf(mx, dpp<kDppRowMirror>(mx));
        if (lane == 0) hmax[grp][m] = mx;
      }
    }
  }
  if constexpr (SQ) return;
  __syncthreads();
  if (threadIdx.x < MM) {
    const int m = threadIdx.x;
    pmax[(size_t)m * (half / 64) + blockIdx.x] = fmaxf(fmaxf(hmax[0][m], hmax[1][m]), fmaxf(hmax[2][m], hmax[3][m]));
  }
}

// Launch the packed single-row kernels for m in 1..4.
void launch_gemv_pk(const void* qa, const float* sa, int sa_rows, const void* qwp, const float* sw, int sw_cols,
                    void* y, int64_t ldy, int64_t m, int64_t n, int64_t k, hipStream_t s) {
#define FF_GEMVPK(MM)                                                                                       \
  case MM:                                                                                                  \
    hipLaunchKernelGGL(gemv_fp8_packed_kernel<MM>, dim3((unsigned)(n / 16)), dim3(kThreads), 0, s,         \
                       (const uint8_t*)qa, sa, sa_rows, (const uint8_t*)qwp, sw, sw_cols, (bf16_t*)y, ldy,   \
                       (int)n, (int)k);                                                                     \
    break;
  switch (m) { FF_GEMVPK(1) FF_GEMVPK(2) FF_GEMVPK(3) FF_GEMVPK(4) }
#undef FF_GEMVPK
}

template <bool SQ>
void launch_gemv_swiglu_pk(const void* qa, const float* sa, int sa_rows, const void* qwp, const float* sw,
                           int sw_cols, void* h, int64_t ldh, float* pmax, void* hq, float qinv, int64_t m, int64_t i,
                           int64_t k, hipStream_t s) {
#define FF_GEMVSPK(MM)                                                                                      \
  case MM:                                                                                                  \
    hipLaunchKernelGGL((gemv_fp8_swiglu_packed_kernel<MM, SQ>), dim3((unsigned)(i / 64)), dim3(1024), 0,    \
                       s, (const uint8_t*)qa, sa, sa_rows, (const uint8_t*)qwp, sw, sw_cols, (bf16_t*)h, ldh, pmax, \
                       (uint8_t*)hq, qinv, (int)i, (int)k);                                                 \
    break;
  switch (m) { FF_GEMVSPK(1) FF_GEMVSPK(2) FF_GEMVSPK(3) FF_GEMVSPK(4) }
#undef FF_GEMVSPK
}

}  // namespace

extern "C" int ff_pack_weight_fp8(const void* w, void* packed, int64_t n, int64_t k, ff_stream_t stream) {
  FF_REQUIRE(w && packed, "ff_pack_weight_fp8: null pointer");
  FF_REQUIRE(n > 0 && n % 16 == 0 && k > 0 && k % 128 == 0 && n * k < (int64_t(1) << 40),
             "ff_pack_weight_fp8: bad sizes (n %% 16, k %% 128)");
  FF_REQUIRE(ff_aligned(w, 16) && ff_aligned(packed, 16), "ff_pack_weight_fp8: alignment");
  const int64_t lanes = (n / 16) * (k / 128) * 64;
  const int64_t blocks = (lanes + kThreads - 1) / kThreads;
  hipLaunchKernelGGL(pack_fp8_kernel, dim3((unsigned)(blocks < 65536 ? blocks : 65536)), dim3(kThreads), 0,
                     (hipStream_t)stream, (const uint8_t*)w, (uint8_t*)packed, n, k);
  FF_LAUNCH_CHECK("ff_pack_weight_fp8");
  return FF_OK;
}

extern "C" int ff_unpack_weight_fp8(const void* packed, void* w, int64_t n, int64_t k, ff_stream_t stream) {
  FF_REQUIRE(w && packed, "ff_unpack_weight_fp8: null pointer");
  FF_REQUIRE(n > 0 && n % 16 == 0 && k > 0 && k % 128 == 0 && n * k < (int64_t(1) << 40),
             "ff_unpack_weight_fp8: bad sizes (n %% 16, k %% 128)");
  FF_REQUIRE(ff_aligned(w, 16) && ff_aligned(packed, 16), "ff_unpack_weight_fp8: alignment");
  const int64_t lanes = (n / 16) * (k / 128) * 64;
  const int64_t blocks = (lanes + kThreads - 1) / kThreads;
  hipLaunchKernelGGL(unpack_fp8_kernel, dim3((unsigned)(blocks < 65536 ? blocks : 65536)), dim3(kThreads), 0,
                     (hipStream_t)stream, (const uint8_t*)packed, (uint8_t*)w, n, k);
  FF_LAUNCH_CHECK("ff_unpack_weight_fp8");
  return FF_OK;
}

extern "C" int ff_gemm_fp8_swiglu_pk(const void* qa, const float* sa, const void* qw, const void* qw_packed,
                                     const float* sw, void* h, int64_t ldh, float* pmax, int64_t m, int64_t i,
                                     int64_t k, ff_stream_t stream) {
  FF_REQUIRE(qa && sa && (qw || qw_packed) && sw && h && pmax, "ff_gemm_fp8_swiglu_pk: null pointer");
  int cw = swiglu_cw(m, i);
  int bm = cw ? swiglu_bm(m, i / (2 * cw), cw) : 0;
  const bool aligned = qw_packed && k % kPkKAlign == 0 && i % 64 == 0 && ldh % 8 == 0 && ldh >= i &&
                       m * k < (int64_t(1) << 31) && 2 * i * k < (int64_t(1) << 31) && ff_aligned(qa, 16) &&
                       ff_aligned(qw_packed, 16) && ff_aligned(h, 16);
  if (!qw) {
    // only the packed copy: the single-row kernel for m <= 4, else a packed tile whatever its grid
    FF_REQUIRE(aligned, "ff_gemm_fp8_swiglu_pk: without the row-major weight, i %% 64, k %% %d, ldh %% 8 and "
                        "16-byte alignment", kPkKAlign);
    if (m == 0) return FF_OK;
    if (m <= kGemvPkMaxM) {
      launch_gemv_swiglu_pk<false>(qa, sa, 1, qw_packed, sw, 1, h, ldh, pmax, nullptr, 0.f, m, i, k,
                                   (hipStream_t)stream);
      FF_LAUNCH_CHECK("ff_gemm_fp8_swiglu_pk");
      return FF_OK;
    }
    if (!bm) swiglu_any_tile(m, i, &cw, &bm);
  }
  const bool packed_fits = aligned && bm && m > 4;
  if (!packed_fits) return ff_gemm_fp8_swiglu(qa, sa, qw, sw, h, ldh, pmax, m, i, k, stream);
  const int64_t tiles_n = i / (2 * cw), tiles_m = (m + bm - 1) / bm;
  bool launched = false;
  // The 144 x 384 (576 tokens) and 176 x 128 (176 tokens) tiles on pk_mainloop_pf.
#define FF_SWIGLU(BM, CW)                                                                                           \
  if (bm == BM && cw == CW && (launched = true))                                                                    \
    hipLaunchKernelGGL((gemm_fp8_swiglu_packed_kernel<BM, CW, kPkP, kPkD, kPkG, false,                              \
                                                      (BM == 144 && CW == 96) || (BM == 176 && CW == 32)>),         \
                       dim3((unsigned)(tiles_m * tiles_n)), dim3(kThreads), 0, (hipStream_t)stream,                 \
                       (const uint8_t*)qa, sa, (const uint8_t*)qw_packed, sw, (bf16_t*)h, ldh, pmax, (int)m,        \
                       (int)i, (int)k, (int)tiles_m, (int)tiles_n, nullptr, 0.f);
  FF_SWIGLU(144, 96) FF_SWIGLU(128, 96) FF_SWIGLU(112, 96) FF_SWIGLU(96, 96) FF_SWIGLU(80, 96)
  FF_SWIGLU(144, 64) FF_SWIGLU(128, 64) FF_SWIGLU(112, 64) FF_SWIGLU(96, 64) FF_SWIGLU(80, 64)
  FF_SWIGLU(176, 32) FF_SWIGLU(144, 32) FF_SWIGLU(112, 32) FF_SWIGLU(80, 32) FF_SWIGLU(64, 32)
#undef FF_SWIGLU
  FF_REQUIRE(launched, "ff_gemm_fp8_swiglu_pk: no %d x %d tile (tuning override)", bm, 8 * cw);
  FF_LAUNCH_CHECK("ff_gemm_fp8_swiglu_pk");
  return FF_OK;
}

extern "C" int ff_gemm_fp8_swiglu_static(const void* qa, const float* sa, const void* qw, const void* qw_packed,
                                         const float* sw, void* hq, int64_t ldh, float inv, int64_t m, int64_t i,
                                         int64_t k, ff_stream_t stream) {
  FF_REQUIRE(qa && sa && (qw || qw_packed) && sw && hq, "ff_gemm_fp8_swiglu_static: null pointer");
  FF_REQUIRE(m >= 0 && i > 0 && i % 64 == 0 && k > 0 && k % 128 == 0 && ldh >= i && ldh % 8 == 0 &&
                 m < (1 << 30) && i < (1 << 29) && k < (1 << 30),
             "ff_gemm_fp8_swiglu_static: bad sizes (i %% 64, k %% 128, ldh %% 8)");
  FF_REQUIRE(ff_aligned(qa, 16) && ff_aligned(qw ? qw : qw_packed, 16) && ff_aligned(hq, 16),
             "ff_gemm_fp8_swiglu_static: operands must be 16-byte aligned");
  int cw = swiglu_cw(m, i);
  int bm = cw ? swiglu_bm(m, i / (2 * cw), cw) : 0;
  const bool aligned = qw_packed && k % kPkKAlign == 0 && m * k < (int64_t(1) << 31) &&
                       2 * i * k < (int64_t(1) << 31) && ff_aligned(qw_packed, 16);
  if (!qw) {
    FF_REQUIRE(aligned, "ff_gemm_fp8_swiglu_static: without the row-major weight, k %% %d and 16-byte alignment",
               kPkKAlign);
    if (m == 0) return FF_OK;
    if (m <= kGemvPkMaxM) {
      launch_gemv_swiglu_pk<true>(qa, sa, 0, qw_packed, sw, 0, nullptr, ldh, nullptr, hq, inv, m, i, k,
                                  (hipStream_t)stream);
      FF_LAUNCH_CHECK("ff_gemm_fp8_swiglu_static");
      return FF_OK;
    }
    if (!bm) swiglu_any_tile(m, i, &cw, &bm);
  }
  const bool packed_fits = aligned && bm && m > 4;
  if (!packed_fits) return gemm_swiglu_static_rowmajor(qa, sa, qw, sw, hq, ldh, inv, m, i, k, (hipStream_t)stream);
  const int64_t tiles_n = i / (2 * cw), tiles_m = (m + bm - 1) / bm;
  bool launched = false;
#define FF_SWIGLU(BM, CW)                                                                                           \
  if (bm == BM && cw == CW && (launched = true))                                                                    \
    hipLaunchKernelGGL((gemm_fp8_swiglu_packed_kernel<BM, CW, kPkP, kPkD, kPkG, true>),                             \
                       dim3((unsigned)(tiles_m * tiles_n)), dim3(kThreads), 0, (hipStream_t)stream,                 \
                       (const uint8_t*)qa, sa, (const uint8_t*)qw_packed, sw, nullptr, ldh, nullptr, (int)m, (int)i, \
                       (int)k, (int)tiles_m, (int)tiles_n, (uint8_t*)hq, inv);
  FF_SWIGLU(144, 96) FF_SWIGLU(128, 96) FF_SWIGLU(112, 96) FF_SWIGLU(96, 96) FF_SWIGLU(80, 96)
  FF_SWIGLU(144, 64) FF_SWIGLU(128, 64) FF_SWIGLU(112, 64) FF_SWIGLU(96, 64) FF_SWIGLU(80, 64)
  FF_SWIGLU(176, 32) FF_SWIGLU(144, 32) FF_SWIGLU(112, 32) FF_SWIGLU(80, 32) FF_SWIGLU(64, 32)
#undef FF_SWIGLU
  FF_REQUIRE(launched, "ff_gemm_fp8_swiglu_static: no %d x %d tile (tuning override)", bm, 8 * cw);
  FF_LAUNCH_CHECK("ff_gemm_fp8_swiglu_static");
  return FF_OK;
}

extern "C" int ff_gemm_fp8_pk_workspace(int64_t m, int64_t n, int64_t k, int64_t* bytes) {
  FF_REQUIRE(bytes && m >= 0 && n >= 0 && k >= 0, "ff_gemm_fp8_pk_workspace: bad arguments");
  *bytes = split_workspace(m, n, k);
  return FF_OK;
}

namespace ff {
int gemm_fp8_pk_partials(const void* qa, const float* sa, int sa_rows, const void* qw_packed, const float* sw,
                         int sw_cols, int64_t m, int64_t n, int64_t k, void* workspace, int64_t workspace_bytes,
                         hipStream_t st, int* splits, int64_t* mp) {
  *splits = 0;
  *mp = 0;
  const SplitPlan p = qw_packed && ff_aligned(qa, 16) && ff_aligned(qw_packed, 16) ? split_plan(m, n, k) : SplitPlan{};
  const int s = p.s;
  if (s <= 1) return FF_OK;
  const int64_t need = split_workspace(m, n, k);
  FF_REQUIRE(workspace && workspace_bytes >= need && ff_aligned(workspace, 16),
             "ff_gemm_fp8_pk: workspace of %lld bytes (16-byte aligned) required", (long long)need);
  launch_plan(p, s, qa, sa, sa_rows, qw_packed, sw, sw_cols, nullptr, 0, m, n, k, workspace, st);
  FF_LAUNCH_CHECK("ff_gemm_fp8_pk");
  *splits = s;
  *mp = (m + p.bm - 1) / p.bm * p.bm;
  return FF_OK;
}
}  // namespace ff

extern "C" int ff_gemm_fp8_pk(const void* qa, const float* sa, int sa_rows, const void* qw, const void* qw_packed,
                              const float* sw, int sw_cols, void* y, int64_t ldy, int64_t m, int64_t n, int64_t k,
                              void* workspace, int64_t workspace_bytes, ff_stream_t stream) {
  FF_REQUIRE(qa && sa && (qw || qw_packed) && sw && y, "ff_gemm_fp8_pk: null pointer");
  const bool pk = qw_packed && ldy % 8 == 0 && ldy >= n && ff_aligned(qa, 16) && ff_aligned(qw_packed, 16) &&
                  ff_aligned(y, 16);
  hipStream_t st = (hipStream_t)stream;
  if (!qw) {
    // only the packed copy: every shape runs on it (the single-row kernels for m <= 4)
    FF_REQUIRE(pk && n % 16 == 0 && k % 128 == 0 && n * k < (int64_t(1) << 31),
               "ff_gemm_fp8_pk: without the row-major weight, n %% 16, k %% 128, ldy %% 8 and 16-byte alignment");
    if (m == 0) return FF_OK;
    if (m <= kGemvPkMaxM) {
      launch_gemv_pk(qa, sa, sa_rows, qw_packed, sw, sw_cols, y, ldy, m, n, k, st);
      FF_LAUNCH_CHECK("ff_gemm_fp8_pk");
      return FF_OK;
    }
  }
  const SplitPlan plan = pk ? split_plan(m, n, k) : SplitPlan{};
  const int s = plan.s;
  if (s == 0) {
    const SmallTile t = pk ? small_plan(m, n, k, !qw) : SmallTile{};
    if (t.bm == 64 && t.cw == 64)
      launch_small<64, 64>(qa, sa, sa_rows, qw_packed, sw, sw_cols, y, ldy, m, n, k, st);
    else if (t.bm == 80)
      launch_small<80, 32>(qa, sa, sa_rows, qw_packed, sw, sw_cols, y, ldy, m, n, k, st);
    else if (t.bm == 96)
      launch_small<96, 32>(qa, sa, sa_rows, qw_packed, sw, sw_cols, y, ldy, m, n, k, st);
    else if (t.bm == 64)
      launch_small<64, 32>(qa, sa, sa_rows, qw_packed, sw, sw_cols, y, ldy, m, n, k, st);
    else if (qw)
      return ff_gemm_fp8(qa, sa, sa_rows, qw, sw, sw_cols, y, ldy, m, n, k, stream);
    else
      FF_REQUIRE(false, "ff_gemm_fp8_pk: %lld x %lld x %lld needs the row-major weight (n %% 128, k %% 512)",
                 (long long)m, (long long)n, (long long)k);
    FF_LAUNCH_CHECK("ff_gemm_fp8_pk");
    return FF_OK;
  }
  if (s == 1) {
    launch_plan(plan, 1, qa, sa, sa_rows, qw_packed, sw, sw_cols, y, ldy, m, n, k, nullptr, st);
    FF_LAUNCH_CHECK("ff_gemm_fp8_pk");
    return FF_OK;
  }
  int splits = 0;
  int64_t mp = 0;
  const int rc = ff::gemm_fp8_pk_partials(qa, sa, sa_rows, qw_packed, sw, sw_cols, m, n, k, workspace,
                                          workspace_bytes, st, &splits, &mp);
  if (rc) return rc;
  const int64_t chunks = m * (n / 8);
  const dim3 rgrid((unsigned)((chunks + kThreads - 1) / kThreads));
#define FF_REDUCE(S)                                                                                                \
  if (splits == S)                                                                                                  \
    hipLaunchKernelGGL((split_reduce_kernel<S>), rgrid, dim3(kThreads), 0, st, (const float*)workspace, mp, sa,     \
                       sa_rows, sw, sw_cols, (bf16_t*)y, ldy, (int)m, (int)n);
  FF_REDUCE(2) FF_REDUCE(3) FF_REDUCE(4) FF_REDUCE(5) FF_REDUCE(6) FF_REDUCE(8)
#undef FF_REDUCE
  FF_LAUNCH_CHECK("ff_gemm_fp8_pk");
  return FF_OK;
}

extern "C" int ff_gemm_fp8_qkv_pk(const void* qa, const float* sa, int sa_rows, const void* qw, const void* qw_packed,
                                  const float* sw, int sw_cols, int64_t m, int64_t k, int64_t hq, int64_t hk,
                                  const void* q_norm, const void* k_norm, float eps_q, float eps_k, const void* cos,
                                  const void* sin, void* yq, void* yk, void* vt, int64_t t_pad, ff_stream_t stream) {
  const int64_t n = (hq + 2 * hk) * kHeadDim;
  // ff_set_tuning(FF_TUNE_QKV_PK_TILE, 1 | 2 | 3 | 4 | 5 | 6): 64 x 256 packed tiles, 64 x 128 packed
  // tiles, the row-major kernel, 96 x 128, 144 x 128, 128 x 128 packed tiles, for measurement sweeps.
  // The library's choice: one-head tiles (128 columns) of the fewest rows among 64, 96 and 128 whose
  // grid fits one round of one workgroup per CU (256 workgroups; 8B shape: 176 tokens 64 rows, 144
  // workgroups, 4.467 -> 4.393 ms against the row-major kernel; 576 tokens 128 rows, 240 workgroups,
  // 29.1 -> 25.3 us per launch and 6.202 -> 6.118 ms per step against 64 rows at two workgroups per
  // CU, 96 rows 28.0 us, 144 rows 27.6 us); else 64 x 128 while the grid is at most 512 workgroups
  // (two per CU), else 64 x 256.
  const int forced = ff_tuning(FF_TUNE_QKV_PK_TILE);
  int bm = forced == 4 ? 96 : forced == 5 ? 144 : forced == 6 ? 128 : kQkBM;
  if (!forced) {
    for (const int c : {64, 96, 128}) {
      const int64_t tm = (m + c - 1) / c;
      if (tm * (n / 128) <= 256 && t_pad <= tm * c) {
        bm = c;
        break;
      }
    }
  }
  const int64_t tiles_m = (m + bm - 1) / bm;
  const int cw = forced >= 4 || forced == 2 || bm != kQkBM || (!forced && tiles_m * (n / 128) <= 512) ? 32 : kQkCW;
  const int64_t tiles_n = n / (4 * cw), tiles = tiles_m * tiles_n;
  const bool fits = forced != 3 && qw_packed && (m > 4 || !qw) && m > 0 && hq > 0 && hk > 0 && hq % hk == 0 &&
                    n % (4 * cw) == 0 && k > 0 && k % (128 * kSpU) == 0 &&
                    (forced || cw == 32 || !qw || (tiles >= 192 && tiles <= 512)) && t_pad >= m &&
                    t_pad % 64 == 0 &&
                    t_pad <= tiles_m * bm && m * k < (int64_t(1) << 31) && n * k < (int64_t(1) << 31) &&
                    ff_aligned(qa, 16) && ff_aligned(qw_packed, 16) && ff_aligned(cos, 16) && ff_aligned(sin, 16) &&
                    ff_aligned(q_norm, 16) && ff_aligned(k_norm, 16) && ff_aligned(yq, 16) && ff_aligned(yk, 16) &&
                    ff_aligned(vt, 16);
  if (!fits) {
    FF_REQUIRE(qw, "ff_gemm_fp8_qkv_pk: this shape needs the row-major weight (k %% %d, 16-byte alignment)",
               128 * kSpU);
    return ff_gemm_fp8_qkv(qa, sa, sa_rows, qw, sw, sw_cols, m, k, hq, hk, q_norm, k_norm, eps_q, eps_k, cos, sin, yq,
                           yk, vt, t_pad, stream);
  }
  FF_REQUIRE(sa && sw && q_norm && k_norm && yq && yk && vt, "ff_gemm_fp8_qkv_pk: null pointer");
  PkQkv qe{(const bf16_t*)q_norm, (const bf16_t*)k_norm, eps_q, eps_k, (const bf16_t*)cos, (const bf16_t*)sin,
           (bf16_t*)yq, (bf16_t*)yk, (bf16_t*)vt, (int)hq, (int)hk, (int)t_pad};
  // The 128 x 128 tile (576 tokens) on pk_mainloop_pf.
#define FF_QKV_BM(BM, PF)                                                                                     \
  if (bm == BM)                                                                                               \
    hipLaunchKernelGGL((gemm_fp8_qkv_packed_kernel<BM, 32, kSpP, kSpD, kSpG, PF>),                            \
                       dim3((unsigned)tiles), dim3(kThreads), 0, (hipStream_t)stream, (const uint8_t*)qa, sa, \
                       sa_rows, (const uint8_t*)qw_packed, sw, sw_cols, (int)m, (int)n, (int)k, (int)tiles_m, \
                       (int)tiles_n, qe);
  if (bm != kQkBM) {
    FF_QKV_BM(96, false) FF_QKV_BM(144, false) FF_QKV_BM(128, true)
  } else if (cw == 32)  // 64 x 128 (176 tokens) on pk_mainloop_pf
    hipLaunchKernelGGL((gemm_fp8_qkv_packed_kernel<kQkBM, 32, kSpP, kSpD, kSpG, true>), dim3((unsigned)tiles),
                       dim3(kThreads), 0, (hipStream_t)stream, (const uint8_t*)qa, sa, sa_rows,
                       (const uint8_t*)qw_packed, sw, sw_cols, (int)m, (int)n, (int)k, (int)tiles_m, (int)tiles_n, qe);
  else
    hipLaunchKernelGGL((gemm_fp8_qkv_packed_kernel<kQkBM, kQkCW, kSpP, kSpD, kSpG>), dim3((unsigned)tiles),
                       dim3(kThreads), 0, (hipStream_t)stream, (const uint8_t*)qa, sa, sa_rows,
                       (const uint8_t*)qw_packed, sw, sw_cols, (int)m, (int)n, (int)k, (int)tiles_m, (int)tiles_n, qe);
#undef FF_QKV_BM
  FF_LAUNCH_CHECK("ff_gemm_fp8_qkv_pk");
  return FF_OK;
}
