// moe_gemm.hip - grouped INT4 expert GEMM for prefill (bf16 MFMA).
//
// Same arithmetic as the decode kernel (moe_expert.hip): weights become bf16
// 136 + q with one AND-OR per pair, every 128-wide group accumulates from
// -136 * sum_{k in g} a[m][k] and the group's scale is applied with one fp32
// fma per output, so the result is sum_g s_g * sum_{k in g} q * a.
// Restates the reference's INT4 GEMM (ChunkGemm, tools/cmdlist/kernels.cpp:
// 691-785; gemmMT4, tools/prefill/prefill.cpp:46-129) for bf16 MFMA.
//
// Block tile: 128 tokens (one expert tile of the dispatch) x 64 * GEMM_WN
// weight rows (GEMM_WN = 4: MODE 0 takes 128 gate rows and the matching 128
// up rows, MODE 1 256 down rows), K in 128-wide groups.  2 x GEMM_WN waves
// as 2 (tokens) x GEMM_WN (rows); a wave owns 64 x 64 = 4 x 4 tiles of
// v_mfma_f32_16x16x32_bf16.  Token subtiles past the tile's count skip
// their MFMAs and A reads.
//
// Data movement: a 3-stage LDS ring per block (2 stages where K > 2048
// leaves no room), one barrier per group.  Each
// stage holds one group of the token rows (128 x 256 B, already in MFMA
// order) and of the raw INT4 weight rows (64 B each).  Both arrive by
// global->LDS DMA (global_load_lds_dwordx4: lane i of a wave lands at
// M0 + 16 i), two groups ahead of the math, with no staging registers.  The
// DMA is issued from inline asm and its completion tracked with explicit
// vmcnt waits, so the compiler's conservative waits do not serialise the
// ring.  Rows are swizzled in 16-byte chunks (A: chunk c of row r at
// c ^ aswz(r); B: chunk q at q ^ bswz(r)) so that the lanes reading 16 rows
// at one column hit distinct bank groups.  Scales and the group sums
// sum_{k in g} a (for x from k_select, for act from this kernel's MODE 0
// epilogue) are copied to LDS once per block.
#include <type_traits>

#include "moe_common.h"
#include "moe_internal.h"

#ifdef AINFER_GEMM_TRACE
// diagnostic builds only: per item (MODE * 16384 + item), the shader clock
// (s_memtime) at the item's start, before its main loop, after the loop's
// last barrier, and after its epilogue
__device__ unsigned long long g_gtrace[2 * 16384 * 4];
#define GTRACE(V) V
extern "C" int ainfer_debug_gemm_trace(void *host) {
  return hipMemcpyFromSymbol(host, HIP_SYMBOL(g_gtrace), sizeof(g_gtrace)) == hipSuccess ? 0 : -1;
}
#else
#define GTRACE(V)
#endif

namespace {

constexpr int BM = 128;  // tokens per tile

// Block geometry: 2 x WN waves; BN = 64 * WN weight rows per block.
template <int WN, int STAGES_>
struct Geo {
  static constexpr int NW = 2 * WN;                  // waves
  static constexpr int THREADS = 64 * NW;
  static constexpr int BN = 64 * WN;                 // weight rows
  static constexpr int STAGES = STAGES_;
  static constexpr int A_STAGE = BM * 256;           // bytes per group
  static constexpr int B_STAGE = BN * 64;            // bytes per group
  static constexpr int STAGE = A_STAGE + B_STAGE;
  static constexpr int A_DMA = A_STAGE / (THREADS * 16);  // DMA per thread per stage
  static constexpr int B_DMA = B_STAGE / (THREADS * 16);
  static constexpr int DMA = A_DMA + B_DMA;
  static constexpr int COLS = 32 * WN;               // MODE 0: act columns per block
};

__device__ __forceinline__ void dma16(const void *g, uint32_t lds_addr) {
  asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off"
               :
               : "v"(g), "s"(lds_addr)
               : "memory", "m0");
}

// The same with a scalar base address and a 32-bit per-lane offset.  The
// base must be wave-uniform; it is moved to SGPRs explicitly, since the
// compiler cannot always prove the uniformity of values loaded per item.
__device__ __forceinline__ void dma16s(uint32_t off, const void *base, uint32_t lds_addr) {
  const uint64_t b = (uint64_t)(uintptr_t)base;
  const uint64_t sb = (uint64_t)(uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)b) |
                      ((uint64_t)(uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)(b >> 32)) << 32);
  asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, %1"
               :
               : "v"(off), "s"(sb), "s"(lds_addr)
               : "memory", "m0");
}

template <int N>
__device__ __forceinline__ void wait_vm() {
  asm volatile("s_waitcnt vmcnt(%0)" : : "n"(N) : "memory");
}

// Every LDS read this wave issued completes before the barrier: s_barrier
// alone does not wait for them, and the compiler is free to place the
// lgkmcnt wait of a fragment read after the barrier (with the MFMA that uses
// it).  A wave past the barrier may then refill that ring stage by DMA while
// the read is still queued.  (Without this wait the router GEMM below read a
// refilled stage now and then: wrong approximate logits, wrong top-k.)
__device__ __forceinline__ void block_barrier() {
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// A chunk swizzle: logical 16-byte chunk c of token row r sits at
// c ^ aswz(r), the 2-bit halves of r & 15 swapped.  The 16 rows that one
// fragment read touches at one logical chunk then spread over all 8
// 16-byte bank groups in each pair of k-quarter lanes (measured: 77% fewer
// LDS bank-conflict cycles than c ^ r).
__device__ __forceinline__ int aswz(int r) { return ((r & 3) << 2) | ((r >> 2) & 3); }

// B chunk swizzle: 2-bit function of the row such that 8 consecutive rows
// (32 banks x 4 B) and 16 consecutive rows (64 banks) both land the 16-byte
// chunks of one logical column in distinct bank groups.
__device__ __forceinline__ int bswz(int r) {
  return (((r >> 1) ^ (r >> 3)) & 1) | (((r >> 2) & 1) << 1);
}

__device__ __forceinline__ u32x4 nib_slice3(u32x4 b, int j, uint32_t magic) {
  const uint32_t mask = 0x000F000Fu;
  return u32x4{((b[0] >> (4 * j)) & mask) | magic, ((b[1] >> (4 * j)) & mask) | magic,
               ((b[2] >> (4 * j)) & mask) | magic, ((b[3] >> (4 * j)) & mask) | magic};
}

// silu(g) * u for the prefill epilogue: the hardware exp2 and reciprocal
// (about 1 ulp each) instead of expf and an IEEE division, which made the
// epilogue several times longer than a group of the main loop.  The result is
// rounded to bf16 (2^-9 relative) right after.  Large |g| behaves: exp2 -> inf
// gives rcp 0 and g * 0; exp2 -> 0 gives g.
__device__ __forceinline__ float silu_mul_fast(float g, float u) {
  const float e = __builtin_amdgcn_exp2f(g * -1.44269504088896341f);
  return g * __builtin_amdgcn_rcpf(1.0f + e) * u;
}

// Byte selectors for v_perm_b32(recv, own, sel) in the epilogues' pair
// exchange: a lane holds rows (0, 1) of its column as own = r0 | r1 << 16
// (lower lane of the pair) or rows (2, 3) (upper lane), sends the other two
// rows to its partner and builds two dwords, each one row of the column
// pair (lower column in the low half).  Selector bytes 0-3 take own, 4-7
// recv.
__device__ __forceinline__ uint32_t pair_sel(bool upper, int d) {
  return upper ? (d == 0 ? 0x01000504u : 0x03020706u) : (d == 0 ? 0x05040100u : 0x07060302u);
}

// sum over the 16 lanes of a DPP row (lane & 15), in every lane of the row
__device__ __forceinline__ float row16_sum(float v) {
  v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0xB1, 0xF, 0xF, false));   // quad [1,0,3,2]
  v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x4E, 0xF, 0xF, false));   // quad [2,3,0,1]
  v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x141, 0xF, 0xF, false));  // half mirror
  v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x140, 0xF, 0xF, false));  // row mirror
  return v;
}

// One item: expert tile lb / n_nblk (its entry t, loaded by the caller one
// item ahead), column block lb % n_nblk.
template <int SD, int MODE, int WN, int STAGES_>
__device__ __forceinline__ void gemm_item(const GemmArgs &a, const int lb, const int4 t) {
  using Gm = Geo<WN, STAGES_>;
  constexpr int BN = Gm::BN, STAGES = Gm::STAGES, A_STAGE = Gm::A_STAGE, STAGE = Gm::STAGE;
  constexpr int NW = Gm::NW, THREADS = Gm::THREADS, COLS = Gm::COLS;
  // dynamic LDS: STAGES x (A | B) ring, scales[G][BN] fp16, xs[G][BM] fp32
  // (group-major: a lane's 4 rows are one 16-byte read); the epilogue's
  // staging and row sums reuse the idle ring
  extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
  const int n_nb = a.n_nblk;
  const int nb = lb % n_nb;
  const int e = t.x, pos0 = t.y, mcnt = t.z;
  const bool shared = e == a.E;
  // MODE 0: N = act columns (I or Is), block covers 64 of them; MODE 1: N = H, 128 rows
  const int N = MODE == 0 ? (shared ? a.Is : a.I) : a.H;
  const int K = MODE == 0 ? a.H : (shared ? a.Is : a.I);
  const int G = K >> 7;
  if (nb * (MODE == 0 ? COLS : BN) >= N) return;

  const uint32_t lds0 = (uint32_t)(uintptr_t)lds;
  uint16_t *sc_lds = (uint16_t *)(lds + STAGES * STAGE);
  float *xs_lds = (float *)(lds + STAGES * STAGE + ((BN * G * 2 + 15) & ~15));

  GTRACE(const unsigned long long t0 = __builtin_amdgcn_s_memtime());
  const int tid = tid_opaque();  // per item: nothing lane-dependent is hoisted across items
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & 63;
  // 2 token waves x WN row waves; wave w runs on SIMD w % 4, so each SIMD
  // hosts waves of both token halves (a tile of <= 64 tokens keeps every
  // SIMD busy)
  const int wn = wave % WN, wm = wave / WN;
  const int m16 = lane & 15, q = lane >> 4;

  // ---- per-thread DMA sources: A_DMA A slots and B_DMA B slots per stage ---
  // slot s = (i*NW + wave)*64 + lane, 16 bytes each.  The block-uniform part
  // of each address is a scalar base (advanced per group); a lane keeps one
  // 32-bit offset per slot.
  const uint8_t *abase;
  uint32_t aoff[Gm::A_DMA];
  if (MODE == 0)
    abase = (const uint8_t *)(a.a_routed + (shared ? (size_t)pos0 * a.H : 0));
  else
    abase = (const uint8_t *)((shared ? a.a_shared : a.a_routed) + (size_t)pos0 * K);
#pragma unroll
  for (int i = 0; i < Gm::A_DMA; ++i) {
    const int s = (i * NW + wave) * 64 + lane;
    const int r = s >> 4, c = (s & 15) ^ aswz(r);
    const int rr = min(r, mcnt - 1);
    // MODE 0 routed: a gathered token row, tok < T <= 4096 and H <= 4096
    const uint32_t row = MODE == 0 && !shared ? (uint32_t)a.ptok[pos0 + rr] : (uint32_t)rr;
    aoff[i] = row * (uint32_t)(MODE == 0 ? a.H : K) * 2u + (uint32_t)c * 16u;
  }
  const size_t rowb = (size_t)K / 2;
  const uint8_t *bbase[Gm::B_DMA];
  uint32_t boff[Gm::B_DMA];
#pragma unroll
  for (int i = 0; i < Gm::B_DMA; ++i) {
    const int s = (i * NW + wave) * 64 + lane;
    const int r = s >> 2, qq = (s & 3) ^ bswz(r);
    // the 16 B-rows of one (i, wave) lie on one side of COLS (16 | COLS)
    const int r0 = (i * NW + wave) * 16;
    int row;
    if (MODE == 0) {  // B-rows [0, COLS) gate, [COLS, 2 COLS) up
      bbase[i] = r0 < COLS ? (shared ? a.ws0 : a.w0 + (size_t)e * N * rowb)
                           : (shared ? a.ws1 : a.w1 + (size_t)e * N * rowb);
      row = nb * COLS + (r % COLS);
    } else {
      bbase[i] = shared ? a.ws0 : a.w0 + (size_t)e * N * rowb;
      row = nb * BN + r;
    }
    row = min(row, N - 1);
    boff[i] = (uint32_t)row * (uint32_t)rowb + (uint32_t)qq * 16u;
  }
  // DMA of group g into stage st (normally g % STAGES)
  auto issue_to = [&](int g, int st) {
    const uint32_t base = lds0 + (uint32_t)st * STAGE;
#pragma unroll
    for (int i = 0; i < Gm::A_DMA; ++i)
      dma16s(aoff[i], abase + g * 256, base + (uint32_t)((i * NW + wave) * 1024));
#pragma unroll
    for (int i = 0; i < Gm::B_DMA; ++i)
      dma16s(boff[i], bbase[i] + g * 64, base + A_STAGE + (uint32_t)((i * NW + wave) * 1024));
  };
  auto issue = [&](int g) { issue_to(g, g % STAGES); };

  // ---- prologue: tables to LDS; groups 0 .. STAGES-2 in flight -------------
  // Tables: every load is issued before the first use (unrolled, clamped
  // indices, no per-lane branches), so the block pays one latency, not one
  // per element.  G <= 32.  Entry idx is (g = idx / rows, row = idx % rows):
  // consecutive threads write consecutive LDS words (the global reads
  // gather instead), so the LDS stores are free of bank conflicts.  The
  // first groups' DMA is issued after the table loads: loads complete in
  // issue order, so a wait for a table value never waits for the DMA.
  {
    constexpr int SC_IT = BN * 32 / THREADS;
    uint16_t scv[SC_IT];
#pragma unroll
    for (int i = 0; i < SC_IT; ++i) {
      const int idx = tid + i * THREADS;
      const int r = idx % BN, g = min(idx / BN, G - 1);
      const uint16_t *sc;
      int row;
      if (MODE == 0) {
        sc = r < COLS ? (shared ? a.ss0 : a.s0 + (size_t)e * N * G)
                      : (shared ? a.ss1 : a.s1 + (size_t)e * N * G);
        row = nb * COLS + (r % COLS);
      } else {
        sc = shared ? a.ss0 : a.s0 + (size_t)e * N * G;
        row = nb * BN + r;
      }
      scv[i] = sc[(size_t)min(row, N - 1) * G + g];
    }
    constexpr int XS_IT = BM * 32 / THREADS;
    float xv[XS_IT];
    if (MODE == 0) {
      int tok[XS_IT];
#pragma unroll
      for (int i = 0; i < XS_IT; ++i) {
        const int row = min((tid + i * THREADS) % BM, mcnt - 1);
        tok[i] = shared ? pos0 + row : a.ptok[pos0 + row];
      }
#pragma unroll
      for (int i = 0; i < XS_IT; ++i) {
        const int g = min((tid + i * THREADS) / BM, G - 1);
        xv[i] = a.xsum[(size_t)tok[i] * G + g];
      }
    } else {
      // act partial sums: a.aslots per 128-wide group, added in order
      const float *asb = shared ? a.asum_s : a.asum;
#pragma unroll
      for (int i = 0; i < XS_IT; ++i) {
        const int idx = tid + i * THREADS;
        const int row = min(idx % BM, mcnt - 1), g = min(idx / BM, G - 1);
        const float *as = asb + (size_t)(pos0 + row) * (a.aslots * G) + a.aslots * g;
        float v = as[0];
        for (int j = 1; j < a.aslots; ++j) v += as[j];
        xv[i] = v;
      }
    }
    issue(0);
    if (STAGES > 2) issue_to(min(1, G - 1), 1);  // group 1, or a dummy into idle stage 1
#pragma unroll
    for (int i = 0; i < SC_IT; ++i) {
      const int idx = tid + i * THREADS;
      if (idx < BN * G) sc_lds[idx] = scv[i];  // [g][r]
    }
#pragma unroll
    for (int i = 0; i < XS_IT; ++i) {
      const int idx = tid + i * THREADS;
      if (idx < BM * G) xs_lds[idx] = idx % BM < mcnt ? -136.0f * xv[i] : 0.0f;  // [g][row]
    }
  }

  // B rows of this wave's 4 N-subtiles
  int brow[4];
#pragma unroll
  for (int ns = 0; ns < 4; ++ns)
    brow[ns] = MODE == 0 ? (ns < 2 ? wn * 32 + ns * 16 : COLS + wn * 32 + (ns - 2) * 16) + m16
                         : wn * 64 + ns * 16 + m16;

  // The main loop, for NMS of this wave's 4 token subtiles (16 tokens each):
  // subtiles past the tile's token count cost no MFMA or A read.
  f32x4 tot[4][4];
#pragma unroll
  for (int ms = 0; ms < 4; ++ms)
#pragma unroll
    for (int ns = 0; ns < 4; ++ns) tot[ms][ns] = f32x4{0.f, 0.f, 0.f, 0.f};
  auto main_loop = [&](auto nms_c) {
    constexpr int NMS = decltype(nms_c)::value;
    uint32_t magic;
    asm volatile("v_mov_b32 %0, 0x43004300" : "=v"(magic));
    // acc and sprev start at zero, so the scale step of "group -1" adds
    // +0 * +0 to tot's +0 and leaves it unchanged (no branch in the loop)
    f32x4 acc[4][4];
#pragma unroll
    for (int ms = 0; ms < 4; ++ms)
#pragma unroll
      for (int ns = 0; ns < 4; ++ns) acc[ms][ns] = f32x4{0.f, 0.f, 0.f, 0.f};
    float sg[4], sprev[4] = {0.f, 0.f, 0.f, 0.f};
    // Group g, part 1: the scale step of group g-1 (VALU only) and the
    // scales of group g.
    auto part_v = [&](int g) {
#pragma unroll
      for (int ns = 0; ns < 4; ++ns) sg[ns] = scale_to_f32<SD>(sc_lds[g * BN + brow[ns]]);
#pragma unroll
      for (int ns = 0; ns < 4; ++ns)
#pragma unroll
        for (int ms = 0; ms < NMS; ++ms) tot[ms][ns] += sprev[ns] * acc[ms][ns];
    };
    // Group g, part 2: group sums and A fragments from LDS, B unpacked per
    // k-slice, and the 4 x NMS MFMAs of each of the 4 k-slices.
    // this wave's raw B chunks of group g (sign bits flipped: 8 + q)
    auto load_bx = [&](int g, u32x4 (&bx)[4]) {
      const uint8_t *sb = lds + (g % STAGES) * STAGE + A_STAGE;
#pragma unroll
      for (int ns = 0; ns < 4; ++ns)
        bx[ns] = *(const u32x4 *)(sb + brow[ns] * 64 + ((q ^ bswz(brow[ns])) << 4)) ^ 0x88888888u;
    };
    auto part_m = [&](int g, const u32x4 (&bx)[4]) {
      const uint8_t *sa = lds + (g % STAGES) * STAGE;
      const uint8_t *arow = sa + (wm * 64 + m16) * 256;
      // group sums (-136 sum_k a): the first k-slice accumulates onto them
      f32x4 c0[4];
#pragma unroll
      for (int ms = 0; ms < NMS; ++ms)
        c0[ms] = *(const f32x4 *)(xs_lds + g * BM + wm * 64 + ms * 16 + 4 * q);
      // A fragments one k-slice ahead; the scheduling barrier after each
      // slice keeps the compiler from hoisting all 16 reads (64 VGPRs) to
      // the top, which spills at this register budget
      u32x4 af[2][4];
#pragma unroll
      for (int ms = 0; ms < NMS; ++ms)
        af[0][ms] = *(const u32x4 *)(arow + ms * 16 * 256 + (((4 * q) ^ aswz(m16)) << 4));
      if constexpr (MODE == 0) {
        // k-slice j's MFMAs run column subtile by column subtile, and each
        // subtile's B operand for slice j+1 is unpacked right after its last
        // use, so the unpacking issues between MFMAs instead of as a block
        // before them; slices 1-3 are pinned to one MFMA, 32 / (4 NMS) VALU
        // and (first NMS) one LDS read per step.  Gate/up 1% faster (c2).
        // The down kernel keeps the form below: with this one its K = 512
        // items spill registers.
        u32x4 bf[4];
#pragma unroll
        for (int ns = 0; ns < 4; ++ns) bf[ns] = nib_slice3(bx[ns], 0, magic);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          if (j < 3) {
            const int chunk = ((4 * q + j + 1) ^ aswz(m16)) << 4;
#pragma unroll
            for (int ms = 0; ms < NMS; ++ms)
              af[(j + 1) & 1][ms] = *(const u32x4 *)(arow + ms * 16 * 256 + chunk);
          }
#pragma unroll
          for (int ns = 0; ns < 4; ++ns) {
#pragma unroll
            for (int ms = 0; ms < NMS; ++ms)
              acc[ms][ns] = mfma_bf16_16x16x32(af[j & 1][ms], bf[ns], j == 0 ? c0[ms] : acc[ms][ns]);
            if (j < 3) bf[ns] = nib_slice3(bx[ns], j + 1, magic);
          }
          // slice 0 also holds the scale step's 16 NMS fmas: left to the
          // compiler (a fixed pattern there spills)
          if (NMS > 0 && j > 0) {
#pragma unroll
            for (int i = 0; i < 4 * NMS; ++i) {
              __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA
              if (j < 3)
                __builtin_amdgcn_sched_group_barrier(0x002, 32 / (4 * (NMS > 0 ? NMS : 1)), 0);  // VALU
              else
                __builtin_amdgcn_sched_group_barrier(0x002, 1, 0);
              if (i < NMS && j < 3) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // LDS read
            }
          }
          __builtin_amdgcn_sched_barrier(0);
        }
      } else {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          if (j < 3) {
            const int chunk = ((4 * q + j + 1) ^ aswz(m16)) << 4;
#pragma unroll
            for (int ms = 0; ms < NMS; ++ms)
              af[(j + 1) & 1][ms] = *(const u32x4 *)(arow + ms * 16 * 256 + chunk);
          }
          u32x4 bf[4];
#pragma unroll
          for (int ns = 0; ns < 4; ++ns) bf[ns] = nib_slice3(bx[ns], j, magic);
#pragma unroll
          for (int ms = 0; ms < NMS; ++ms)
#pragma unroll
            for (int ns = 0; ns < 4; ++ns)
              acc[ms][ns] = mfma_bf16_16x16x32(af[j & 1][ms], bf[ns], j == 0 ? c0[ms] : acc[ms][ns]);
          __builtin_amdgcn_sched_barrier(0);
        }
      }
#pragma unroll
      for (int ns = 0; ns < 4; ++ns) sprev[ns] = sg[ns];
    };

    u32x4 bx[4];
    if constexpr (STAGES == 2) {
      // One barrier per group.  At the top of iteration g every wave has
      // issued all its MFMAs of group g-1 (they may still be executing) and
      // has read its last fragment of stage g-1, so after the barrier the DMA
      // of group g+1 may overwrite that stage.
      for (int g = 0; g < G; ++g) {
        wait_vm<0>();  // this thread's DMA of group g (issued one group ago)
        // stage g complete for every thread (and, at g = 0, the LDS tables)
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        block_barrier();
        if (g + 1 < G) issue(g + 1);
        load_bx(g, bx);
        part_v(g);
        part_m(g, bx);
      }
    } else {
      // Three stages; the barrier that ends iteration g-1 also makes group
      // g+1 visible, so each wave reads its B chunks of the next group into
      // registers at the end of a group, and a group starts with the scale
      // step (VALU) that hides its first LDS reads, then unpacks at once.
      // The DMA of group g+2 is issued after that barrier into stage
      // (g+2) % 3, which held group g-1, and every thread waits for it
      // before the next barrier: one iteration of latency per DMA.
      asm volatile("s_waitcnt vmcnt(0)\n\ts_waitcnt lgkmcnt(0)" ::: "memory");
      block_barrier();  // groups 0 and 1 and the LDS tables complete
      for (int g = 0; g < G; ++g) {
        if (g + 2 < G) issue(g + 2);
        load_bx(g, bx);
        part_v(g);
        part_m(g, bx);
        wait_vm<0>();
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        block_barrier();
      }
    }
#pragma unroll
    for (int ns = 0; ns < 4; ++ns)
#pragma unroll
      for (int ms = 0; ms < NMS; ++ms) tot[ms][ns] += sprev[ns] * acc[ms][ns];
  };
  // token subtiles of this wave holding tokens of the tile (wave-uniform)
  GTRACE(const unsigned long long t1 = __builtin_amdgcn_s_memtime());
  const int nms = __builtin_amdgcn_readfirstlane(max(0, min(4, (mcnt - wm * 64 + 15) >> 4)));
  if (nms > 2)
    main_loop(std::integral_constant<int, 4>());
  else if (nms > 0)
    main_loop(std::integral_constant<int, 2>());
  else
    main_loop(std::integral_constant<int, 0>());
  wait_vm<0>();  // no DMA into the ring remains in flight
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
  block_barrier();  // every wave's last read of the ring precedes the staging below
  GTRACE(if (tid == 0 && lb < 16384) {
    const int o = (MODE * 16384 + lb) * 4;
    g_gtrace[o] = t0;
    g_gtrace[o + 1] = t1;
    g_gtrace[o + 2] = __builtin_amdgcn_s_memtime();
  });

  // ---- epilogue -------------------------------------------------------
  // lane (q, m16) of tile (ms, ns) holds rows wm*64 + ms*16 + 4q + r, column
  // m16.  Results are staged in the (now idle) LDS ring and leave as 16-byte
  // row chunks.
  if (MODE == 0) {
    constexpr int OST = COLS * 2 + 16;  // staged row stride, bytes
    // staged rows, then red_sum[WN][BM] fp32 (per row-wave row sums)
    float *red_sum = (float *)(lds + BM * OST);
    static_assert(BM * OST + WN * BM * 4 <= STAGES * STAGE, "staging exceeds the ring");
    float rowsum[4][4];
#pragma unroll
    for (int ms = 0; ms < 4; ++ms)
#pragma unroll
      for (int r = 0; r < 4; ++r) rowsum[ms][r] = 0.0f;
    // Columns k and k + 4 of a 32-column block are neighbours in MFMA order
    // (perm32_pos), and live in lanes m16 and m16 ^ 4: the pair trades
    // halves so that each lane stores whole dwords (lane bit 2 clear: rows
    // r = 0, 1; set: rows 2, 3).  2-byte LDS stores cost several times a
    // dword store.
    // Branch-free: the selects below are plain values and v_perm_b32 takes
    // a per-lane selector (ternaries over expressions became divergent
    // branches around every store).
    const bool hi4 = (m16 & 4) != 0;
    const uint32_t sel0 = pair_sel(hi4, 0), sel1 = pair_sel(hi4, 1);
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      // within a 32-aligned block of columns, MFMA order is block-local
      const int p = perm32_pos(wn * 32 + h * 16 + (m16 & ~4));  // the pair's even position
#pragma unroll
      for (int ms = 0; ms < 4; ++ms) {
        float f[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) f[r] = silu_mul_fast(tot[ms][h][r], tot[ms][h + 2][r]);
        const uint32_t p01 = bf16x2_bits(f[0], f[1]), p23 = bf16x2_bits(f[2], f[3]);
        rowsum[ms][0] += __uint_as_float(p01 << 16);
        rowsum[ms][1] += __uint_as_float(p01 & 0xFFFF0000u);
        rowsum[ms][2] += __uint_as_float(p23 << 16);
        rowsum[ms][3] += __uint_as_float(p23 & 0xFFFF0000u);
        const uint32_t send = hi4 ? p01 : p23, own = hi4 ? p23 : p01;
        // lane ^ 4 inside each group of 32 lanes (ds_swizzle bit mode)
        const uint32_t recv = (uint32_t)__builtin_amdgcn_ds_swizzle((int)send, 0x101F);
        const int row0 = wm * 64 + ms * 16 + 4 * q + (hi4 ? 2 : 0);
        *(uint32_t *)(lds + row0 * OST + p * 2) = __builtin_amdgcn_perm(recv, own, sel0);
        *(uint32_t *)(lds + (row0 + 1) * OST + p * 2) = __builtin_amdgcn_perm(recv, own, sel1);
      }
    }
    // per-row sum over this wave's 32 columns: reduce over the 16 lanes m16
#pragma unroll
    for (int ms = 0; ms < 4; ++ms)
#pragma unroll
      for (int r = 0; r < 4; ++r) rowsum[ms][r] = row16_sum(rowsum[ms][r]);
    if (m16 == 0)
#pragma unroll
      for (int ms = 0; ms < 4; ++ms)
#pragma unroll
        for (int r = 0; r < 4; ++r) red_sum[wn * BM + wm * 64 + ms * 16 + 4 * q + r] = rowsum[ms][r];
    __syncthreads();
    uint16_t *dst = shared ? a.act_s : a.act;
    constexpr int CPR = COLS / 8;  // 16-byte chunks per row
    constexpr int NST = BM * CPR / THREADS;
    u32x4 out[NST];  // every LDS read before the (predicated) stores
#pragma unroll
    for (int i = 0; i < NST; ++i) {
      const int idx = tid + i * THREADS;
      out[i] = *(const u32x4 *)(lds + (idx / CPR) * OST + (idx % CPR) * 16);
    }
#pragma unroll
    for (int i = 0; i < NST; ++i) {
      const int idx = tid + i * THREADS, row = idx / CPR, c = idx % CPR;
      if (row < mcnt) *(u32x4 *)(dst + (size_t)(pos0 + row) * N + nb * COLS + c * 8) = out[i];
    }
    if (tid < BM && tid < mcnt) {
      float *as = shared ? a.asum_s : a.asum;
      // one partial per COLS act columns (slot nb), row waves summed in order
      float v = 0.0f;
#pragma unroll
      for (int w = 0; w < WN; ++w) v += red_sum[w * BM + tid];
      as[(size_t)(pos0 + tid) * (N / COLS) + nb] = v;
    }
  } else {
    constexpr int OST = BN * 2 + 16;
    static_assert(BM * OST <= STAGES * STAGE, "staging exceeds the ring");
    // Neighbouring columns live in lanes m16 and m16 ^ 1: the pair trades
    // halves so that each lane stores whole dwords (even lane: rows r = 0,
    // 1; odd lane: rows 2, 3).  With the 528-byte row stride the 32 lanes of
    // one store hit 32 distinct banks.
    const bool odd = (m16 & 1) != 0;
    const uint32_t sel0 = pair_sel(odd, 0), sel1 = pair_sel(odd, 1);
#pragma unroll
    for (int ns = 0; ns < 4; ++ns) {
      const int cl = wn * 64 + 16 * ns + (m16 & ~1);
#pragma unroll
      for (int ms = 0; ms < 4; ++ms) {
        const uint32_t p01 = bf16x2_bits(tot[ms][ns][0], tot[ms][ns][1]);
        const uint32_t p23 = bf16x2_bits(tot[ms][ns][2], tot[ms][ns][3]);
        const uint32_t send = odd ? p01 : p23, own = odd ? p23 : p01;
        const uint32_t recv =
            (uint32_t)__builtin_amdgcn_update_dpp(0, (int)send, 0xB1, 0xF, 0xF, false);  // lane ^ 1
        const int row0 = wm * 64 + ms * 16 + 4 * q + (odd ? 2 : 0);
        *(uint32_t *)(lds + row0 * OST + cl * 2) = __builtin_amdgcn_perm(recv, own, sel0);
        *(uint32_t *)(lds + (row0 + 1) * OST + cl * 2) = __builtin_amdgcn_perm(recv, own, sel1);
      }
    }
    __syncthreads();
    constexpr int CPR = BN / 8;
    constexpr int NST = BM * CPR / THREADS;
    u32x4 out[NST];  // every LDS read before the (predicated) stores
#pragma unroll
    for (int i = 0; i < NST; ++i) {
      const int idx = tid + i * THREADS;
      out[i] = *(const u32x4 *)(lds + (idx / CPR) * OST + (idx % CPR) * 16);
    }
#pragma unroll
    for (int i = 0; i < NST; ++i) {
      const int idx = tid + i * THREADS, row = idx / CPR, c = idx % CPR;
      const int col = nb * BN + c * 8;
      if (row < mcnt && col < N) {
        const size_t orow = shared ? (size_t)a.T * a.k + pos0 + row : (size_t)(pos0 + row);
        *(u32x4 *)(a.o + orow * a.H + col) = out[i];
      }
    }
  }
}

// Persistent grid: one block per resident slot (occupancy x CUs) walks the
// items in rounds of gridDim.x.  Within a round the items a block takes are
// XCD-contiguous (xcd_remap), so the column blocks of one expert tile run on
// one XCD at the same time and share its A rows through that L2.  The item
// count comes from the dispatch on the device; the host sizes the grid from
// its upper bound.
template <int SD, int MODE, int WN, int STAGES_>
__global__ __launch_bounds__(128 * WN) void k_expert_gemm(GemmArgs a) {
  const int n_items = *a.n_tiles * a.n_nblk;
  const int P = gridDim.x, me = xcd_remap(blockIdx.x, P);
  // the tile entry of the next item is loaded while this one runs (it is a
  // global load the item's whole prologue would otherwise wait on)
  int4 t = me < n_items ? a.tiles[me / a.n_nblk] : int4{0, 0, 0, 0};
  for (int base = 0; base < n_items; base += P) {
    const int lb = base + me;
    if (lb >= n_items) break;  // later rounds only hold larger items
    const int ln = lb + P;
    const int4 tn = ln < n_items ? a.tiles[ln / a.n_nblk] : t;
    gemm_item<SD, MODE, WN, STAGES_>(a, lb, t);
    t = tn;
    __syncthreads();  // the epilogue's LDS reads precede the next item's DMA
    GTRACE(if (threadIdx.x == 0 && lb < 16384) g_gtrace[(MODE * 16384 + lb) * 4 + 3] =
               __builtin_amdgcn_s_memtime());
  }
}

// ---------------------------------------------------------------------------
// Router logits for prefill: approx[t][e] = sum_k x[t][k] * w[e][k] (+ bias)
// on bf16 MFMA, fp32 accumulation.  Block tile: 64 tokens x 128 experts,
// 4 waves as 2 (tokens) x 2 (experts), each 32 x 64 = 2 x 4 MFMA tiles.  K
// streams through a 3-stage LDS ring in 64-wide steps (x rows and w rows,
// 128 bytes each, 16-byte chunk c of row r stored at c ^ (r & 7)).  The
// blocks after the GEMM tiles compute ||w_e|| (used only as the bound of
// the canonical refine).
// ---------------------------------------------------------------------------
#ifndef RG_BM_
#define RG_BM_ 64
#endif
constexpr int RG_BM = RG_BM_, RG_BN = 128, RG_BK = 64, RG_ST = 3;
constexpr int RG_MS = RG_BM / 32;  // 16-token MFMA rows per wave
constexpr int RG_A = RG_BM * RG_BK * 2, RG_B = RG_BN * RG_BK * 2;  // bytes per stage
constexpr int RG_STAGE = RG_A + RG_B;
constexpr int RG_DMA = RG_STAGE / (256 * 16);  // per thread per stage: 6
constexpr int RG_NORM_ROWS = 16;                // experts per norm block

__global__ __launch_bounds__(256) void k_router_gemm(const uint16_t *__restrict__ x,
                                                     const uint16_t *__restrict__ rw,
                                                     const float *__restrict__ bias,
                                                     float *__restrict__ approx,
                                                     float *__restrict__ wnorm, int T, int H,
                                                     int E, int n_mt, int n_nt,
                                                     uint32_t *__restrict__ zbuf, int zwords) {
  extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
  const int n_items = n_mt * n_nt;
  if ((int)blockIdx.x >= n_items) {
    // ---- the dispatch counts and masks k_select fills next start at zero --
    const int nb = (int)gridDim.x - n_items, b = (int)blockIdx.x - n_items;
    for (int i = b * 256 + tid; i < zwords; i += nb * 256) zbuf[i] = 0u;
    // ---- row norms: wave w takes rows e0 + 4w .. e0 + 4w + 3 -------------
    const int e0 = ((int)blockIdx.x - n_items) * RG_NORM_ROWS + wave * 4;
    for (int r = 0; r < 4; ++r) {
      const int e = e0 + r;
      if (e >= E) break;
      const uint16_t *row = rw + (size_t)e * H;
      float ss = 0.0f;
      for (int c = lane; c < (H >> 3); c += 64) {
        const u32x4 v = *(const u32x4 *)(row + 8 * c);
#pragma unroll
        for (int d = 0; d < 4; ++d) {
          const float lo = __uint_as_float(v[d] << 16), hi = __uint_as_float(v[d] & 0xFFFF0000u);
          ss = __builtin_fmaf(lo, lo, ss);
          ss = __builtin_fmaf(hi, hi, ss);
        }
      }
      for (int m = 32; m >= 1; m >>= 1) ss += __shfl_xor(ss, m, 64);
      if (lane == 0) wnorm[e] = sqrtf(ss);
    }
    return;
  }
  const int lb = xcd_remap(blockIdx.x, n_items);
  const int mt = lb / n_nt, nt = lb % n_nt;  // the n_nt expert tiles of a token tile share an XCD
  const int t0 = mt * RG_BM, e0 = nt * RG_BN;
  const int wm = wave & 1, wn = wave >> 1;
  const int m16 = lane & 15, q = lane >> 4;
  const uint32_t lds0 = (uint32_t)(uintptr_t)lds;

  // DMA sources: slot s = (i*4 + wave)*64 + lane; row s/8, stored chunk s%8
  const uint8_t *src[RG_DMA];
#pragma unroll
  for (int i = 0; i < RG_DMA; ++i) {
    const int sl = (i * 4 + wave) * 64 + lane;
    const int r = sl >> 3, c = (sl & 7) ^ (r & 7);
    if (r < RG_BM) {
      src[i] = (const uint8_t *)(x + (size_t)min(t0 + r, T - 1) * H) + c * 16;
    } else {
      src[i] = (const uint8_t *)(rw + (size_t)min(e0 + r - RG_BM, E - 1) * H) + c * 16;
    }
  }
  auto issue = [&](int g) {
    const uint32_t base = lds0 + (uint32_t)(g % RG_ST) * RG_STAGE;
#pragma unroll
    for (int i = 0; i < RG_DMA; ++i)
      dma16(src[i] + g * (RG_BK * 2), base + (uint32_t)((i * 4 + wave) * 1024));
  };
  const int G = H / RG_BK;
  issue(0);
  if (G > 1) issue(1);
  f32x4 acc[RG_MS][4];
#pragma unroll
  for (int ms = 0; ms < RG_MS; ++ms)
#pragma unroll
    for (int ns = 0; ns < 4; ++ns) acc[ms][ns] = f32x4{0.f, 0.f, 0.f, 0.f};
  for (int g = 0; g < G; ++g) {
    if (g + 2 < G) {
      issue(g + 2);
      wait_vm<2 * RG_DMA>();
    } else if (g + 1 < G) {
      wait_vm<RG_DMA>();
    } else {
      wait_vm<0>();
    }
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    block_barrier();
    const uint8_t *sa = lds + (g % RG_ST) * RG_STAGE, *sb = sa + RG_A;
#pragma unroll
    for (int s2 = 0; s2 < 2; ++s2) {  // two 32-wide MFMA steps
      u32x4 af[RG_MS], bf[4];
#pragma unroll
      for (int ms = 0; ms < RG_MS; ++ms) {
        const int r = wm * (RG_BM / 2) + ms * 16 + m16;
        af[ms] = *(const u32x4 *)(sa + r * 128 + (((4 * s2 + q) ^ (r & 7)) << 4));
      }
#pragma unroll
      for (int ns = 0; ns < 4; ++ns) {
        const int r = wn * 64 + ns * 16 + m16;
        bf[ns] = *(const u32x4 *)(sb + r * 128 + (((4 * s2 + q) ^ (r & 7)) << 4));
      }
#pragma unroll
      for (int ms = 0; ms < RG_MS; ++ms)
#pragma unroll
        for (int ns = 0; ns < 4; ++ns) acc[ms][ns] = mfma_bf16_16x16x32(af[ms], bf[ns], acc[ms][ns]);
    }
    block_barrier();  // stage g may be overwritten by the DMA issued next iteration
  }
  // lane (q, m16) of tile (ms, ns): tokens wm*32 + ms*16 + 4q + r, expert wn*64 + ns*16 + m16
#pragma unroll
  for (int ns = 0; ns < 4; ++ns) {
    const int e = e0 + wn * 64 + ns * 16 + m16;
    if (e >= E) continue;
    const float b = bias ? bias[e] : 0.0f;
#pragma unroll
    for (int ms = 0; ms < RG_MS; ++ms)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int t = t0 + wm * (RG_BM / 2) + ms * 16 + 4 * q + r;
        if (t < T) approx[(size_t)t * E + e] = bias ? acc[ms][ns][r] + b : acc[ms][ns][r];
      }
  }
}

constexpr size_t GEMM_LDS_MAX = 160 * 1024;  // LDS per workgroup on gfx950

template <int WN>
size_t gemm_lds_bytes(int stages, int Gmax) {
  using Gm = Geo<WN, 2>;
  return (size_t)stages * Gm::STAGE + (((size_t)Gm::BN * Gmax * 2 + 15) & ~(size_t)15) +
         sizeof(float) * (size_t)BM * Gmax;
}

template <int WN, int STAGES_>
hipError_t launch_geo(int mode, int scale_dtype, GemmArgs a, int max_tiles, hipStream_t s) {
  using Gm = Geo<WN, STAGES_>;
  const int Nmax = mode == 0 ? (a.I > a.Is ? a.I : a.Is) : a.H;
  a.n_nblk = mode == 0 ? (Nmax + Gm::COLS - 1) / Gm::COLS : (Nmax + Gm::BN - 1) / Gm::BN;
  a.aslots = 128 / Gm::COLS;  // act partial sums per 128-wide group (MODE 0 writes them)
  const long grid = (long)max_tiles * a.n_nblk;
  if (grid > 0x7FFFFFFF) return hipErrorInvalidValue;
  const int Gmax = (mode == 0 ? a.H : (a.I > a.Is ? a.I : a.Is)) / 128;
  if (Gmax > 32) return hipErrorInvalidValue;  // table loads assume K <= 4096
  const size_t lds = gemm_lds_bytes<WN>(Gm::STAGES, Gmax);
  if (lds > GEMM_LDS_MAX) return hipErrorInvalidValue;
  void (*kern)(GemmArgs);
  if (mode == 0)
    kern = scale_dtype == AINFER_SCALE_FP16 ? k_expert_gemm<AINFER_SCALE_FP16, 0, WN, STAGES_>
                                            : k_expert_gemm<AINFER_SCALE_BF16, 0, WN, STAGES_>;
  else
    kern = scale_dtype == AINFER_SCALE_FP16 ? k_expert_gemm<AINFER_SCALE_FP16, 1, WN, STAGES_>
                                            : k_expert_gemm<AINFER_SCALE_BF16, 1, WN, STAGES_>;
  // resident blocks per CU for this kernel and LDS size, times the CUs
  int dev = 0, cus = 0, per_cu = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e == hipSuccess) e = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
  if (e == hipSuccess)
    e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kern, Gm::THREADS, lds);
  if (e != hipSuccess) return e;
  if (per_cu < 1) return hipErrorInvalidConfiguration;
  const long resident = (long)per_cu * cus;
  kern<<<(unsigned)(grid < resident ? grid : resident), Gm::THREADS, lds, s>>>(a);
  return hipGetLastError();
}

}  // namespace

hipError_t launch_router_gemm(const void *x, const void *rw, const float *bias, float *approx,
                              float *wnorm, int T, int H, int E, uint32_t *zbuf, int zwords,
                              hipStream_t s) {
  if (T <= 0) return hipSuccess;
  if (H % RG_BK) return hipErrorInvalidValue;
  const int n_mt = (T + RG_BM - 1) / RG_BM, n_nt = (E + RG_BN - 1) / RG_BN;
  const int n_norm = (E + RG_NORM_ROWS - 1) / RG_NORM_ROWS;
  const long grid = (long)n_mt * n_nt + n_norm;
  if (grid > 0x7FFFFFFF) return hipErrorInvalidValue;
  k_router_gemm<<<(unsigned)grid, 256, RG_ST * RG_STAGE, s>>>(
      (const uint16_t *)x, (const uint16_t *)rw, bias, approx, wnorm, T, H, E, n_mt, n_nt,
      zbuf, zbuf ? zwords : 0);
  return hipGetLastError();
}

// Both GEMM modes of one forward must use the same geometry (MODE 1 reads
// the act partial sums MODE 0 wrote).
hipError_t launch_expert_gemm(int mode, int scale_dtype, GemmArgs a, int max_tiles,
                              hipStream_t s) {
  if (max_tiles <= 0) return hipSuccess;
  // the 3-stage ring where its LDS fits (K <= 2048 at GEMM_WN = 4)
  const int Gmax = (mode == 0 ? a.H : (a.I > a.Is ? a.I : a.Is)) / 128;
  if (gemm_lds_bytes<GEMM_WN>(3, Gmax) <= GEMM_LDS_MAX)
    return launch_geo<GEMM_WN, 3>(mode, scale_dtype, a, max_tiles, s);
  return launch_geo<GEMM_WN, 2>(mode, scale_dtype, a, max_tiles, s);
}

// ---------------------------------------------------------------------------
// MFMA-rate probe: every wave issues ITERS x 16 independent
// v_mfma_f32_16x16x32_bf16 (16 accumulator tiles) with NV independent fp32
// FMAs after each, so the rate it reports is the ceiling of a main loop that
// spends NV VALU instructions per MFMA.  One block per CU of 64 * 4 * WPS
// threads (WPS waves per SIMD).  The results are stored only when iters < 0,
// which never holds, so nothing is written and nothing is optimised away.
// ---------------------------------------------------------------------------
namespace {
template <int NV>
__global__ void k_mfma_probe(float *sink, int iters) {
  f32x4 acc[16];
#pragma unroll
  for (int i = 0; i < 16; ++i) acc[i] = f32x4{0.f, 0.f, 0.f, 0.f};
  u32x4 a, b;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    a[i] = 0x3F803F80u + threadIdx.x + i;
    b[i] = 0x3F803F80u + 3u * threadIdx.x + i;
  }
  float v[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) v[i] = (float)threadIdx.x * 0.001f + (float)i;
  for (int it = 0; it < iters; ++it) {
#pragma unroll
    for (int m = 0; m < 16; ++m) {
      acc[m] = mfma_bf16_16x16x32(a, b, acc[m]);
#pragma unroll
      for (int j = 0; j < NV; ++j) v[j & 7] = __builtin_fmaf(v[j & 7], 1.0001f, 0.5f);
    }
  }
  if (iters < 0) {
    float s = 0.f;
#pragma unroll
    for (int i = 0; i < 16; ++i) s += acc[i][0] + acc[i][1] + acc[i][2] + acc[i][3];
#pragma unroll
    for (int i = 0; i < 8; ++i) s += v[i];
    sink[threadIdx.x] = s;
  }
}
}  // namespace

extern "C" int ainfer_moe_mfma_probe(int32_t valu_per_mfma, int32_t waves_per_simd, int32_t iters,
                                     void *stream, float *tflops) {
  if (!tflops || iters <= 0 || iters > (1 << 20) || waves_per_simd < 1 || waves_per_simd > 4 ||
      valu_per_mfma < 0 || valu_per_mfma > 4)
    return AINFER_ERR_ARG;
  int dev = 0, cus = 0;
  if (hipGetDevice(&dev) != hipSuccess ||
      hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
    return AINFER_ERR_HIP;
  const hipStream_t s = (hipStream_t)stream;
  const dim3 grid((unsigned)cus), block(256u * (unsigned)waves_per_simd);
  auto launch = [&]() {
    switch (valu_per_mfma) {
      case 0: k_mfma_probe<0><<<grid, block, 0, s>>>(nullptr, iters); break;
      case 1: k_mfma_probe<1><<<grid, block, 0, s>>>(nullptr, iters); break;
      case 2: k_mfma_probe<2><<<grid, block, 0, s>>>(nullptr, iters); break;
      case 3: k_mfma_probe<3><<<grid, block, 0, s>>>(nullptr, iters); break;
      case 4: k_mfma_probe<4><<<grid, block, 0, s>>>(nullptr, iters); break;
      default: return false;
    }
    return true;
  };
  hipEvent_t e0, e1;
  if (hipEventCreate(&e0) != hipSuccess) return AINFER_ERR_HIP;
  if (hipEventCreate(&e1) != hipSuccess) {
    (void)hipEventDestroy(e0);
    return AINFER_ERR_HIP;
  }
  int rc = 0;
  float ms = 0.f;
  if (!launch()) {
    rc = AINFER_ERR_ARG;
  } else if (hipEventRecord(e0, s) != hipSuccess || !launch() || hipEventRecord(e1, s) != hipSuccess ||
             hipEventSynchronize(e1) != hipSuccess || hipEventElapsedTime(&ms, e0, e1) != hipSuccess ||
             hipGetLastError() != hipSuccess) {
    rc = AINFER_ERR_HIP;
  } else {
    const double flop = (double)cus * 4 * waves_per_simd * iters * 16 * (2.0 * 16 * 16 * 32);
    *tflops = (float)(flop / (ms * 1e-3) / 1e12);
  }
  (void)hipEventDestroy(e0);
  (void)hipEventDestroy(e1);
  return rc;
}
