// gemm.hip — MFMA GEMM kernels for gfx950 (CDNA4), fp16-in/fp32-acc and fp32.
//
//   C[M,N] = act(alpha * op(A) * op(B) + beta * C + bias[n]),  row-major, batched.
//
// Replaces the reference's MPSMatrixMultiplication call (internal/cgo/
// metal_bridge_matrix.m:90-113), its optimized_gemm / batch_matmul_optimized MSL
// kernels (metal_bridge_kernels.m:28-110) and the fused_linear_activation kernel
// (default.metal:459-509).
//
// Two kernel families share the epilogue and the tile order: the DMA-ring kernels
// gemm_f16_ring_kernel and gemm_f32_ring_kernel (large fp16 and fp32 problems; described
// at their definitions; gemm_f16_ring_mf32_kernel is the NN 256 x 256 ring on 32 x 32 x 16
// instructions, kept for measurement behind GONNGPU_F16_MFMA32=1) and the register-staged
// gemm_f16_kernel / gemm_f32_kernel for every other shape, structured as follows
// (one workgroup per BM x BN output tile, WM x WN waves, 64 lanes each):
//  * global -> VGPR prefetch of the next BK slice overlaps the MFMAs of the current
//    one; LDS is double buffered, one barrier per BK slice;
//  * operands whose K index is contiguous in memory are kept K-contiguous in LDS and
//    read with ds_read_b128; fp16 operands whose M/N index is contiguous are kept in
//    their memory layout and read with ds_read_b64_tr_b16, which transposes 4x16
//    blocks across a 16-lane group (out lane i, element e <- source lane 4e+i/4,
//    element i%4), giving the MFMA K-contiguous operand directly;
//  * fp32 operands keep their memory layout in LDS too; an M/N-contiguous fp32 operand
//    is read one float per lane and MFMA step (see gemm_f32_kernel);
//  * a grouped, XCD-aware tile order: hardware dispatches workgroup w to XCD w % 8,
//    so w is remapped to give each XCD a contiguous band of tiles that share A/B
//    panels in that XCD's L2.
#include "act.h"
#include "common.h"
#include "ring_plan.h"

namespace gn {
namespace {

typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef float float4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));
typedef __fp16 trh4_t __attribute__((__vector_size__(4 * sizeof(__fp16))));
typedef _Float16 half4_t __attribute__((ext_vector_type(4)));

#define LDS_AS __attribute__((address_space(3)))

struct GemmParams {
  const void *A;
  const void *B;
  float *C;
  const float *bias;
  long M, N, K;
  long lda, ldb, ldc;
  long strideA, strideB, strideC;
  float alpha, beta, act_alpha;
  int act;
  int tiles_m, tiles_n;
  int group_m;  // tile rows per raster group (tile_coords); 0 selects the default of 4
};

// ------------------------------------------------------------------ epilogue
// Workgroup barrier that orders LDS accesses only (s_waitcnt lgkmcnt(0); s_barrier).
// __syncthreads() also waits for vmcnt(0), i.e. for every global store the wave has
// issued to complete, which between the epilogue's passes serialised each pass behind
// the previous pass's C writes.
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

template <int V>
struct ActCode {
  static constexpr int value = V;
};
constexpr int kActRuntime = -1000;  // ActCode value: apply p.act, decided per element

// Writes a workgroup's BM x BN accumulator tile to C in row order. Pass f stages MFMA
// block-row f of every wave (WM x 16 tile rows, all BN columns) in LDS at `stg` (pitch
// BN + 4 floats: the 4 row groups of one ds_write_b32 fall on distinct banks), then the
// workgroup stores those rows as 16-byte vectors with consecutive lanes along a row, so
// each store instruction writes long contiguous row segments (one whole 1 KiB row at
// BN = 256). All CUs write their tiles at about the same time; when each wave stored
// only its own 256-byte row pieces (rows 32 KiB apart), the writes drained so slowly
// that the 8192^3 GEMM took 11% longer (4096^3: 17%). Each thread owns one column quad
// for the whole epilogue, so its bias values are loaded once, before the first pass: a
// load inside the passes would wait for all earlier stores (vmcnt counts stores too).
// The passes are separated by LDS-only barriers, so the stores of one pass drain while
// the next is staged. alpha, beta*C, bias and the activation are applied on the way;
// scalar stores at ragged edges or when ldc / C do not allow aligned 16-byte stores.
// The pass loop is unrolled so every accumulator index is static (a runtime index would
// move the accumulators to scratch memory). stage(f) writes the wave's rows of pass f (wave
// tile rows 16 f .. 16 f + 15) into stg at rows wm * 16 + 0..15, pitch BN + 4, columns
// wn * (BN / WN) + 0..BN / WN - 1.
template <int BM, int BN, int WM, int WN, typename Stage>
__device__ __forceinline__ void store_tile_passes(const GemmParams &p, long m0, long n0, long z, float *stg,
                                                  Stage &&stage) {
  constexpr int WTM = BM / WM, FM = WTM / 16;
  constexpr int LP = BN + 4, CPR = BN / 4, NTH = WM * WN * 64;
  constexpr int ROWS = WM * 16;       // tile rows staged per pass
  constexpr int RPS = NTH / CPR;      // rows one sweep of the workgroup's threads covers
  constexpr int SWEEPS = (ROWS + RPS - 1) / RPS;
  static_assert(BN % 4 == 0 && CPR <= NTH, "row vectors");
  const int c4 = threadIdx.x % CPR, r0 = threadIdx.x / CPR;  // threads with r0 >= RPS only stage
  const long col = n0 + 4 * c4;
  float *C = p.C + z * p.strideC;
  const bool vec = (p.ldc % 4 == 0) && (((uintptr_t)C & 15) == 0) && col + 3 < p.N;
  float bv[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) bv[e] = (p.bias && col + e < p.N) ? p.bias[col + e] : 0.0f;
#pragma unroll
  for (int f = 0; f < FM; ++f) {
    lds_barrier();  // the previous pass (or the main loop) is done with stg
    stage(f);
    lds_barrier();
    // The common activations get their own copy of the row sweep with the code fixed at
    // compile time: the generic one inlines every case of apply_act for every element,
    // and that long branchy code cost 3.5 us per launch at 512 x 11008 x 512 (ReLU).
    auto sweep = [&](auto act_c) {
      constexpr int ACT = decltype(act_c)::value;
      const int act = ACT == kActRuntime ? p.act : ACT;
      // a runtime loop: unrolling it as well made the pass loop too large to unroll
      // fully (the 256 x 256 kernels then kept the accumulators in scratch memory)
#pragma unroll 1
      for (int s = 0; s < SWEEPS; ++s) {
        const int t = r0 + s * RPS;
        if (r0 >= RPS || t >= ROWS) continue;
        const long row = m0 + (t / 16) * WTM + f * 16 + (t % 16);
        if (row >= p.M) continue;
        const float4_t v = *reinterpret_cast<const float4_t *>(stg + t * LP + 4 * c4);
        float *dst = C + row * p.ldc + col;
        if (vec) {
          float4_t o;
          const float4_t old =
              p.beta != 0.0f ? *reinterpret_cast<const float4_t *>(dst) : float4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
          for (int e = 0; e < 4; ++e) o[e] = apply_act(act, p.alpha * v[e] + p.beta * old[e] + bv[e], p.act_alpha);
          __builtin_nontemporal_store(o, reinterpret_cast<float4_t *>(dst));  // C is not re-read: keep L2 for A/B
        } else {
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            if (col + e < p.N) {
              float x = p.alpha * v[e];
              if (p.beta != 0.0f) x += p.beta * dst[e];
              dst[e] = apply_act(act, x + bv[e], p.act_alpha);
            }
          }
        }
      }
    };
    switch (p.act) {
      case -1: sweep(ActCode<-1>{}); break;
      case 0: sweep(ActCode<0>{}); break;
      case 7: sweep(ActCode<7>{}); break;
      default: sweep(ActCode<kActRuntime>{}); break;
    }
  }
}

// store_tile_passes for 16 x 16 MFMA accumulators: lane (c, g) of block (f, j) holds rows
// 4 g + 0..3 of column c.
template <int BM, int BN, int WM, int WN>
__device__ __forceinline__ void store_tile_rows(const GemmParams &p, long m0, long n0, long z, float *stg,
                                                const float4_t (&acc)[BM / WM / 16][BN / WN / 16]) {
  constexpr int WTN = BN / WN, FN = WTN / 16, LP = BN + 4;
  const int wave = threadIdx.x >> 6, wm = wave / WN, wn = wave % WN, lane = threadIdx.x & 63;
  const int c = lane & 15, g = lane >> 4;
  store_tile_passes<BM, BN, WM, WN>(p, m0, n0, z, stg, [&](int f) {
#pragma unroll
    for (int j = 0; j < FN; ++j)
#pragma unroll
      for (int r = 0; r < 4; ++r) stg[(wm * 16 + 4 * g + r) * LP + wn * WTN + 16 * j + c] = acc[f][j][r];
  });
}

// Grouped + XCD-aware mapping of the linear workgroup id to a (tile_m, tile_n) pair.
__device__ __forceinline__ void tile_coords(const GemmParams &p, int &tm, int &tn) {
  // Workgroup w runs on XCD w % 8; give XCD x the contiguous tile range
  // [x*base + min(x, rem), ...) of base (+1 for the first rem XCDs) tiles.
  const int total = p.tiles_m * p.tiles_n;
  int w = blockIdx.x;
  {
    const int base = total >> 3, rem = total & 7, x = w & 7;
    w = x * base + min(x, rem) + (w >> 3);
  }
  const int GROUP_M = p.group_m > 0 ? p.group_m : 4;
  const int in_group = GROUP_M * p.tiles_n;
  const int group = w / in_group;
  const int first_m = group * GROUP_M;
  const int gsize = min(p.tiles_m - first_m, GROUP_M);
  const int r = w - group * in_group;
  tm = first_m + r % gsize;
  tn = r / gsize;
}

// ------------------------------------------------------------------ tile loads
// A tile of R rows x CC contiguous elements is moved global -> registers -> LDS in
// 16-byte vectors (8 halves or 4 floats). VEC: the contiguous extent, the leading
// dimension and the base are multiples of the vector, so a vector is either fully
// in or fully out of bounds; otherwise elements are bounds-checked one by one.
template <typename T, int R, int CC, int NT, bool VEC>
struct TileLoader {
  static constexpr int EPV = 16 / sizeof(T);  // elements per vector
  static constexpr int VPR = CC / EPV;        // vectors per row
  static constexpr int NV = R * CC / EPV;
  static_assert(NV % NT == 0, "tile vectors must divide evenly among threads");
  static constexpr int VPT = NV / NT;
  u32x4_t reg[VPT];

  __device__ __forceinline__ void load(const T *base, long ld, long rlim, long clim) {
#pragma unroll
    for (int j = 0; j < VPT; ++j) {
      const int v = threadIdx.x + j * NT;
      const int r = v / VPR;
      const int c = (v % VPR) * EPV;
      if (VEC) {
        if (r < rlim && c < clim) {
          reg[j] = *reinterpret_cast<const u32x4_t *>(base + (long)r * ld + c);
        } else {
          reg[j] = u32x4_t{0, 0, 0, 0};
        }
      } else {
        T tmp[EPV];
#pragma unroll
        for (int e = 0; e < EPV; ++e)
          tmp[e] = (r < rlim && c + e < clim) ? base[(long)r * ld + c + e] : T(0);
        reg[j] = *reinterpret_cast<u32x4_t *>(tmp);
      }
    }
  }
  // Same-layout store: LDS row pitch P elements.
  template <int P>
  __device__ __forceinline__ void store(T *lds) const {
#pragma unroll
    for (int j = 0; j < VPT; ++j) {
      const int v = threadIdx.x + j * NT;
      const int r = v / VPR;
      const int c = (v % VPR) * EPV;
      *reinterpret_cast<u32x4_t *>(lds + r * P + c) = reg[j];
    }
  }
  // Transposed store: element (r, c + e) of the tile goes to lds[(c + e) * P + r].
  template <int P>
  __device__ __forceinline__ void store_t(T *lds) const {
#pragma unroll
    for (int j = 0; j < VPT; ++j) {
      const int v = threadIdx.x + j * NT;
      const int r = v / VPR;
      const int c = (v % VPR) * EPV;
      const T *e = reinterpret_cast<const T *>(&reg[j]);
#pragma unroll
      for (int q = 0; q < EPV; ++q) lds[(c + q) * P + r] = e[q];
    }
  }
  // Same-layout store for an MN-contiguous fp16 tile that frag_tr reads: the
  // 16-half column block is XOR-swizzled by bit 3 of the row (frag_tr undoes it).
  template <int P>
  __device__ __forceinline__ void store_sw(T *lds) const {
#pragma unroll
    for (int j = 0; j < VPT; ++j) {
      const int v = threadIdx.x + j * NT;
      const int r = v / VPR;
      const int c = (v % VPR) * EPV;
      *reinterpret_cast<u32x4_t *>(lds + r * P + (c ^ ((r & 8) << 1))) = reg[j];
    }
  }
};

// ------------------------------------------------------------------ fp16 fragments
// K-contiguous LDS ([rows][P]): lane (i = l%16, g = l/16) gets row0+i, k0+8g..+7.
__device__ __forceinline__ half8_t frag_kc(const _Float16 *lds, int P, int row0, int k0) {
  const int lane = threadIdx.x & 63;
  const _Float16 *p = lds + (row0 + (lane & 15)) * P + k0 + 8 * (lane >> 4);
  return *reinterpret_cast<const half8_t *>(p);
}

// MN-contiguous LDS ([k][P]): lane (i, g) gets elements (k0+8g+e, col0+i), e=0..7,
// via two transposing 64-bit reads (rows k0+8g..+3 and k0+8g+4..+7).
__device__ __forceinline__ half8_t frag_tr(const _Float16 *lds, int P, int col0, int k0) {
  const int lane = threadIdx.x & 63;
  const int s = lane & 15, g = lane >> 4;
  const int row = k0 + 8 * g + (s >> 2);
  const _Float16 *p0 = lds + row * P + ((col0 + 4 * (s & 3)) ^ ((row & 8) << 1));
  const _Float16 *p1 = p0 + 4 * P;
  trh4_t lo = __builtin_amdgcn_ds_read_tr16_b64_v4f16((LDS_AS trh4_t *)(p0));
  trh4_t hi = __builtin_amdgcn_ds_read_tr16_b64_v4f16((LDS_AS trh4_t *)(p1));
  const half4_t l4 = __builtin_bit_cast(half4_t, lo);
  const half4_t h4 = __builtin_bit_cast(half4_t, hi);
  return __builtin_shufflevector(l4, h4, 0, 1, 2, 3, 4, 5, 6, 7);
}

// ------------------------------------------------------------------ fp16 kernel
template <int BM, int BN, int BK, int WM, int WN, bool TA, bool TB, bool VEC>
__global__ void __launch_bounds__(WM * WN * 64) gemm_f16_kernel(GemmParams p) {
  constexpr int NT = WM * WN * 64;
  constexpr int WTM = BM / WM, WTN = BN / WN;  // wave tile
  constexpr int FM = WTM / 16, FN = WTN / 16;  // 16x16 blocks per wave
  static_assert(BK % 32 == 0 && WTM % 16 == 0 && WTN % 16 == 0, "tile shape");
  // LDS pitches (halves). gfx950's LDS has 64 four-byte banks. K-contiguous rows get
  // +8 halves: the 16 rows one 16-lane phase of ds_read_b128 touches then start on
  // distinct 4-bank groups. MN-contiguous rows get +32 halves (pitch = 16 or 48
  // banks mod 64) plus the row-bit-3 XOR of store_sw / frag_tr: the 8 rows (k0+8g+r,
  // g < 2, r < 4) one 32-lane phase of ds_read_b64_tr_b16 touches then cover all 64
  // banks exactly once.
  constexpr int PA = TA ? BM + 32 : BK + 8;
  constexpr int PB = TB ? BK + 8 : BN + 32;
  static_assert(TA ? (PA % 128 == 32 || PA % 128 == 96) : true, "MN-contiguous pitch");
  static_assert(TB ? true : (PB % 128 == 32 || PB % 128 == 96), "MN-contiguous pitch");
  constexpr int A_ELEMS = TA ? BK * PA : BM * PA;
  constexpr int B_ELEMS = TB ? BN * PB : BK * PB;
  __shared__ __attribute__((aligned(16))) _Float16 smem[2 * (A_ELEMS + B_ELEMS)];

  int tm, tn;
  tile_coords(p, tm, tn);
  const long m0 = (long)tm * BM, n0 = (long)tn * BN;
  const long z = blockIdx.z;
  const _Float16 *A = static_cast<const _Float16 *>(p.A) + z * p.strideA;
  const _Float16 *B = static_cast<const _Float16 *>(p.B) + z * p.strideB;

  const int wave = threadIdx.x >> 6;
  const int wm = wave / WN, wn = wave % WN;

  TileLoader<_Float16, TA ? BK : BM, TA ? BM : BK, NT, VEC> la;
  TileLoader<_Float16, TB ? BN : BK, TB ? BK : BN, NT, VEC> lb;

  auto load_tiles = [&](long k0) {
    if (TA) la.load(A + k0 * p.lda + m0, p.lda, p.K - k0, p.M - m0);
    else    la.load(A + m0 * p.lda + k0, p.lda, p.M - m0, p.K - k0);
    if (TB) lb.load(B + n0 * p.ldb + k0, p.ldb, p.N - n0, p.K - k0);
    else    lb.load(B + k0 * p.ldb + n0, p.ldb, p.K - k0, p.N - n0);
  };
  auto store_tiles = [&](int stage) {
    _Float16 *as = smem + stage * (A_ELEMS + B_ELEMS);
    _Float16 *bs = as + A_ELEMS;
    if (TA) la.template store_sw<PA>(as); else la.template store<PA>(as);
    if (TB) lb.template store<PB>(bs); else lb.template store_sw<PB>(bs);
  };

  float4_t acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j) acc[i][j] = float4_t{0.f, 0.f, 0.f, 0.f};

  const int nk = (int)((p.K + BK - 1) / BK);
  if (nk > 0) {
    load_tiles(0);
    store_tiles(0);
  }
  __syncthreads();

  for (int kt = 0; kt < nk; ++kt) {
    const bool more = kt + 1 < nk;
    if (more) load_tiles((long)(kt + 1) * BK);
    const _Float16 *as = smem + (kt & 1) * (A_ELEMS + B_ELEMS);
    const _Float16 *bs = as + A_ELEMS;
#pragma unroll
    for (int kk = 0; kk < BK; kk += 32) {
      half8_t af[FM], bf[FN];
#pragma unroll
      for (int i = 0; i < FM; ++i)
        af[i] = TA ? frag_tr(as, PA, wm * WTM + i * 16, kk) : frag_kc(as, PA, wm * WTM + i * 16, kk);
#pragma unroll
      for (int j = 0; j < FN; ++j)
        bf[j] = TB ? frag_kc(bs, PB, wn * WTN + j * 16, kk) : frag_tr(bs, PB, wn * WTN + j * 16, kk);
#pragma unroll
      for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(af[i], bf[j], acc[i][j], 0, 0, 0);
    }
    if (more) store_tiles((kt + 1) & 1);
    __syncthreads();
  }

  static_assert(WM * 16 * (BN + 4) * 4 <= 2 * (A_ELEMS + B_ELEMS) * 2, "epilogue staging exceeds LDS");
  store_tile_rows<BM, BN, WM, WN>(p, m0, n0, z, reinterpret_cast<float *>(smem), acc);
}

// ------------------------------------------------------------------ fp32 kernel
// v_mfma_f32_16x16x4_f32: lane (i, g) supplies A[i][k_g], B[k_g][j]. Within a
// 16-wide K chunk, MFMA step s uses k = 4g + s (the same K order for A and B):
//  * a K-contiguous operand is stored K-contiguous (pitch BK + 4) and each lane reads
//    its 4 steps as one 16-byte vector;
//  * an M/N-contiguous operand keeps its memory layout (k rows of BM or BN floats,
//    pitch + 4, so the 4 rows 4g + s of one step fall on distinct banks) and each lane
//    reads one float per step. Storing it transposed instead would turn every 16-byte
//    tile store into four 4-byte LDS writes;
//  * except NT with BK = 16: both operands K-contiguous put bank conflicts on both
//    16-byte fragment reads (25 M conflict cycles per operand at 4096^3), so both tiles
//    are stored transposed (four 4-byte writes, conflict-free for these loaders) and read
//    as M/N-contiguous ones: 4096^3 NT 1045 -> 1020 us; NN, TN and TT do not gain.
template <int BM, int BN, int BK, int WM, int WN, bool TA, bool TB, bool VEC>
__global__ void __launch_bounds__(WM * WN * 64) gemm_f32_kernel(GemmParams p) {
  constexpr int NT = WM * WN * 64;
  constexpr int WTM = BM / WM, WTN = BN / WN;
  constexpr int FM = WTM / 16, FN = WTN / 16;
  static_assert(BK % 16 == 0, "tile shape");
  constexpr bool XT = !TA && TB && BK == 16;  // NT: both tiles stored transposed
  constexpr bool MA = TA || XT, MB = !TB || XT;  // tile is M/N-contiguous in LDS
  constexpr int PA = MA ? BM + 4 : BK + 4;  // LDS pitches (floats)
  constexpr int PB = MB ? BN + 4 : BK + 4;
  constexpr int A_ELEMS = MA ? BK * PA : BM * PA;
  constexpr int B_ELEMS = MB ? BK * PB : BN * PB;
  __shared__ __attribute__((aligned(16))) float smem[2 * (A_ELEMS + B_ELEMS)];

  int tm, tn;
  tile_coords(p, tm, tn);
  const long m0 = (long)tm * BM, n0 = (long)tn * BN;
  const long z = blockIdx.z;
  const float *A = static_cast<const float *>(p.A) + z * p.strideA;
  const float *B = static_cast<const float *>(p.B) + z * p.strideB;

  const int wave = threadIdx.x >> 6;
  const int wm = wave / WN, wn = wave % WN;
  const int lane = threadIdx.x & 63;

  TileLoader<float, TA ? BK : BM, TA ? BM : BK, NT, VEC> la;
  TileLoader<float, TB ? BN : BK, TB ? BK : BN, NT, VEC> lb;

  auto load_tiles = [&](long k0) {
    if (TA) la.load(A + k0 * p.lda + m0, p.lda, p.K - k0, p.M - m0);
    else    la.load(A + m0 * p.lda + k0, p.lda, p.M - m0, p.K - k0);
    if (TB) lb.load(B + n0 * p.ldb + k0, p.ldb, p.N - n0, p.K - k0);
    else    lb.load(B + k0 * p.ldb + n0, p.ldb, p.K - k0, p.N - n0);
  };
  auto store_tiles = [&](int stage) {
    float *as = smem + stage * (A_ELEMS + B_ELEMS);
    float *bs = as + A_ELEMS;
    if constexpr (XT) {
      la.template store_t<PA>(as);
      lb.template store_t<PB>(bs);
    } else {
      la.template store<PA>(as);
      lb.template store<PB>(bs);
    }
  };

  float4_t acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j) acc[i][j] = float4_t{0.f, 0.f, 0.f, 0.f};

  const int nk = (int)((p.K + BK - 1) / BK);
  if (nk > 0) {
    load_tiles(0);
    store_tiles(0);
  }
  __syncthreads();

  const int li = lane & 15, lg = lane >> 4;
  for (int kt = 0; kt < nk; ++kt) {
    const bool more = kt + 1 < nk;
    if (more) load_tiles((long)(kt + 1) * BK);
    const float *as = smem + (kt & 1) * (A_ELEMS + B_ELEMS);
    const float *bs = as + A_ELEMS;
#pragma unroll
    for (int kc = 0; kc < BK; kc += 16) {
      float4_t af[FM], bf[FN];
#pragma unroll
      for (int i = 0; i < FM; ++i) {
        const int r = wm * WTM + i * 16 + li;
        if (MA) {
#pragma unroll
          for (int s = 0; s < 4; ++s) af[i][s] = as[(kc + 4 * lg + s) * PA + r];
        } else {
          af[i] = *reinterpret_cast<const float4_t *>(as + r * PA + kc + 4 * lg);
        }
      }
#pragma unroll
      for (int j = 0; j < FN; ++j) {
        const int c = wn * WTN + j * 16 + li;
        if (!MB) {
          bf[j] = *reinterpret_cast<const float4_t *>(bs + c * PB + kc + 4 * lg);
        } else {
#pragma unroll
          for (int s = 0; s < 4; ++s) bf[j][s] = bs[(kc + 4 * lg + s) * PB + c];
        }
      }
#pragma unroll
      for (int s = 0; s < 4; ++s)
#pragma unroll
        for (int i = 0; i < FM; ++i)
#pragma unroll
          for (int j = 0; j < FN; ++j)
            acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(af[i][s], bf[j][s], acc[i][j], 0, 0, 0);
    }
    if (more) store_tiles((kt + 1) & 1);
    __syncthreads();
  }

  static_assert(WM * 16 * (BN + 4) <= 2 * (A_ELEMS + B_ELEMS), "epilogue staging exceeds LDS");
  store_tile_rows<BM, BN, WM, WN>(p, m0, n0, z, smem, acc);
}

// The small-product kernels' end: wave w's partial tile goes to red[w], the workgroup adds
// the KW partials in wave order, ((w0 + w1) + w2) + ..., and applies the epilogue
// C = act(alpha * sum + beta * C + bias[col]) (C is not read when beta = 0).
template <int KW, int FM, int FN>
__device__ __forceinline__ void small_reduce_store(const GemmParams &p, float4_t (&red)[KW][FM * FN][64],
                                                   const float4_t (&acc)[FM][FN], long m0, long n0, long z) {
  constexpr int NF = FM * FN;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j) red[wave][i * FN + j][lane] = acc[i][j];
  __syncthreads();
  // thread (f, l) finishes lane l's four elements of fragment f: rows 4 (l >> 4) + 0..3,
  // column l & 15; wave w takes fragments w, w + KW, ...
  const int l = threadIdx.x & 63;
  float *C = p.C + z * p.strideC;
  for (int f = threadIdx.x >> 6; f < NF; f += KW) {
    float4_t v = red[0][f][l];
#pragma unroll
    for (int w = 1; w < KW; ++w) v = v + red[w][f][l];
    const long col = n0 + 16 * (f % FN) + (l & 15), row0 = m0 + 16 * (f / FN) + 4 * (l >> 4);
    if (col >= p.N) continue;
    const float bv = p.bias ? p.bias[col] : 0.0f;
    auto finish = [&](auto act_c) {
      constexpr int ACT = decltype(act_c)::value;
      const int act = ACT == kActRuntime ? p.act : ACT;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        if (row0 + e >= p.M) break;
        float *dst = C + (row0 + e) * p.ldc + col;
        const float old = p.beta != 0.0f ? *dst : 0.0f;
        *dst = apply_act(act, p.alpha * v[e] + p.beta * old + bv, p.act_alpha);
      }
    };
    switch (p.act) {
      case -1: finish(ActCode<-1>{}); break;
      case 0: finish(ActCode<0>{}); break;
      case 7: finish(ActCode<7>{}); break;
      default: finish(ActCode<kActRuntime>{}); break;
    }
  }
}

// ------------------------------------------------------------------ small products (fp32, fp16)
// Products too small to fill the chip with the tiled kernels (256^3 makes 16 workgroups of
// 64 x 64, on 16 of the 256 CUs, each wave a chain of 256 fp32 MFMAs). Here a workgroup
// computes a BM x BN = 16 FM x 16 FN tile and its KW waves split K: wave w sums the K steps
// [w S / KW, (w + 1) S / KW) of the S = ceil(K / KS) steps (KS = 16 elements for fp32, 32 for
// fp16). No operand is reused between waves, so the fragments go from global memory (L2)
// straight into the MFMA source registers, without LDS staging: lane (i, g) of a fragment
// takes row i and k = KS t + E g + s, s < E, as the tiled kernels do (fp32: E = 4, one
// v_mfma_f32_16x16x4_f32 per s; fp16: E = 8, one v_mfma_f32_16x16x32_f16 per step), a
// K-contiguous operand as one 16-byte vector when aligned. 64 elements of K are loaded before
// their MFMAs run (a second register set that loads the next ones during the MFMAs measured
// 10-20% slower: fewer waves fit). The KW partial tiles are added in LDS in wave order before
// the epilogue (small_reduce_store), so each element's summation order depends on K and KW
// alone: the same for all four transpose layouts, aligned or not.
// Per element type: the fragment vector V (E elements per lane and K step of KS elements)
// and the MFMA steps MPS of one K step.
template <typename T>
struct SmallOps;
template <>
struct SmallOps<float> {
  typedef float4_t V;
  static constexpr int E = 4, KS = 16, MPS = 4;
  static __device__ __forceinline__ float4_t mma(const V &a, const V &b, int s, float4_t c) {
    return __builtin_amdgcn_mfma_f32_16x16x4f32(a[s], b[s], c, 0, 0, 0);
  }
};
template <>
struct SmallOps<_Float16> {
  typedef half8_t V;
  static constexpr int E = 8, KS = 32, MPS = 1;
  static __device__ __forceinline__ float4_t mma(const V &a, const V &b, int, float4_t c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
  }
};

template <typename T, int KW, int FM, int FN, bool TA, bool TB, bool VEC, int KB = 64>
__global__ void __launch_bounds__(KW * 64) gemm_small_kernel(GemmParams p) {
  typedef SmallOps<T> Ops;
  typedef typename Ops::V V;
  constexpr int NF = FM * FN, U = KB / Ops::KS, E = Ops::E, KS = Ops::KS;  // KB elements of K per load batch
  __shared__ float4_t red[KW][NF][64];
  const long m0 = (long)(blockIdx.x / p.tiles_n) * 16 * FM, n0 = (long)(blockIdx.x % p.tiles_n) * 16 * FN;
  const long z = blockIdx.z;
  const T *A = static_cast<const T *>(p.A) + z * p.strideA;
  const T *B = static_cast<const T *>(p.B) + z * p.strideB;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, li = lane & 15, lg = lane >> 4;
  const long steps = (p.K + KS - 1) / KS;
  const long sb = steps * wave / KW, se = steps * (wave + 1) / KW;

  // One lane's E elements (k .. k + E - 1) of row r of op(A) or column r of op(B): rows past
  // the product and k past K read as zero.
  auto frag = [&](const T *X, long ld, bool kcontig, long r, bool rin, long k) {
    V v;
#pragma unroll
    for (int e = 0; e < E; ++e) v[e] = T(0);
    if (!rin) return v;
    if (kcontig) {
      const T *q = X + r * ld + k;
      if (VEC) {  // K is a multiple of E: the E elements are all inside or all past K
        if (k < p.K) v = *reinterpret_cast<const V *>(q);
      } else {
#pragma unroll
        for (int e = 0; e < E; ++e)
          if (k + e < p.K) v[e] = q[e];
      }
    } else {
#pragma unroll
      for (int e = 0; e < E; ++e)
        if (k + e < p.K) v[e] = X[(k + e) * ld + r];
    }
    return v;
  };

  float4_t acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j) acc[i][j] = float4_t{0.f, 0.f, 0.f, 0.f};
  for (long t0 = sb; t0 < se; t0 += U) {
    V af[U][FM], bf[U][FN];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const bool live = t0 + u < se;
      const long k = (t0 + u) * KS + E * lg;
#pragma unroll
      for (int i = 0; i < FM; ++i) {
        const long r = m0 + 16 * i + li;
        af[u][i] = frag(A, p.lda, !TA, r, live && r < p.M, k);
      }
#pragma unroll
      for (int j = 0; j < FN; ++j) {
        const long c = n0 + 16 * j + li;
        bf[u][j] = frag(B, p.ldb, TB, c, live && c < p.N, k);
      }
    }
#pragma unroll
    for (int u = 0; u < U; ++u)
#pragma unroll
      for (int s = 0; s < Ops::MPS; ++s)
#pragma unroll
        for (int i = 0; i < FM; ++i)
#pragma unroll
          for (int j = 0; j < FN; ++j) acc[i][j] = Ops::mma(af[u][i], bf[u][j], s, acc[i][j]);
  }
  small_reduce_store<KW, FM, FN>(p, red, acc, m0, n0, z);
}

// ------------------------------------------------------------------ fp16 DMA-ring kernel
// Large aligned fp16 GEMMs. Differences from gemm_f16_kernel:
//  * global -> LDS copies are buffer loads with the LDS-direct bit (16 bytes per lane
//    written to M0 + 16*lane): no staging VGPRs and no ds_write instructions;
//  * the LDS ring holds two slots of two consecutive K-tiles each (BK = 32, 64 KiB per
//    slot at 256 x 256): the DMA fills one slot while the other is multiplied (at
//    256 x 256 in two bursts, A then B, spread over the MFMAs), and only one barrier per
//    pair of K-tiles is needed;
//  * out-of-range lanes (rows past M/N, the K tail) get a buffer offset beyond the
//    descriptor's range, which the hardware turns into zeros;
//  * K-contiguous operands are stored in 1 KiB chunks of 8 rows x 64 k (both K-tiles
//    of a pair), each MFMA fragment one ds_read_b128 (lane octets copy whole 128-byte
//    lines; see kc8_slot);
//  * MN-contiguous operands keep their memory layout, rows of 2*BM (or 2*BN) bytes,
//    with the 32-byte block index XORed by hsw(k) so the 8 rows one 32-lane phase of
//    ds_read_b64_tr_b16 reads (k0+8g+r, g < 2, r < 4) fall on distinct banks;
//  * MFMA fragments are double-buffered in registers: tile k+1's fragments are read
//    while tile k's MFMAs run.
// The DMA is issued from inline assembly so the compiler does not track these LDS
// writes (it would otherwise wait for every outstanding load before each LDS read);
// the kernel orders them itself with s_waitcnt vmcnt and the barriers.
typedef int i32x4_t __attribute__((ext_vector_type(4)));

struct BufRsrc {
  i32x4_t r;
};

// Raw buffer descriptor: 48-bit base, stride 0, num_records ring::kNumRecords (offsets at
// or beyond it read as zero), gfx9 dword3.
__device__ __forceinline__ BufRsrc make_rsrc(const void *base) {
  const unsigned long long b = (unsigned long long)base;
  BufRsrc s;
  s.r.x = __builtin_amdgcn_readfirstlane((int)(b & 0xffffffffu));
  s.r.y = __builtin_amdgcn_readfirstlane((int)(b >> 32) & 0xffff);
  s.r.z = (int)ring::kNumRecords;
  s.r.w = 0x00020000;
  return s;
}

__device__ __forceinline__ void rsrc_advance(BufRsrc &s, long bytes) {
  unsigned long long b =
      ((unsigned long long)(unsigned)s.r.x) | ((unsigned long long)(unsigned)(s.r.y & 0xffff) << 32);
  b += (unsigned long long)bytes;
  s.r.x = __builtin_amdgcn_readfirstlane((int)(b & 0xffffffffu));
  s.r.y = __builtin_amdgcn_readfirstlane((int)(b >> 32) & 0xffff);
}

// 16 bytes per lane from the buffer at voff into LDS at lds + 16 * lane (lds is
// wave-uniform). M0 is saved and restored around the load.
__device__ __forceinline__ void dma16(const BufRsrc &s, unsigned voff, unsigned lds) {
  int saved;
  asm volatile(
      "s_mov_b32 %0, m0\n\t"
      "s_mov_b32 m0, %3\n\t"
      "buffer_load_dwordx4 %1, %2, 0 offen lds\n\t"
      "s_mov_b32 m0, %0"
      : "=&s"(saved)
      : "v"(voff), "s"(s.r), "s"(lds)
      : "memory");
}

using ring::hsw;
using ring::kc8_octet;
using ring::kc8_slot;
using ring::kOutOfRange;
using ring::msw32;

// s_waitcnt immediate that waits for vmcnt <= n only (vmcnt[3:0] in bits 3:0 and
// vmcnt[5:4] in bits 15:14; expcnt and lgkmcnt at their maxima).
constexpr int vmcnt_imm(int n) { return (n & 0xF) | ((n >> 4) << 14) | (0x7 << 4) | (0xF << 8); }

__device__ __forceinline__ unsigned lds_offset(const void *p) {
  return (unsigned)(unsigned long)(const LDS_AS void *)p;
}


// K-contiguous tiles: a 1 KiB DMA chunk holds rows 8c..8c+7 with the 64 k of a K-tile
// pair (128 bytes) each. Lane L copies 16 bytes of row 8c + (L >> 3), so each lane
// octet reads one whole 128-byte line: half the L1 requests of 16 rows x 64 bytes per
// chunk (NT 882 -> 836 us at 8192^3), and lane quads stay on one row (quads spread over
// four rows stalled the address unit on the L1 cache). The hardware writes lane L's
// bytes to slot L of the chunk, so the octet it loads is permuted: octet o of row r sits
// in slot 8 (r & 7) + (o ^ ((r >> 1) & 7)), and the 16 rows an MFMA fragment read
// touches (two chunks, fixed o) land on 16 distinct 16-byte bank groups (ring::kc8_slot,
// ring::kc8_octet).

// A scheduling region of NM MFMAs and NR LDS reads, interleaved 1:1 (then the rest).
template <int NM, int NR>
__device__ __forceinline__ void sched_interleave() {
  constexpr int NP = NR < NM ? NR : NM;
#pragma unroll
  for (int g = 0; g < NP; ++g) {
    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
    __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
  }
  if constexpr (NM > NP) __builtin_amdgcn_sched_group_barrier(0x008, NM - NP, 0);
  if constexpr (NR > NP) __builtin_amdgcn_sched_group_barrier(0x100, NR - NP, 0);
}

// The copy side of the fp16 ring for one output tile: each wave's share of a K-tile pair's
// 1 KiB DMA chunks into a ring slot. For a K-contiguous operand chunk c of a pair holds rows
// 8c..8c+7 of both K-tiles, octets as kc8_slot lays out. For an MN-contiguous one it belongs
// to tile h = c / (nchunks / 2) and holds k rows cl * (1024 / row bytes).. (cl = c %
// (nchunks / 2)) with 32-byte blocks XOR-swizzled by hsw(k). Each lane keeps its offset from
// the pair's start and the k (0..63) it covers; lanes whose rows or columns lie past M (or N)
// get the out-of-range offset.
template <int BM, int BN, int WM, int WN, bool TA, bool TB>
struct F16RingCopies {
  static constexpr int BK = 32, NW = WM * WN;
  static constexpr int OPA = BM * BK * 2, OPB = BN * BK * 2;  // bytes of one K-tile of A / B
  static constexpr int SLOT = 2 * (OPA + OPB);                // A tiles 2pp, 2pp+1, then B tiles
  static constexpr int CA = 2 * OPA / 1024, CB = 2 * OPB / 1024;
  static constexpr int IPA = CA / NW, IPB = CB / NW;  // 1 KiB DMA chunks per wave per pair
  static constexpr int LPW = IPA + IPB;
  static constexpr int RBA = BM * 2, RBB = BN * 2;  // LDS row bytes of MN-contiguous tiles (one k row)
  static_assert(CA % NW == 0 && CB % NW == 0 && IPA >= 1 && IPB >= 1, "DMA split");
  BufRsrc ra, rb;
  unsigned voa[IPA], vob[IPB];
  int kla[IPA], klb[IPB];
  long K, a_step, b_step;
  unsigned sbase;
  int wave;

  __device__ __forceinline__ F16RingCopies(const GemmParams &p, long m0, long n0, long z, const char *smem, int w,
                                           int lane)
      : K(p.K), wave(w) {
    const _Float16 *A = static_cast<const _Float16 *>(p.A) + z * p.strideA;
    const _Float16 *B = static_cast<const _Float16 *>(p.B) + z * p.strideB;
    ra = make_rsrc(A + ring::base_elems(!TA, m0, p.lda));
    rb = make_rsrc(B + ring::base_elems(TB, n0, p.ldb));
#pragma unroll
    for (int i = 0; i < IPA; ++i) {
      const ring::Copy cp = ring::plan_f16(!TA, wave * IPA + i, CA, RBA, p.lda, p.M - m0, lane);
      voa[i] = cp.vo;
      kla[i] = cp.kl;
    }
#pragma unroll
    for (int i = 0; i < IPB; ++i) {
      const ring::Copy cp = ring::plan_f16(TB, wave * IPB + i, CB, RBB, p.ldb, p.N - n0, lane);
      vob[i] = cp.vo;
      klb[i] = cp.kl;
    }
    a_step = ring::pair_step_bytes(!TA, BK, p.lda, 2);
    b_step = ring::pair_step_bytes(TB, BK, p.ldb, 2);
    sbase = lds_offset(smem);
  }

  // DMA of pair pp (K-tiles 2pp, 2pp+1) into slot `slot`, in parts: part q of NPRT copies
  // the q-th share of the wave's A chunks (q < NPRT / 2) or of its B chunks; the last part
  // also advances both descriptors to the next pair.
  __device__ __forceinline__ void issue(int pp, int slot, int q, int NPRT) {
    const unsigned st = sbase + (unsigned)(slot * SLOT);
    const int krem = ring::f16_krem(K, pp);
    const int half = NPRT / 2;
    if (q < half) {
#pragma unroll
      for (int i = 0; i < IPA; ++i)
        if (i * half / IPA == q)
          dma16(ra, ring::f16_offset({voa[i], kla[i]}, krem),
                __builtin_amdgcn_readfirstlane(st + (wave * IPA + i) * 1024));
    } else {
#pragma unroll
      for (int i = 0; i < IPB; ++i)
        if (i * half / IPB == q - half)
          dma16(rb, ring::f16_offset({vob[i], klb[i]}, krem),
                __builtin_amdgcn_readfirstlane(st + 2 * OPA + (wave * IPB + i) * 1024));
    }
    if (q == NPRT - 1) {
      rsrc_advance(ra, a_step);
      rsrc_advance(rb, b_step);
    }
  }
};

// Main loop of the ring kernel for one output tile (rows m0.., columns n0.., batch z),
// nk K-tiles: adds the products into acc. K-tiles go in pairs: slot pp & 1 holds tiles
// 2pp and 2pp+1 of A, then of B (a K-contiguous operand holds both tiles in each of its
// chunks; an MN-contiguous one has a region per tile). Per pair, the even step
// multiplies tile 2pp while reading tile 2pp+1's fragments from the same, already
// visible slot; the odd step waits for pair pp+1, passes the pair's one barrier,
// refills the slot just consumed with pair pp+2 and reads tile 2pp+2's fragments.
// Measured against a 4-stage ring of single K-tiles with one barrier per tile: NN
// 1139 -> 1170, TN 1139 -> 1179, TT 1145 -> 1156, NT equal (TFLOP/s, 8192^3). Leaves
// every DMA complete and every wave past a barrier, so the caller may reuse smem.
template <int BM, int BN, int WM, int WN, bool TA, bool TB, int NS>
__device__ __forceinline__ void ring_mainloop(const GemmParams &p, long m0, long n0, long z, int nk, char *smem,
                                              float4_t (&acc)[BM / WM / 16][BN / WN / 16]) {
  constexpr int NW = WM * WN;
  constexpr int WTM = BM / WM, WTN = BN / WN;
  constexpr int FM = WTM / 16, FN = WTN / 16;
  using Copies = F16RingCopies<BM, BN, WM, WN, TA, TB>;
  constexpr int OPA = Copies::OPA, OPB = Copies::OPB, SLOT = Copies::SLOT, LPW = Copies::LPW;
  constexpr int RBA = Copies::RBA, RBB = Copies::RBB;
  static_assert(NS >= 2 && (NS - 1) * LPW < 64, "ring slots within the vmcnt range");
  // Splitting each pair's DMA into two bursts (A at the barrier, B halfway through the
  // MFMAs) measured 2-4% faster at 256 x 256 with 8 waves (8192^3: NN 884 -> 851 us, NT
  // 872 -> 851 us) and 10% slower for the 4-wave 128 x 96 tiles of the C4 shape; four
  // bursts (A and B halves at quarter points) measured within 1% of two.
  constexpr int kDmaParts = NW >= 8 ? 2 : 1;
  static_assert(kDmaParts == 1 || FM % 4 == 0, "DMA burst split rows");
  static_assert((!TA || BM >= 128) && (TB || BN >= 128), "MN-contiguous rows need 8 XOR blocks of 32 B");
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const int wm = wave / WN, wn = wave % WN;
  Copies dma(p, m0, n0, z, smem, wave, lane);
  const int np = max(1, (nk + 1) >> 1);  // pairs the loop runs; tiles past nk are zeros
  auto issue = [&](int pp, int slot, int q, int NPRT) { dma.issue(pp, slot, q, NPRT); };

  auto frag_t = [&](const char *base, int col0, int rowb) -> half8_t {
    const int s = lane & 15, g = lane >> 4;
    const int k = 8 * g + (s >> 2);
    const int col = col0 + 4 * (s & 3);
    const char *p0 = base + k * rowb + (((col >> 4) ^ hsw(k)) << 5) + ((col & 15) << 1);
    const trh4_t lo = __builtin_amdgcn_ds_read_tr16_b64_v4f16((LDS_AS trh4_t *)(p0));
    const trh4_t hi = __builtin_amdgcn_ds_read_tr16_b64_v4f16((LDS_AS trh4_t *)(p0 + 4 * rowb));
    const half4_t l4 = __builtin_bit_cast(half4_t, lo);
    const half4_t h4 = __builtin_bit_cast(half4_t, hi);
    return __builtin_shufflevector(l4, h4, 0, 1, 2, 3, 4, 5, 6, 7);
  };

  auto frag_k = [&](const char *base, int row0, int h) -> half8_t {
    const int row = row0 + (lane & 15);
    return *reinterpret_cast<const half8_t *>(base + (row >> 3) * 1024 + 16 * kc8_slot(row, 4 * h + (lane >> 4)));
  };

  half8_t fa[2][FM], fb[2][FN];
  // Fragments of tile h of slot `slot` into register set `set`; part q of NPRT reads
  // the q-th share of the A and of the B fragments.
  auto read_part = [&](int slot, int h, int set, int q, int NPRT) {
    // K-contiguous operands hold both K-tiles of the pair in each chunk (no h offset)
    const char *sa = smem + slot * SLOT + (TA ? h * OPA : 0);
    const char *sb = smem + slot * SLOT + 2 * OPA + (TB ? 0 : h * OPB);
#pragma unroll
    for (int i = 0; i < FM; ++i)
      if (i * NPRT / FM == q)
        fa[set][i] = TA ? frag_t(sa, wm * WTM + i * 16, RBA) : frag_k(sa, wm * WTM + i * 16, h);
#pragma unroll
    for (int j = 0; j < FN; ++j)
      if (j * NPRT / FN == q)
        fb[set][j] = TB ? frag_k(sb, wn * WTN + j * 16, h) : frag_t(sb, wn * WTN + j * 16, RBB);
  };
  auto read_frags = [&](int slot, int h, int set) { read_part(slot, h, set, 0, 1); };
  constexpr int NDS = (TA ? 2 : 1) * FM + (TB ? 1 : 2) * FN;  // LDS read instructions per tile
  constexpr int NIL = NDS < FM * FN ? NDS : FM * FN;
  auto mfma_rows = [&](int set, int i0, int i1) {
#pragma unroll
    for (int i = i0; i < i1; ++i)
#pragma unroll
      for (int j = 0; j < FN; ++j)
        acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(fa[set][i], fb[set][j], acc[i][j], 0, 0, 0);
  };
  auto mfma_set = [&](int set) {
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
      for (int j = 0; j < FN; ++j)
        acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(fa[set][i], fb[set][j], acc[i][j], 0, 0, 0);
  };
  auto interleave = [&]() {
#pragma unroll
    for (int g = 0; g < NIL; ++g) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
    }
    __builtin_amdgcn_sched_group_barrier(0x008, FM * FN - NIL, 0);
  };

#pragma unroll
  for (int q = 0; q < NS; ++q) {  // the first NS pairs, one per slot
    issue(q, q, 0, 2);
    issue(q, q, 1, 2);
  }
  __builtin_amdgcn_s_waitcnt(vmcnt_imm((NS - 1) * LPW));
  __syncthreads();
  read_frags(0, 0, 0);
  int cur = 0, nxt = 1;  // slot of pair pp, slot of pair pp + 1
  for (int pp = 0; pp < np; ++pp) {
    // even step: multiply tile 2pp, read tile 2pp+1 (same slot, already visible)
    __builtin_amdgcn_sched_barrier(0);
    // With the DMA in bursts, NT / TN / TT also split the even step's fragment reads over
    // both halves of its MFMAs (8192^3: NT 821 -> 814, TN 843 -> 832, TT 839 -> 828 us);
    // NN measured 827 -> 830 us with it and keeps all reads in the first half.
    if constexpr (kDmaParts > 1 && (TA || TB)) {
#pragma unroll
      for (int q = 0; q < 2; ++q) {
        if (q) __builtin_amdgcn_sched_barrier(0);
        constexpr int NRH = (TA ? 2 : 1) * (FM / 2) + (TB ? 1 : 2) * (FN / 2);
        read_part(cur, 1, 1, q, 2);
        mfma_rows(0, q * (FM / 2), (q + 1) * (FM / 2));
        sched_interleave<(FM / 2) * FN, NRH>();
      }
    } else {
      read_frags(cur, 1, 1);
      mfma_set(0);
      interleave();
    }
    // odd step: pair pp+1 lands (the later NS - 2 pairs may still be in flight); refill this
    // pair's slot with pair pp+NS
    __builtin_amdgcn_sched_barrier(0);
    __builtin_amdgcn_s_waitcnt(vmcnt_imm((NS - 2) * LPW));
    __syncthreads();
    __builtin_amdgcn_sched_barrier(0);
    if constexpr (kDmaParts > 1) {
      // Two bursts: A's copies with the first R0 MFMA rows, B's with the rest; the next
      // tile's fragment reads are split between the two regions. B's burst after 3/4 of
      // the rows measured best for NN (8192^3: 808 -> 803 us against 1/2; 1/4: 824 us),
      // after 1/2 for NT / TN / TT (3/4 cost them 1-1.5%).
      constexpr int R0 = (!TA && !TB) ? 3 * FM / 4 : FM / 2;
      constexpr int NRH = (TA ? 2 : 1) * (FM / 2) + (TB ? 1 : 2) * (FN / 2);  // reads per part
      if constexpr (FM >= 8) {
        // Each burst follows the first MFMA row of its region, so the SIMD's MFMA pipe has
        // work while the CU's address unit takes the copies in (8192^3: NT 831 -> 821, TN
        // 845 -> 835, TT 848 -> 837, NN 835 -> 832 us; the 4-row C4 tiles lost 3% with it).
        mfma_rows(1, 0, 1);
        __builtin_amdgcn_sched_barrier(0);
        issue(pp + NS, cur, 0, 2);
        read_part(nxt, 0, 0, 0, 2);
        mfma_rows(1, 1, R0);
        sched_interleave<(R0 - 1) * FN, NRH>();
        __builtin_amdgcn_sched_barrier(0);
        mfma_rows(1, R0, R0 + 1);
        __builtin_amdgcn_sched_barrier(0);
        issue(pp + NS, cur, 1, 2);
        read_part(nxt, 0, 0, 1, 2);
        mfma_rows(1, R0 + 1, FM);
        sched_interleave<(FM - R0 - 1) * FN, NRH>();
      } else {
        issue(pp + NS, cur, 0, 2);
        read_part(nxt, 0, 0, 0, 2);
        mfma_rows(1, 0, R0);
        sched_interleave<R0 * FN, NRH>();
        __builtin_amdgcn_sched_barrier(0);
        issue(pp + NS, cur, 1, 2);
        read_part(nxt, 0, 0, 1, 2);
        mfma_rows(1, R0, FM);
        sched_interleave<(FM - R0) * FN, NRH>();
      }
    } else {
      issue(pp + NS, cur, 0, 2);
      issue(pp + NS, cur, 1, 2);
      read_frags(nxt, 0, 0);
      mfma_set(1);
      interleave();
    }
    cur = nxt;
    nxt = nxt + 1 == NS ? 0 : nxt + 1;
  }
  __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));
  __syncthreads();
}

// One workgroup per output tile, the whole K range. WPE: waves per SIMD the register
// allocation is sized for.
template <int BM, int BN, int WM, int WN, bool TA, bool TB, int WPE, int NS>
__global__ void __launch_bounds__(WM * WN * 64) __attribute__((amdgpu_waves_per_eu(WPE, WPE)))
gemm_f16_ring_kernel(GemmParams p) {
  constexpr int FM = BM / WM / 16, FN = BN / WN / 16;
  constexpr int RING = NS * 2 * (BM + BN) * 32 * 2;  // NS slots of two K-tiles of A and B
  __shared__ __attribute__((aligned(1024))) char smem[RING];
  int tm, tn;
  tile_coords(p, tm, tn);
  float4_t acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j) acc[i][j] = float4_t{0.f, 0.f, 0.f, 0.f};
  const long m0 = (long)tm * BM, n0 = (long)tn * BN, z = blockIdx.z;
  ring_mainloop<BM, BN, WM, WN, TA, TB, NS>(p, m0, n0, z, (int)((p.K + 31) / 32), smem, acc);
  static_assert(WM * 16 * (BN + 4) * 4 <= RING, "epilogue staging exceeds the ring");
  store_tile_rows<BM, BN, WM, WN>(p, m0, n0, z, reinterpret_cast<float *>(smem), acc);
}

// ------------------------------------------------------------------ 32 x 32 x 16 variant
// The NN 256 x 256 ring kernel on v_mfma_f32_32x32x16_f16, selected with
// GONNGPU_F16_MFMA32=1 (for measurement; the dispatch otherwise keeps 16 x 16 x 32). Same ring,
// copies, barriers and DMA bursts; each wave's 128 x 64 tile is 4 x 2 blocks of 32 x 32, and
// per K-tile it runs 16 MFMAs of 32 cycles where the product kernel runs 32 of 16, reading the
// same 16 fragments, and gives the product kernel's bits (the matrix unit accumulates K in the
// same order for both shapes). Measured at 8192^3 on one box, alternating libraries:
// 0.878-0.908 ms against 0.790-0.817 ms, the same MFMA-busy cycles and no LDS bank conflicts,
// but at the 1400 W board limit the clock settles at 1.60-1.72 GHz against 1.76-1.86 GHz. Each
// 32 x 32 x 16 instruction reads and writes 16 accumulator registers per lane in 32 cycles, the
// 16 x 16 x 32 one 4 in 16: twice the accumulator register traffic per flop.
typedef float float16_t __attribute__((ext_vector_type(16)));

template <int BM, int BN, int WM, int WN, int NS>
__device__ __forceinline__ void ring_mainloop_mf32(const GemmParams &p, long m0, long n0, long z, int nk, char *smem,
                                                   float16_t (&acc)[BM / WM / 32][BN / WN / 32]) {
  constexpr int WTM = BM / WM, WTN = BN / WN;
  constexpr int FM = WTM / 32, FN = WTN / 32;
  constexpr int NU = 2 * FM;  // MFMA units per K-tile: (k-step, 32-row block), FN instructions each
  using Copies = F16RingCopies<BM, BN, WM, WN, false, false>;
  constexpr int OPA = Copies::OPA, OPB = Copies::OPB, SLOT = Copies::SLOT, LPW = Copies::LPW;
  constexpr int RBB = Copies::RBB;
  static_assert(NS >= 2 && (NS - 1) * LPW < 64, "ring slots within the vmcnt range");
  static_assert(WM * WN >= 8 && BN >= 128 && NU >= 8, "two DMA bursts, 8 XOR blocks per B row");
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const int wm = wave / WN, wn = wave % WN;
  Copies dma(p, m0, n0, z, smem, wave, lane);
  const int np = max(1, (nk + 1) >> 1);
  // B (MN-contiguous): 16-lane group G reads k rows 16 st + 8 (G >> 1) + 0..3 (then + 4) of
  // columns col0 + 16 (G & 1) + 0..15, so lane l holds column col0 + (l & 31) with k
  // 16 st + 8 (l >> 5) + 0..7. With hsw(k), the 32 lanes of each half-wave read 8 distinct
  // 32-byte blocks (as the 16 x 16 fragment reads do).
  auto frag_t = [&](const char *base, int col0, int stp) -> half8_t {
    const int s = lane & 15, G = lane >> 4;
    const int k = 16 * stp + 8 * (G >> 1) + (s >> 2);
    const int col = col0 + 16 * (G & 1) + 4 * (s & 3);
    const char *p0 = base + k * RBB + (((col >> 4) ^ hsw(k)) << 5) + ((col & 15) << 1);
    const trh4_t lo = __builtin_amdgcn_ds_read_tr16_b64_v4f16((LDS_AS trh4_t *)(p0));
    const trh4_t hi = __builtin_amdgcn_ds_read_tr16_b64_v4f16((LDS_AS trh4_t *)(p0 + 4 * RBB));
    const half4_t l4 = __builtin_bit_cast(half4_t, lo);
    const half4_t h4 = __builtin_bit_cast(half4_t, hi);
    return __builtin_shufflevector(l4, h4, 0, 1, 2, 3, 4, 5, 6, 7);
  };
  // A (K-contiguous): lane l reads row row0 + (l & 31), octet 4 h + 2 st + (l >> 5) of the pair
  auto frag_k = [&](const char *base, int row0, int h, int stp) -> half8_t {
    const int row = row0 + (lane & 31);
    return *reinterpret_cast<const half8_t *>(base + (row >> 3) * 1024 +
                                              16 * kc8_slot(row, 4 * h + 2 * stp + (lane >> 5)));
  };
  half8_t fa[2][2][FM], fb[2][2][FN];  // [register set][k-step][block]
  auto read_part = [&](int slot, int h, int set, int q, int NPRT) {
    const char *sa = smem + slot * SLOT;
    const char *sb = smem + slot * SLOT + 2 * OPA + h * OPB;
#pragma unroll
    for (int a = 0; a < 2 * FM; ++a)
      if (a * NPRT / (2 * FM) == q) fa[set][a / FM][a % FM] = frag_k(sa, wm * WTM + (a % FM) * 32, h, a / FM);
#pragma unroll
    for (int b = 0; b < 2 * FN; ++b)
      if (b * NPRT / (2 * FN) == q) fb[set][b / FN][b % FN] = frag_t(sb, wn * WTN + (b % FN) * 32, b / FN);
  };
  constexpr int NDS = 2 * FM + 4 * FN;  // LDS read instructions per K-tile
  constexpr int NMT = NU * FN;          // MFMAs per K-tile
  // units in k-step-major order, so an accumulator's two updates per K-tile are FM units apart
  auto mfma_units = [&](int set, int u0, int u1) {
#pragma unroll
    for (int u = u0; u < u1; ++u)
#pragma unroll
      for (int j = 0; j < FN; ++j)
        acc[u % FM][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(fa[set][u / FM][u % FM], fb[set][u / FM][j],
                                                                acc[u % FM][j], 0, 0, 0);
  };
#pragma unroll
  for (int q = 0; q < NS; ++q) {
    dma.issue(q, q, 0, 2);
    dma.issue(q, q, 1, 2);
  }
  __builtin_amdgcn_s_waitcnt(vmcnt_imm((NS - 1) * LPW));
  __syncthreads();
  read_part(0, 0, 0, 0, 1);
  int cur = 0, nxt = 1;
  for (int pp = 0; pp < np; ++pp) {
    // even step: tile 2pp, reading tile 2pp+1's fragments
    __builtin_amdgcn_sched_barrier(0);
    read_part(cur, 1, 1, 0, 1);
    mfma_units(0, 0, NU);
    sched_interleave<NMT, NDS>();
    // odd step: wait for pair pp+1, refill this slot with pair pp+NS in two bursts (A after
    // the first unit, B after 3/4 of them), reading tile 2pp+2's fragments in between
    __builtin_amdgcn_sched_barrier(0);
    __builtin_amdgcn_s_waitcnt(vmcnt_imm((NS - 2) * LPW));
    __syncthreads();
    __builtin_amdgcn_sched_barrier(0);
    constexpr int R0 = 3 * NU / 4;
    constexpr int NRH = FM + 2 * FN;  // LDS reads per part
    mfma_units(1, 0, 1);
    __builtin_amdgcn_sched_barrier(0);
    dma.issue(pp + NS, cur, 0, 2);
    read_part(nxt, 0, 0, 0, 2);
    mfma_units(1, 1, R0);
    sched_interleave<(R0 - 1) * FN, NRH>();
    __builtin_amdgcn_sched_barrier(0);
    mfma_units(1, R0, R0 + 1);
    __builtin_amdgcn_sched_barrier(0);
    dma.issue(pp + NS, cur, 1, 2);
    read_part(nxt, 0, 0, 1, 2);
    mfma_units(1, R0 + 1, NU);
    sched_interleave<(NU - R0 - 1) * FN, NRH>();
    cur = nxt;
    nxt = nxt + 1 == NS ? 0 : nxt + 1;
  }
  __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));
  __syncthreads();
}

template <int BM, int BN, int WM, int WN, int WPE, int NS>
__global__ void __launch_bounds__(WM * WN * 64) __attribute__((amdgpu_waves_per_eu(WPE, WPE)))
gemm_f16_ring_mf32_kernel(GemmParams p) {
  constexpr int WTN = BN / WN, FM = BM / WM / 32, FN = WTN / 32, LP = BN + 4;
  constexpr int RING = NS * 2 * (BM + BN) * 32 * 2;
  __shared__ __attribute__((aligned(1024))) char smem[RING];
  static_assert(WM * 16 * (BN + 4) * 4 <= RING, "epilogue staging exceeds the ring");
  int tm, tn;
  tile_coords(p, tm, tn);
  float16_t acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.0f;
  const long m0 = (long)tm * BM, n0 = (long)tn * BN, z = blockIdx.z;
  ring_mainloop_mf32<BM, BN, WM, WN, NS>(p, m0, n0, z, (int)((p.K + 31) / 32), smem, acc);
  // lane l of a 32 x 32 block holds column l & 31, rows 8 (e >> 2) + 4 (l >> 5) + (e & 3);
  // pass f stages the block's rows 16 (f & 1) .. + 15, i.e. its elements e = 8 (f & 1) .. + 7
  const int wave = threadIdx.x >> 6, wm = wave / WN, wn = wave % WN, lane = threadIdx.x & 63;
  float *stg = reinterpret_cast<float *>(smem);
  store_tile_passes<BM, BN, WM, WN>(p, m0, n0, z, stg, [&](int f) {
    const int b = f >> 1, hh = f & 1;
#pragma unroll
    for (int j = 0; j < FN; ++j)
#pragma unroll
      for (int ii = 0; ii < 8; ++ii) {
        const int e = 8 * hh + ii;
        const int rr = 8 * ((e >> 2) - 2 * hh) + 4 * (lane >> 5) + (e & 3);
        stg[(wm * 16 + rr) * LP + wn * WTN + 32 * j + (lane & 31)] = acc[b][j][e];
      }
  });
}

// ------------------------------------------------------------------ fp32 DMA-ring kernel
// The fp16 ring's structure for fp32 operands. A K-tile is 16 floats (64 bytes per row,
// as a 32-half fp16 K-tile), so K-contiguous tiles use the same 1 KiB chunks of 8 rows x
// one K-tile pair (kc8 layout) and one ds_read_b128 per fragment gives lane (i, g) the
// four k = 4g..4g+3 that MFMA steps s = 0..3 take. MN-contiguous tiles keep their k rows
// (BM or BN floats, 256 to 1024 bytes) with the 16-byte block index XORed by
// msw32(k): the rows k and k + 4 that one 32-lane phase of a fragment read touches
// (lane groups g = 0, 1 at step s) land 16 banks apart; each lane reads its four k
// with ds_read_b32. Copies are whole 16-byte blocks checked by their first element, so
// every contiguous extent (K of a K-contiguous operand, M or N of an MN-contiguous one)
// must be a multiple of 4 floats, as the dispatch's vector path guarantees.

template <int BM, int BN, int WM, int WN, bool TA, bool TB, int NS>
__device__ __forceinline__ void ring_mainloop_f32(const GemmParams &p, long m0, long n0, long z, int nk, char *smem,
                                                  float4_t (&acc)[BM / WM / 16][BN / WN / 16]) {
  constexpr int BK = 16;
  constexpr int NW = WM * WN;
  constexpr int WTM = BM / WM, WTN = BN / WN;
  constexpr int FM = WTM / 16, FN = WTN / 16;
  constexpr int OPA = BM * BK * 4, OPB = BN * BK * 4;  // bytes of one K-tile of A / B
  constexpr int SLOT = 2 * (OPA + OPB);
  constexpr int CA = 2 * OPA / 1024, CB = 2 * OPB / 1024;
  constexpr int IPA = CA / NW, IPB = CB / NW;
  constexpr int LPW = IPA + IPB;
  constexpr int RBA = BM * 4, RBB = BN * 4;  // bytes of one k row of an MN-contiguous tile
  static_assert(CA % NW == 0 && CB % NW == 0 && IPA >= 1 && IPB >= 1, "DMA split");
  static_assert(NS >= 2 && (NS - 1) * LPW < 64, "ring slots within the vmcnt range");
  static_assert((!TA || RBA == 256 || RBA == 512 || RBA == 1024) && (TB || RBB == 256 || RBB == 512 || RBB == 1024),
                "MN-contiguous k rows of 64, 128 or 256 floats");
  // mn_bases folds the swizzle into fragment j's parity, which holds when a wave's first
  // column (or row) of an MN-contiguous operand starts a 32-float group.
  static_assert((!TA || WTM % 32 == 0) && (TB || WTN % 32 == 0), "MN-contiguous wave offsets in 32-float groups");
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const int wm = wave / WN, wn = wave % WN;

  BufRsrc ra, rb;
  unsigned voa[IPA], vob[IPB];
  // Byte offset (from the pair's start) of this lane's 16-byte copy in chunk c; rows or
  // columns past M (or N) get the out-of-range offset.
  // (K-contiguous chunk c: rows 8c..8c+7, the pair's 32 k (128 bytes) each; MN-contiguous
  // chunk cl of tile h: k rows cl * (1024 / rb_bytes) .., lane L filling slot L % bpr of its
  // row with block (L % bpr) ^ msw32(k).)
  auto plan = [&](bool kcontig, int c, int nchunks, int rb_bytes, long ld, long lim, unsigned &vo) {
    vo = ring::plan_f32(kcontig, c, nchunks, rb_bytes, ld, lim, lane);
  };
  {
    const float *A = static_cast<const float *>(p.A) + z * p.strideA;
    const float *B = static_cast<const float *>(p.B) + z * p.strideB;
    ra = make_rsrc(A + ring::base_elems(!TA, m0, p.lda));
    rb = make_rsrc(B + ring::base_elems(TB, n0, p.ldb));
  }
#pragma unroll
  for (int i = 0; i < IPA; ++i) plan(!TA, wave * IPA + i, CA, RBA, p.lda, p.M - m0, voa[i]);
#pragma unroll
  for (int i = 0; i < IPB; ++i) plan(TB, wave * IPB + i, CB, RBB, p.ldb, p.N - n0, vob[i]);
  const long a_step = ring::pair_step_bytes(!TA, BK, p.lda, 4);
  const long b_step = ring::pair_step_bytes(TB, BK, p.ldb, 4);
  const unsigned sbase = lds_offset(smem);
  const int np = max(1, (nk + 1) >> 1);

  // The caller guarantees K % (2 BK) == 0, so a pair is either whole or past the end of
  // K. Pairs past the end (the ring refills of the last NS steps, and the prologue's when
  // np < NS) still issue their LPW copies, which the vmcnt waits count, but through
  // descriptors with num_records 0: every offset is out of range, so they read zeros and
  // touch no memory. (A wave-uniform switch: per-lane offset selects would need temporary
  // VGPRs beside the fragments.)
  // Part q of NQ issues the wave's copies d (A's IPA, then B's IPB) with d * NQ / LPW == q;
  // the last part advances both descriptors.
  auto issue_part = [&](int pp, int slot, int q, int NQ) {
    const bool live = ring::f32_pair_live(pp, np);
    BufRsrc da = ra, db = rb;
    if (!live) {
      da.r.z = 0;
      db.r.z = 0;
    }
    const unsigned st = sbase + (unsigned)(slot * SLOT);
#pragma unroll
    for (int i = 0; i < IPA; ++i)
      if (i * NQ / LPW == q) dma16(da, voa[i], __builtin_amdgcn_readfirstlane(st + (wave * IPA + i) * 1024));
#pragma unroll
    for (int i = 0; i < IPB; ++i)
      if ((IPA + i) * NQ / LPW == q)
        dma16(db, vob[i], __builtin_amdgcn_readfirstlane(st + 2 * OPA + (wave * IPB + i) * 1024));
    if (q == NQ - 1) {
      rsrc_advance(ra, a_step);
      rsrc_advance(rb, b_step);
    }
  };
  auto issue = [&](int pp, int slot) { issue_part(pp, slot, 0, 1); };

  // K-contiguous: rows row0..row0+15 of K-tile h; MN-contiguous: columns col0..col0+15.
  auto frag_k = [&](const char *base, int row0, int h) -> float4_t {
    const int row = row0 + (lane & 15);
    return *reinterpret_cast<const float4_t *>(base + (row >> 3) * 1024 + 16 * kc8_slot(row, 4 * h + (lane >> 4)));
  };
  // MN-contiguous fragment j of a wave: lane (i, g) reads column wave_off + 16 j + i of k
  // rows 4g..4g+3. msw32(4g + s) = 4 (g & 1) flips bit 0 of j, so the byte offset is
  // lane_base(g, i) + 64 (j ^ (g & 1)) + s * rowb: one base for even j, one for odd j.
  auto mn_bases = [&](int wave_off, int rowb, int &even, int &odd) {
    const int i = lane & 15, g = lane >> 4;
    const int base = 4 * wave_off + 16 * (i >> 2) + 4 * (i & 3) + 4 * g * rowb;
    even = base + 64 * (g & 1);
    odd = base - 64 * (g & 1);
  };
  int mna_e = 0, mna_o = 0, mnb_e = 0, mnb_o = 0;
  if (TA) mn_bases(wm * WTM, RBA, mna_e, mna_o);
  if (!TB) mn_bases(wn * WTN, RBB, mnb_e, mnb_o);
  auto frag_mn = [&](const char *region, int j, int even, int odd, int rowb) -> float4_t {
    const char *p0 = region + ((j & 1) ? odd : even) + 64 * j;
    float4_t f;
#pragma unroll
    for (int s = 0; s < 4; ++s) f[s] = *reinterpret_cast<const float *>(p0 + s * rowb);
    return f;
  };

  constexpr int NSET = (TA && !TB) ? 1 : 2;
  float4_t fa[NSET][FM], fb[NSET][FN];
  // Part q of NQ reads the fragments i (of A) and j (of B) with i * NQ / FM == q and
  // j * NQ / FN == q.
  auto read_frags_part = [&](int slot, int h, int set, int q, int NQ) {
    const char *sa = smem + slot * SLOT + (TA ? h * OPA : 0);
    const char *sb = smem + slot * SLOT + 2 * OPA + (TB ? 0 : h * OPB);
#pragma unroll
    for (int i = 0; i < FM; ++i)
      if (i * NQ / FM == q)
        fa[set % NSET][i] = TA ? frag_mn(sa, i, mna_e, mna_o, RBA) : frag_k(sa, wm * WTM + i * 16, h);
#pragma unroll
    for (int j = 0; j < FN; ++j)
      if (j * NQ / FN == q)
        fb[set % NSET][j] = TB ? frag_k(sb, wn * WTN + j * 16, h) : frag_mn(sb, j, mnb_e, mnb_o, RBB);
  };
  auto read_frags = [&](int slot, int h, int set) { read_frags_part(slot, h, set, 0, 1); };
  constexpr int NDS = (TA ? 4 : 1) * FM + (TB ? 1 : 4) * FN;  // LDS read instructions per K-tile
  auto mfma_step = [&](int set, int s) {
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
      for (int j = 0; j < FN; ++j)
        acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(fa[set % NSET][i][s], fb[set % NSET][j][s], acc[i][j], 0, 0, 0);
  };
  auto mfma_set = [&](int set) {
#pragma unroll
    for (int s = 0; s < 4; ++s) mfma_step(set, s);
  };

  if constexpr (TA && !TB) {
    // Both operands MN-contiguous: one fragment set, refilled a component at a time. The
    // step-s MFMAs of a K-tile are the last readers of component s, so the next K-tile's
    // component s is read right after them (4 ds_read_b32 per fragment either way).
    auto read_comp = [&](int slot, int h, int s) {
      const char *sa = smem + slot * SLOT + h * OPA;
      const char *sb = smem + slot * SLOT + 2 * OPA + h * OPB;
#pragma unroll
      for (int i = 0; i < FM; ++i)
        fa[0][i][s] = *reinterpret_cast<const float *>(sa + ((i & 1) ? mna_o : mna_e) + 64 * i + s * RBA);
#pragma unroll
      for (int j = 0; j < FN; ++j)
        fb[0][j][s] = *reinterpret_cast<const float *>(sb + ((j & 1) ? mnb_o : mnb_e) + 64 * j + s * RBB);
    };
    // The step-s MFMAs run beside the reads of the next K-tile's component s - 1, whose
    // registers the step-(s-1) MFMAs have released; component 3 follows the last MFMAs.
    auto step = [&](int slot_next, int h_next, int refill_pp, int refill_slot) {
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        if (refill_pp >= 0) issue_part(refill_pp, refill_slot, s, 4);
#pragma unroll
        for (int i = 0; i < FM; ++i)
#pragma unroll
          for (int j = 0; j < FN; ++j)
            acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(fa[0][i][s], fb[0][j][s], acc[i][j], 0, 0, 0);
        if (s > 0) {
          read_comp(slot_next, h_next, s - 1);
          sched_interleave<FM * FN, FM + FN>();
        }
        __builtin_amdgcn_sched_barrier(0);
      }
      read_comp(slot_next, h_next, 3);
    };
#pragma unroll
    for (int q = 0; q < NS; ++q) issue(q, q);
    __builtin_amdgcn_s_waitcnt(vmcnt_imm((NS - 1) * LPW));
    __syncthreads();
#pragma unroll
    for (int s = 0; s < 4; ++s) read_comp(0, 0, s);
    int cur = 0, nxt = 1;
    for (int pp = 0; pp < np; ++pp) {
      __builtin_amdgcn_sched_barrier(0);
      step(cur, 1, -1, 0);  // multiply K-tile 2pp, read 2pp+1 (same slot)
      __builtin_amdgcn_sched_barrier(0);
      __builtin_amdgcn_s_waitcnt(vmcnt_imm((NS - 2) * LPW));
      __syncthreads();
      __builtin_amdgcn_sched_barrier(0);
      // multiply K-tile 2pp+1 and read the next pair's first (past the last pair: zeros),
      // refilling this pair's slot with pair pp + NS a quarter per MFMA step
      step(nxt, 0, pp + NS, cur);
      cur = nxt;
      nxt = nxt + 1 == NS ? 0 : nxt + 1;
    }
    __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));
    __syncthreads();
    return;
  }
#pragma unroll
  for (int q = 0; q < NS; ++q) issue(q, q);
  __builtin_amdgcn_s_waitcnt(vmcnt_imm((NS - 1) * LPW));
  __syncthreads();
  read_frags(0, 0, 0);
  int cur = 0, nxt = 1;
  for (int pp = 0; pp < np; ++pp) {
    __builtin_amdgcn_sched_barrier(0);
    read_frags(cur, 1, 1);
    mfma_set(0);
    sched_interleave<4 * FM * FN, NDS>();
    __builtin_amdgcn_sched_barrier(0);
    __builtin_amdgcn_s_waitcnt(vmcnt_imm((NS - 2) * LPW));
    __syncthreads();
    // The odd step in four parts, one per MFMA step: a quarter of the refill of this
    // pair's slot with pair pp + NS, a quarter of the next pair's first fragments, and the
    // step's MFMAs. Issued together after the barrier, the refill's copies held back every
    // wave's MFMAs while the CU's address unit took them in (4096^3 NN 952 -> 921 us, NT
    // 940 -> 908 us spread this way).
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      __builtin_amdgcn_sched_barrier(0);
      issue_part(pp + NS, cur, q, 4);
      read_frags_part(nxt, 0, 0, q, 4);
      mfma_step(1, q);
      sched_interleave<FM * FN, NDS / 4>();
    }
    __builtin_amdgcn_sched_barrier(0);
    cur = nxt;
    nxt = nxt + 1 == NS ? 0 : nxt + 1;
  }
  __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));
  __syncthreads();
}

template <int BM, int BN, int WM, int WN, bool TA, bool TB, int WPE, int NS>
__global__ void __launch_bounds__(WM * WN * 64) __attribute__((amdgpu_waves_per_eu(WPE, WPE)))
gemm_f32_ring_kernel(GemmParams p) {
  constexpr int FM = BM / WM / 16, FN = BN / WN / 16;
  constexpr int RING = NS * 2 * (BM + BN) * 16 * 4;  // NS slots of two K-tiles of A and B
  __shared__ __attribute__((aligned(1024))) char smem[RING];
  int tm, tn;
  tile_coords(p, tm, tn);
  float4_t acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j) acc[i][j] = float4_t{0.f, 0.f, 0.f, 0.f};
  const long m0 = (long)tm * BM, n0 = (long)tn * BN, z = blockIdx.z;
  ring_mainloop_f32<BM, BN, WM, WN, TA, TB, NS>(p, m0, n0, z, (int)((p.K + 15) / 16), smem, acc);
  static_assert(WM * 16 * (BN + 4) * 4 <= RING, "epilogue staging exceeds the ring");
  store_tile_rows<BM, BN, WM, WN>(p, m0, n0, z, reinterpret_cast<float *>(smem), acc);
}

// ------------------------------------------------------------------ dispatch
template <int BM, int BN, int BK, int WM, int WN, bool TA, bool TB, bool VEC>
hipError_t launch_f16(GemmParams p, long batch, hipStream_t s) {
  p.tiles_m = (int)((p.M + BM - 1) / BM);
  p.tiles_n = (int)((p.N + BN - 1) / BN);
  dim3 grid((unsigned)(p.tiles_m * p.tiles_n), 1, (unsigned)batch);
  hipLaunchKernelGGL((gemm_f16_kernel<BM, BN, BK, WM, WN, TA, TB, VEC>), grid, dim3(WM * WN * 64), 0, s, p);
  return hipGetLastError();
}

template <typename T, int KW, int FM, int FN, bool TA, bool TB, bool VEC, int KB = 64>
hipError_t launch_small(GemmParams p, long batch, hipStream_t s) {
  p.tiles_m = (int)((p.M + 16 * FM - 1) / (16 * FM));
  p.tiles_n = (int)((p.N + 16 * FN - 1) / (16 * FN));
  dim3 grid((unsigned)(p.tiles_m * p.tiles_n), 1, (unsigned)batch);
  hipLaunchKernelGGL((gemm_small_kernel<T, KW, FM, FN, TA, TB, VEC, KB>), grid, dim3(KW * 64), 0, s, p);
  return hipGetLastError();
}

// ------------------------------------------------------------------ NN products of 1-4 rows (GEMV)
// C = act(alpha X W + beta C + bias) for X of R <= 4 rows (row-major), W stored K x N
// (N-contiguous), batch 1: HBM-bound on reading W once, at 2 R flops per W element, so the MFMA
// layout's 16-row fragments would be mostly padding and the tiled kernels' few column tiles
// stream W from few CUs. Lane l of a workgroup owns columns n0 + E l .. + E - 1 (4 bytes of each
// row of W, so a wave's load is 256 contiguous bytes); the KW waves split K into contiguous
// ranges, each summed in k order with fmaf on the VALU, and the partials are added in LDS in wave
// order before the epilogue. X's entries are uniform across the workgroup.
template <typename T, int R, int E, int KW>
__global__ void __launch_bounds__(KW * 64) gemv_nn_kernel(GemmParams p) {
  __shared__ float red[KW][R][64 * E];
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const long nb = (long)blockIdx.x * 64 * E, n0 = nb + (long)lane * E;
  const T *__restrict__ W = static_cast<const T *>(p.B);
  const T *__restrict__ X = static_cast<const T *>(p.A);
  const long kb = p.K * wave / KW, ke = p.K * (wave + 1) / KW;
  float acc[R][E];
#pragma unroll
  for (int m = 0; m < R; ++m)
#pragma unroll
    for (int e = 0; e < E; ++e) acc[m][e] = 0.0f;
  if (n0 < p.N) {  // N is a multiple of E: the E columns are all inside or all past N
    typedef T VE __attribute__((ext_vector_type(E == 1 ? 2 : E)));
    auto step = [&](long k) {
      T w[E];
      if constexpr (E == 1) {
        w[0] = W[k * p.ldb + n0];
      } else {  // n0 and the pitch are even: one 4-byte load
        const VE v = *reinterpret_cast<const VE *>(W + k * p.ldb + n0);
#pragma unroll
        for (int e = 0; e < E; ++e) w[e] = v[e];
      }
#pragma unroll
      for (int m = 0; m < R; ++m) {
        const float x = (float)X[m * p.lda + k];
#pragma unroll
        for (int e = 0; e < E; ++e) acc[m][e] = fmaf(x, (float)w[e], acc[m][e]);
      }
    };
    long k = kb;
    for (; k + 8 <= ke; k += 8) {
#pragma unroll
      for (int u = 0; u < 8; ++u) step(k + u);
    }
    for (; k < ke; ++k) step(k);
  }
#pragma unroll
  for (int m = 0; m < R; ++m)
#pragma unroll
    for (int e = 0; e < E; ++e) red[wave][m][lane * E + e] = acc[m][e];
  __syncthreads();
  float *C = p.C;
  for (int o = threadIdx.x; o < R * 64 * E; o += KW * 64) {
    const int m = o / (64 * E), c = o % (64 * E);
    const long n = nb + c;
    if (n >= p.N) continue;
    float v = red[0][m][c];
#pragma unroll
    for (int w = 1; w < KW; ++w) v += red[w][m][c];
    float *dst = C + m * p.ldc + n;
    const float old = p.beta != 0.0f ? *dst : 0.0f;
    *dst = apply_act(p.act, p.alpha * v + p.beta * old + (p.bias ? p.bias[n] : 0.0f), p.act_alpha);
  }
}

template <typename T, int R>
hipError_t launch_gemv_r(const GemmParams &p, hipStream_t s) {
  constexpr int E = sizeof(T) == 2 ? 2 : 1;  // 4 bytes per lane and row of W
  const unsigned grid = (unsigned)((p.N + 64 * E - 1) / (64 * E));
  hipLaunchKernelGGL((gemv_nn_kernel<T, R, E, 16>), dim3(grid), dim3(1024), 0, s, p);
  return hipGetLastError();
}

// The NN GEMV kernel for a product of M <= 4 rows (batch 1, W aligned, N a multiple of 4 or 8).
template <typename T>
hipError_t launch_gemv(const GemmParams &p, hipStream_t s) {
  switch (p.M) {
    case 1: return launch_gemv_r<T, 1>(p, s);
    case 2: return launch_gemv_r<T, 2>(p, s);
    case 3: return launch_gemv_r<T, 3>(p, s);
    default: return launch_gemv_r<T, 4>(p, s);
  }
}

// The small-product kernel of shape code 100 KW + 10 FM + FN; hipErrorInvalidValue for
// another code.
template <typename T, bool TA, bool TB, bool VEC>
hipError_t launch_small_code(int code, const GemmParams &p, long batch, hipStream_t s) {
  switch (code) {
    case 411: return launch_small<T, 4, 1, 1, TA, TB, VEC>(p, batch, s);
    case 811: return launch_small<T, 8, 1, 1, TA, TB, VEC>(p, batch, s);
    case 1611: return launch_small<T, 16, 1, 1, TA, TB, VEC>(p, batch, s);
    case 422: return launch_small<T, 4, 2, 2, TA, TB, VEC>(p, batch, s);
    case 822: return launch_small<T, 8, 2, 2, TA, TB, VEC>(p, batch, s);
    default: return hipErrorInvalidValue;
  }
}

template <int BM, int BN, int BK, int WM, int WN, bool TA, bool TB, bool VEC>
hipError_t launch_f32(GemmParams p, long batch, hipStream_t s) {
  p.tiles_m = (int)((p.M + BM - 1) / BM);
  p.tiles_n = (int)((p.N + BN - 1) / BN);
  dim3 grid((unsigned)(p.tiles_m * p.tiles_n), 1, (unsigned)batch);
  hipLaunchKernelGGL((gemm_f32_kernel<BM, BN, BK, WM, WN, TA, TB, VEC>), grid, dim3(WM * WN * 64), 0, s, p);
  return hipGetLastError();
}

template <int BM, int BN, int WM, int WN, bool TA, bool TB, int WPE = 2, int NS = 2>
hipError_t launch_f16_ring(GemmParams p, long batch, hipStream_t s) {
  p.tiles_m = (int)((p.M + BM - 1) / BM);
  p.tiles_n = (int)((p.N + BN - 1) / BN);
  dim3 grid((unsigned)(p.tiles_m * p.tiles_n), 1, (unsigned)batch);
  hipLaunchKernelGGL((gemm_f16_ring_kernel<BM, BN, WM, WN, TA, TB, WPE, NS>), grid, dim3(WM * WN * 64), 0, s, p);
  return hipGetLastError();
}

template <int BM, int BN, int WM, int WN, bool TA, bool TB, int WPE = 2, int NS = 2>
hipError_t launch_f32_ring(GemmParams p, long batch, hipStream_t s) {
  p.tiles_m = (int)((p.M + BM - 1) / BM);
  p.tiles_n = (int)((p.N + BN - 1) / BN);
  dim3 grid((unsigned)(p.tiles_m * p.tiles_n), 1, (unsigned)batch);
  hipLaunchKernelGGL((gemm_f32_ring_kernel<BM, BN, WM, WN, TA, TB, WPE, NS>), grid, dim3(WM * WN * 64), 0, s, p);
  return hipGetLastError();
}

// The ring kernel's 32-bit buffer offsets reach 256 rows (K-contiguous) or 32 k-rows
// (MN-contiguous) past the tile base.
bool ring_offsets_fit(const GemmParams &p) { return p.lda < (1L << 21) && p.ldb < (1L << 21); }

// The fp16 ring kernel's tile from a time model. A round is 256 tiles (one per CU) for the
// one-workgroup-per-CU tiles (256x256 and 128x192, 8 waves; 128x128 with 8 waves when one
// round holds every tile) and 512 for the two-per-CU ones (128x128 and 128x96, 4 waves).
// Each tile type takes a measured time per round, relative to a round of 256x256 tiles at
// the same K: 128x192 0.509, 128x128 8-wave 0.508; two co-resident 128x128 0.638 (0.52 for
// one alone), 128x96 0.542 (0.43 alone, estimated). A last, partial round costs its fill
// fraction but at least 0.75 of a full one: with fewer CUs busy the power-limited clock
// rises (3072^3: 144 tiles of 256x256 on 256 CUs take 0.75 of a full round's time), so a
// 256x256 round that is half full still beats twice the 128x128 tiles. The model picks the
// measured best of these tiles at n^3 from 1536 to 6144 and at M x 11008 x 4096 for M =
// 512..2048, NT and TT (3072^3: 63 us against 82 us for the earlier 128x128 choice; 1536 x
// 11008 x 4096 NT: 147 us against 179 us for 256x256; the 512 x 11008 x 4096 linear layer:
// 128x192).
enum class F16Tile { k256, k128w8, k128w4, k192, k96 };
struct F16Choice {
  double cost;
  F16Tile tile;
};

inline double f16_rounds1(long t, double r, double fl = 0.75) {
  const long u = t % 256;
  return (double)(t / 256) * r + (u ? r * fmax(fl, u / 256.0) : 0.0);
}
// A last round of two-per-CU tiles with more than 256 tiles (some CUs run two, some one)
// costs 0.325 + 0.69 u / 512 of a full one, and never less than a full round of one per CU:
// 512 x 12288 x 4096 NT with 384 tiles of 128 x 128 took 0.84 of the 512-tile round
// (57.2 against 67.9 us), 512 x 14336 x 4096 with 448 tiles 0.93 (63.0 us). With the 0.75
// floor alone the model took those 384 tiles (57.2 us) over one full round of 256 tiles of
// 128 x 192 (51.5 us); same at 1024 x 6144 and 2048 x 3072.
inline double f16_rounds2(long t, double r2, double r1, double fl = 0.75) {
  const long u = t % 512;
  if (u == 0) return (double)(t / 512) * r2;
  if (u <= 256) return (double)(t / 512) * r2 + r1 * fmax(fl, u / 256.0);
  const double f = fmax(fmax(fl, u / 512.0), fmax(0.325 + 0.69 * (u / 512.0), r1 / r2));
  return (double)(t / 512) * r2 + r2 * f;
}

template <bool TB>
F16Choice f16_best(long M, long N, long batch) {
  const long tiles256 = ((M + 255) / 256) * ((N + 255) / 256) * batch;
  const long tiles128 = ((M + 127) / 128) * ((N + 127) / 128) * batch;
  F16Choice b{f16_rounds1(tiles256, 1.0), F16Tile::k256};
  // When one round of 128 x 128 tiles holds the product, the smaller tiles' partial rounds
  // are priced as full ones: the 0.75 floor models the clock a power-limited round of
  // 256 x 256 tiles gains with fewer CUs busy, and the lighter tiles did not show it (NT,
  // forced choices, us: 2048^2 x 4096 128x128 45.0 against 128x192 on 176 CUs 47.2;
  // 2048^3 25.7 against 27.7; 1536^2 x 4096 128x96 41.6 against 128x128 42.6).
  const double fl = tiles128 <= 256 ? 1.0 : 0.75;
  const double c128 = tiles128 <= 256 ? f16_rounds1(tiles128, 0.508, fl) : f16_rounds2(tiles128, 0.638, 0.52);
  if (c128 < b.cost) b = {c128, tiles128 <= 256 ? F16Tile::k128w8 : F16Tile::k128w4};
  if constexpr (TB) {
    // 128 x 192 and 128 x 96 only for a K-contiguous B: 384- and 192-byte MN-contiguous rows
    // would not take the 32-byte block swizzle of the transposing reads.
    const long tiles192 = ((M + 127) / 128) * ((N + 191) / 192) * batch;
    const long tiles96 = ((M + 127) / 128) * ((N + 95) / 96) * batch;
    const double c192 = f16_rounds1(tiles192, 0.509, fl), c96 = f16_rounds2(tiles96, 0.542, 0.43, fl);
    if (c192 < b.cost) b = {c192, F16Tile::k192};
    if (c96 < b.cost) b = {c96, F16Tile::k96};
  }
  return b;
}

template <bool TA, bool TB>
hipError_t launch_f16_tile(const GemmParams &p, long batch, hipStream_t s, F16Tile t) {
  switch (t) {
    case F16Tile::k256:
      if constexpr (!TA && !TB) {
        const char *mf = getenv("GONNGPU_F16_MFMA32");  // the measured 32 x 32 x 16 variant
        if (mf && mf[0] == '1') {
          GemmParams q = p;
          q.tiles_m = (int)((q.M + 255) / 256);
          q.tiles_n = (int)((q.N + 255) / 256);
          dim3 grid((unsigned)(q.tiles_m * q.tiles_n), 1, (unsigned)batch);
          hipLaunchKernelGGL((gemm_f16_ring_mf32_kernel<256, 256, 2, 4, 2, 2>), grid, dim3(512), 0, s, q);
          return hipGetLastError();
        }
      }
      return launch_f16_ring<256, 256, 2, 4, TA, TB>(p, batch, s);
    case F16Tile::k128w8:
      return launch_f16_ring<128, 128, 2, 4, TA, TB>(p, batch, s);
    case F16Tile::k128w4:
      return launch_f16_ring<128, 128, 2, 2, TA, TB>(p, batch, s);
    default:
      if constexpr (TB) {
        // 128 x 192: 8 waves, one workgroup per CU and a ring of three K-tile pairs (120 KiB),
        // two pairs in flight (the 512 x 11008 x 4096 linear layer: 49.0 -> 46.9 us ReLU
        // against two-slot 128 x 96 tiles)
        if (t == F16Tile::k192) return launch_f16_ring<128, 192, 2, 4, TA, TB, 2, 3>(p, batch, s);
        return launch_f16_ring<128, 96, 2, 2, TA, TB>(p, batch, s);
      }
      return hipErrorInvalidValue;  // f16_best offers these tiles only for a K-contiguous B
  }
}

// NN products of at most 4 rows (batch 1) take the GEMV kernel where it measured faster than the
// tiled and small-product kernels on a grid of M 1-4, N 512-32768, K 512-11008 (kernel times,
// tiled -> GEMV): fp32 1 x 11008 x 4096 54.4 -> 28.5 us (6.3 TB/s of W), 2 x 16384 x 2048 37.3 ->
// 21.0 us, 4 x 11008 x 4096 54.9 -> 43.4 us, 1 x 4096 x 4096 24.8 -> 20.2 us; fp16 1 x 16384 x
// 2048 18.2 -> 12.1 us, 2 x 2048 x 2048 16.8 -> 9.7 us, 4 x 32768 x 1024 15.2 -> 12.1 us. With
// fewer columns its grid has too few workgroups (N / 64 or N / 128 of them) and with more rows
// the VALU work grows: fp32 2 x 4096 x 11008 52.8 against 70.0 us, fp16 4 x 4096 x 4096 13.7
// against 27.1 us stay on the other kernels.
inline bool gemv_nn(long M, long N, long K, long batch, bool f16) {
  if (batch != 1 || M > 4) return false;
  if (!f16) return N >= 11008 || (M <= 2 && N >= 8192) || (M == 1 && N >= 4096);
  if (M <= 2 && (N >= 8192 || (N >= 1024 && N <= 2048 && K >= 1024))) return true;
  return N >= 16384;
}

// Skinny products in the linear-layer layout Y = X W^T (A row-major, B = W stored N x K,
// K-contiguous; at most 16 rows, batch 1, N and K of 2048 and more) are bound by reading W
// once from HBM. The small-product kernel with 16 x 16 tiles reads each W element once, as one
// 16-byte vector per lane and K step, and each tile's A rows from L2, and its K-splitting waves
// keep more loads in flight than the tiled kernels' few workgroups: up to 4096 waves (16 per
// workgroup while ceil(N / 16) <= 256, 8 while <= 512, else 4). Kernel times on MI355X (tiled
// -> this): fp32 1 x 11008 x 4096 54.9 -> 33.9 us (5.3 TB/s of W), 8 x 4096 x 8192 38.9 ->
// 28.4 us, 16 x 16384 x 4096 81.8 -> 63.5 us; fp16 1 x 4096 x 2048 17.0 -> 6.1 us, 2 x 11008 x
// 4096 22.1 -> 16.5 us, 16 x 4096 x 4096 14.0 -> 10.4 us. The bounds leave out the shapes where
// it lost on a grid of M 1-16, N 2048-16384, K 2048-8192: fp32 past 2 rows needs N >= 4096 (16 x
// 2048 x 8192: 25.6 against 31.6 us) and M N K < 2^31; fp16 past 2 rows needs M N <= 65536 and
// K <= 4096 (8 x 16384 x 8192: 45.8 against 50.5 us). With W stored K x N (NN) the kernel's W
// loads are 4- or 2-byte scalars and it ran 1.1-5x slower than the tiled kernels, so other
// layouts keep them; a skinny NT product therefore differs from the same product in NN in its
// rounding (K summed in four to sixteen wave ranges), both within the fp32 bar.
inline int skinny_tile(long M, long N, long K, long batch, bool f16, bool ta, bool tb) {
  if (ta || !tb || batch != 1 || M > 16 || N < 2048 || K < 2048) return 0;
  if (M > 2) {
    if (f16 && (M * N > 65536 || K > 4096)) return 0;
    if (!f16 && (N < 4096 || (double)M * N * K >= (double)(1L << 31))) return 0;
  }
  const long t16 = (N + 15) / 16;
  return t16 * 16 <= 4096 ? 1611 : t16 * 8 <= 4096 ? 811 : 411;
}

// The small-product kernel's shape for an fp16 product (100 KW + 10 FM + FN), or 0 for the
// tiled kernels. fp16 MFMAs are 8x the fp32 rate, so the 64 x 64 register-staged kernel stays
// ahead from fewer tiles than in fp32: the small kernel is taken for at most 16 of them, for
// K up to 1024 or below 2^24 multiply-adds in all (no split-K there), always with 16 x 16
// workgroup tiles and 16 waves from 24 32-element K steps (K > 736), 8 from 8 (K > 224), else
// 4: with fp16 a wave's K step is one MFMA, and more waves with fewer steps each measured
// faster. Kernel times on MI355X (rocprofv3 kernel trace), tiled -> small, NN: 256^3 5.70 ->
// 4.47 us; 100 x 130 x 1000 30.9 -> 9.5 us; 64 x 128 x 784 9.0 -> 6.1 us; 256^2 x 1024 10.2
// -> 6.9 us; 16 x 16 x 4096 29.1 -> 12.8 us. 384^2 and larger, and 64^2 x 4096, stay on the
// tiled kernels (4.5 against 4.6 us at 384^2 x 64, 11.9 against 13.9 us at 64^2 x 4096).
inline int f16_small_tile(long M, long N, long K, long batch, bool ta, bool tb) {
  if (const int c = skinny_tile(M, N, K, batch, true, ta, tb)) return c;
  const long tiles64 = ((M + 63) / 64) * ((N + 63) / 64) * batch;
  if (tiles64 > 16) return 0;
  if (!(K <= 1024 || (double)M * N * K * batch < (double)(1L << 24))) return 0;
  const long steps = (K + 31) / 32;
  return steps >= 24 ? 1611 : steps >= 8 ? 811 : 411;
}

template <bool TA, bool TB, bool VEC>
hipError_t pick_f16(const GemmParams &p, long batch, hipStream_t s) {
  if (const int code = f16_small_tile(p.M, p.N, p.K, batch, TA, TB)) return launch_small_code<_Float16, TA, TB, VEC>(code, p, batch, s);
  if constexpr (!VEC) {
    // Unaligned shapes take the element-wise load path on the smallest tile only.
    return launch_f16<64, 64, 64, 2, 2, TA, TB, VEC>(p, batch, s);
  } else {
    const long tiles256 = ((p.M + 255) / 256) * ((p.N + 255) / 256) * batch;
    const long tiles128 = ((p.M + 127) / 128) * ((p.N + 127) / 128) * batch;
    if (tiles128 >= 128 && ring_offsets_fit(p)) {
      const F16Choice whole = f16_best<TB>(p.M, p.N, batch);
      if (batch == 1) {
        // Two launches over row blocks, rows 0..256k-1 on 256x256 tiles and the rest on the
        // remainder's own best tile, when the model puts that at least 10% under one launch:
        // a partial round of 256x256 tiles becomes a fuller one plus a round of smaller
        // tiles. Each output element still comes from one tile in the same K order, so the
        // result is bit-identical. fp16 4608^3: 224.5 -> 188.7 us (rows split at 3328); 6144^3:
        // 415 -> 375 us (5120); at 5120^3, 3072^3 and 2560^3 every split measured slower, and
        // the model keeps those in one launch.
        const long tm = (p.M + 255) / 256, tn = (p.N + 255) / 256;
        double best = 0.9 * whole.cost;
        long k_best = 0;
        F16Tile bottom = F16Tile::k256;
        for (long k = 1; k < tm; ++k) {
          const F16Choice b = f16_best<TB>(p.M - 256 * k, p.N, 1);
          const double c = f16_rounds1(k * tn, 1.0) + b.cost;
          if (c < best) best = c, k_best = k, bottom = b.tile;
        }
        if (k_best > 0) {
          GemmParams top = p, bot = p;
          top.M = 256 * k_best;
          bot.M = p.M - top.M;
          bot.A = static_cast<const _Float16 *>(p.A) + (TA ? top.M : top.M * p.lda);
          bot.C = p.C + top.M * p.ldc;
          if (hipError_t e = launch_f16_ring<256, 256, 2, 4, TA, TB>(top, 1, s)) return e;
          return launch_f16_tile<TA, TB>(bot, 1, s, bottom);
        }
      }
      return launch_f16_tile<TA, TB>(p, batch, s, whole.tile);
    }
    if (tiles256 >= 512) return launch_f16<256, 256, 64, 2, 4, TA, TB, VEC>(p, batch, s);
    if (tiles128 >= 128) return launch_f16<128, 128, 64, 2, 2, TA, TB, VEC>(p, batch, s);
    return launch_f16<64, 64, 64, 2, 2, TA, TB, VEC>(p, batch, s);
  }
}

// The fp32 ring's tile (K a multiple of 32): each candidate's time is modelled as its rounds
// (ceil(tiles / 256), the CU count) times the tile's area over the tile's per-CU efficiency
// with the CU kept busy. The efficiencies are fits to n^3 problems from 2048 to 6144 in all
// four layouts (256: 0.95; 128: 0.93, 0.89 for a single round of 8-wave tiles; 64: 0.88),
// and the model picks the measured best at every size tried: 64 x 64 at 2560..5120 (5120^3:
// 1920 us against 2040 for 128 x 128 and 2302 for 256 x 256), 128 x 128 at 2048 and 6144
// (3145 us against 3269 and 4155), 256 x 256 at 4096 and 8192.
//  * 256 x 256, 8 waves, one workgroup per CU: NN with 2 x 4 waves of 128 x 64; NT, TN and TT
//    with 4 x 2 waves of 64 x 128 (an MN-contiguous A takes the shorter wave side; TN streams
//    its fragments a component at a time);
//  * 128 x 128: 8 waves (2 x 4, or 4 x 2 for a K-contiguous B) when one round holds every
//    tile, else 4 waves with two workgroups per CU;
//  * 64 x 64, 4 waves, up to five workgroups per CU.
struct F32Costs {
  double c256, c128, c64;
  double best() const { return fmin(c256, fmin(c128, c64)); }
};
inline F32Costs f32_ring_costs(long M, long N, long batch) {
  const long tiles256 = ((M + 255) / 256) * ((N + 255) / 256) * batch;
  const long tiles128 = ((M + 127) / 128) * ((N + 127) / 128) * batch;
  const long tiles64 = ((M + 63) / 64) * ((N + 63) / 64) * batch;
  auto cost = [](long tiles, double area, double eff) { return (double)((tiles + 255) / 256) * area / eff; };
  return {cost(tiles256, 256.0 * 256.0, 0.95), cost(tiles128, 128.0 * 128.0, tiles128 <= 256 ? 0.89 : 0.93),
          cost(tiles64, 64.0 * 64.0, 0.88)};
}

template <bool TA, bool TB>
hipError_t launch_f32_ring_best(const GemmParams &p, long batch, hipStream_t s) {
  const long tiles128 = ((p.M + 127) / 128) * ((p.N + 127) / 128) * batch;
  const F32Costs k = f32_ring_costs(p.M, p.N, batch);
  const double c256 = k.c256, c128 = k.c128, c64 = k.c64;
  if (c256 <= c128 && c256 <= c64) {
    if constexpr (!TA && !TB) return launch_f32_ring<256, 256, 2, 4, TA, TB>(p, batch, s);
    else return launch_f32_ring<256, 256, 4, 2, TA, TB>(p, batch, s);
  }
  if (c128 <= c64) {
    if (tiles128 > 256) return launch_f32_ring<128, 128, 2, 2, TA, TB>(p, batch, s);
    if constexpr (TB) return launch_f32_ring<128, 128, 4, 2, TA, TB>(p, batch, s);
    else return launch_f32_ring<128, 128, 2, 4, TA, TB>(p, batch, s);
  }
  return launch_f32_ring<64, 64, 2, 2, TA, TB>(p, batch, s);
}

// The small-product kernel's shape for an fp32 product, as 100 KW + 10 FM + FN, or 0 for the
// tiled kernels. It is taken while the 64 x 64 tiles would leave at least three quarters of
// the CUs idle (at most 64 tiles), for K up to 1024, for K up to 4096 at 4 tiles or fewer,
// and for any K below 2^24 multiply-adds in all (where the tiled path has no split-K).
// Workgroups of 16 x 16 tiles while there are at most 256 of them (or K is at most 32), or at
// most 512 with K over 272; 32 x 32 beyond (128 x 784 x 784: 8.4 us on 16 x 16 tiles against
// 10.2 on 32 x 32; 256 x 512 x 256: 7.3 against 6.6). As many K-splitting waves (4, 8, or 16
// with 16 x 16 tiles) as leave each wave at least three 16-element K steps and the grid at most
// 2048 waves. Kernel times on MI355X (rocprofv3 kernel trace), tiled -> small: 256^3 7.7 -> 4.2
// us; 128 x 784 x 784 21.5 -> 8.4 us; 100 x 130 x 1000 49.7 -> 10.6 us; 512^2 x 1024 16.3 ->
// 11.1 us; 16 x 16 x 4096 66.3 -> 13.6 us. At 768^2 (144 tiles), at 256^2 x 4096 and at 64^2 x
// 16384 the tiled path (split-K for the long K) is as fast or faster.
inline int f32_small_tile(long M, long N, long K, long batch, bool ta, bool tb) {
  if (const int c = skinny_tile(M, N, K, batch, false, ta, tb)) return c;
  const long tiles64 = ((M + 63) / 64) * ((N + 63) / 64) * batch;
  if (tiles64 > 64) return 0;
  const bool few_macs = (double)M * N * K * batch < (double)(1L << 24);
  if (!(K <= 1024 || (tiles64 <= 4 && K <= 4096) || few_macs)) return 0;
  const long t16 = ((M + 15) / 16) * ((N + 15) / 16) * batch, steps = (K + 15) / 16;
  const bool f11 = t16 <= 256 || steps <= 2 || (t16 <= 512 && steps >= 18);
  const long wgs = f11 ? t16 : (t16 + 3) / 4;
  int kw = 4;
  for (int c : {16, 8}) {
    if ((c == 16 && !f11) || 3 * c > steps || wgs * c > 2048) continue;
    kw = c;
    break;
  }
  return kw * 100 + (f11 ? 11 : 22);
}

template <bool TA, bool TB, bool VEC>
hipError_t pick_f32(const GemmParams &p, long batch, hipStream_t s) {
  if (const int code = f32_small_tile(p.M, p.N, p.K, batch, TA, TB)) return launch_small_code<float, TA, TB, VEC>(code, p, batch, s);
  if constexpr (!VEC) {
    return launch_f32<64, 64, 16, 2, 2, TA, TB, VEC>(p, batch, s);
  } else {
    // The DMA ring for the vector path, whose alignment (every contiguous extent a multiple
    // of 4 floats) keeps its 16-byte copies inside the operands. The ring takes whole K-tile
    // pairs (it carries no K-tail masking, which would cost it registers), so a K that is not
    // a multiple of 32 runs in two launches: the ring over the first K - K % 32 (alpha, beta,
    // no bias or activation), then the register-staged kernel over the last K % 32 with
    // beta = 1 on that partial result, bias and activation. The tail pointers stay 16-byte
    // aligned: K is a multiple of 4 for a K-contiguous operand, and leading dimensions are.
    // The result differs from one launch only in where the two partial sums are rounded
    // together. Against the register-staged kernel: 1000^3 35.3 -> 28.7 us, 3000^3 616 ->
    // 424 us, 4096 x 4096 x 4100 1026 -> 950 us (torch.matmul 24.0, 431, 907 us). Leading dimensions too large for the ring's 32-bit offsets, and K < 32, take
    // the register-staged kernel with the largest tile that still gives 256 tiles (256 x 256
    // with 16 waves of 64 x 64: 4096^3 132-135 TFLOP/s against 125 / 120 for 128 x 128).
    const long tiles256 = ((p.M + 255) / 256) * ((p.N + 255) / 256) * batch;
    const long tiles128 = ((p.M + 127) / 128) * ((p.N + 127) / 128) * batch;
    if (ring_offsets_fit(p) && p.K >= 32) {
      const long kt = p.K % 32;
      if (kt == 0) return launch_f32_ring_best<TA, TB>(p, batch, s);
      GemmParams head = p, tail = p;
      head.K = p.K - kt;
      head.bias = nullptr;
      head.act = -1;
      tail.K = kt;
      tail.beta = 1.0f;
      tail.A = static_cast<const float *>(p.A) + (TA ? head.K * p.lda : head.K);
      tail.B = static_cast<const float *>(p.B) + (TB ? head.K : head.K * p.ldb);
      if (hipError_t e = launch_f32_ring_best<TA, TB>(head, batch, s)) return e;
      return launch_f32<64, 64, 16, 2, 2, TA, TB, VEC>(tail, batch, s);
    }
    if (tiles256 >= 256) return launch_f32<256, 256, 16, 4, 4, TA, TB, VEC>(p, batch, s);
    if (tiles128 >= 256) return launch_f32<128, 128, 32, 2, 2, TA, TB, VEC>(p, batch, s);
    return launch_f32<64, 64, 16, 2, 2, TA, TB, VEC>(p, batch, s);
  }
}

template <bool VEC>
hipError_t dispatch(const GemmDesc &d, const GemmParams &p, long batch, hipStream_t s) {
  const int v = (d.ta ? 2 : 0) | (d.tb ? 1 : 0);
  if (d.dtype == GN_F16) {
    switch (v) {
      case 0: return pick_f16<false, false, VEC>(p, batch, s);
      case 1: return pick_f16<false, true, VEC>(p, batch, s);
      case 2: return pick_f16<true, false, VEC>(p, batch, s);
      default: return pick_f16<true, true, VEC>(p, batch, s);
    }
  }
  switch (v) {
    case 0: return pick_f32<false, false, VEC>(p, batch, s);
    case 1: return pick_f32<false, true, VEC>(p, batch, s);
    case 2: return pick_f32<true, false, VEC>(p, batch, s);
    default: return pick_f32<true, true, VEC>(p, batch, s);
  }
}

// Packs an operand for the aligned path: dst[z] (rows x Kp, row pitch Kp, 16-byte aligned)
// = op(src[z]) zero-padded from K to Kp, where op(src) is src (rows x K, pitch ld) or, for
// TRANS, the transpose of src (K x rows, pitch ld). 64 x 64 tiles, 256 threads; each thread
// stores whole 16-byte vectors (VL elements) of a destination row. Loads are element-wise,
// so src needs no alignment; the transposing form stages the tile in LDS so that its reads
// run along src's rows (staging the other form too measured slower: 7.1 -> 9.7 us for a
// 2047 x 2047 fp16 operand).
template <typename T, bool TRANS>
__device__ __forceinline__ void pack_tile(const T *__restrict__ src, long rows, long K, long ld, T *__restrict__ dst,
                                          long Kp, long tile_row, T (*tile)[65]) {
  constexpr int VL = 16 / sizeof(T);   // elements per 16-byte store
  constexpr int VPR = 64 / VL;         // vectors per tile row
  constexpr int RPP = 256 / VPR;       // tile rows per pass
  typedef T vec_t __attribute__((ext_vector_type(VL)));
  const long r0 = tile_row * 64, k0 = (long)blockIdx.x * 64;
  if constexpr (TRANS) {
    // all 16 loads of a thread are issued before the first LDS store
    const int tx = threadIdx.x & 63, ty = threadIdx.x >> 6;
    const long r = r0 + tx;
    T x[16];
#pragma unroll
    for (int u = 0; u < 16; ++u) {
      const long k = k0 + ty + 4 * u;
      x[u] = (k < K && r < rows) ? src[k * ld + r] : T(0);
    }
#pragma unroll
    for (int u = 0; u < 16; ++u) tile[ty + 4 * u][tx] = x[u];
    __syncthreads();
  }
  const int vr = threadIdx.x / VPR, vc = (threadIdx.x % VPR) * VL;
  const long k = k0 + vc;
  if (k >= Kp) return;  // Kp is a multiple of 64 here, so a vector never straddles it
  constexpr int NP = 64 / RPP;  // passes over the tile's rows
  vec_t v[NP];
#pragma unroll
  for (int u = 0; u < NP; ++u) {
    const int i = vr + u * RPP;
    const long r = r0 + i;
#pragma unroll
    for (int j = 0; j < VL; ++j) {
      if constexpr (TRANS) v[u][j] = tile[vc + j][i];
      else v[u][j] = (r < rows && k + j < K) ? src[r * ld + k + j] : T(0);
    }
  }
#pragma unroll
  for (int u = 0; u < NP; ++u) {
    const long r = r0 + vr + u * RPP;
    if (r < rows) *reinterpret_cast<vec_t *>(dst + r * Kp + k) = v[u];
  }
}

// One operand: grid (Kp / 64, tile rows, batch).
template <typename T, bool TRANS>
__global__ void __launch_bounds__(256) pack_kcontig_kernel(const T *__restrict__ src, long rows, long K, long ld,
                                                           long sstride, T *__restrict__ dst, long Kp, long dstride) {
  __shared__ T tile[64][65];
  pack_tile<T, TRANS>(src + (long)blockIdx.z * sstride, rows, K, ld, dst + (long)blockIdx.z * dstride, Kp, blockIdx.y,
                      tile);
}

template <typename T>
struct PackOp {
  const T *src;
  T *dst;
  long rows, ld, sstride;
};

// Both operands in one launch: grid rows below ya pack A's tile rows, the rest B's (the branch
// is uniform within a workgroup), so the two copies run side by side.
template <typename T, bool TA, bool TB>
__global__ void __launch_bounds__(256) pack2_kcontig_kernel(PackOp<T> a, PackOp<T> b, long K, long Kp, long ya) {
  __shared__ T tile[64][65];
  const long z = blockIdx.z;
  if ((long)blockIdx.y < ya)
    pack_tile<T, TA>(a.src + z * a.sstride, a.rows, K, a.ld, a.dst + z * a.rows * Kp, Kp, blockIdx.y, tile);
  else
    pack_tile<T, TB>(b.src + z * b.sstride, b.rows, K, b.ld, b.dst + z * b.rows * Kp, Kp, blockIdx.y - ya, tile);
}

template <typename T>
hipError_t launch_pack(const void *src, long rows, long K, long ld, long sstride, bool trans, void *dst, long Kp,
                       long batch, hipStream_t s) {
  const dim3 g((unsigned)((Kp + 63) / 64), (unsigned)((rows + 63) / 64), (unsigned)batch);
  const T *sp = static_cast<const T *>(src);
  T *dp = static_cast<T *>(dst);
  if (trans) hipLaunchKernelGGL((pack_kcontig_kernel<T, true>), g, dim3(256), 0, s, sp, rows, K, ld, sstride, dp, Kp, rows * Kp);
  else hipLaunchKernelGGL((pack_kcontig_kernel<T, false>), g, dim3(256), 0, s, sp, rows, K, ld, sstride, dp, Kp, rows * Kp);
  return hipGetLastError();
}

// A (M x K after op) and B (N x K after op) packed by one launch; ta / tb: the stored operand
// is the transpose of the K-contiguous layout.
template <typename T>
hipError_t launch_pack2(PackOp<T> a, bool ta, PackOp<T> b, bool tb, long K, long Kp, long batch, hipStream_t s) {
  const long ya = (a.rows + 63) / 64, yb = (b.rows + 63) / 64;
  const dim3 g((unsigned)((Kp + 63) / 64), (unsigned)(ya + yb), (unsigned)batch), blk(256);
  if (ta && tb) hipLaunchKernelGGL((pack2_kcontig_kernel<T, true, true>), g, blk, 0, s, a, b, K, Kp, ya);
  else if (ta) hipLaunchKernelGGL((pack2_kcontig_kernel<T, true, false>), g, blk, 0, s, a, b, K, Kp, ya);
  else if (tb) hipLaunchKernelGGL((pack2_kcontig_kernel<T, false, true>), g, blk, 0, s, a, b, K, Kp, ya);
  else hipLaunchKernelGGL((pack2_kcontig_kernel<T, false, false>), g, blk, 0, s, a, b, K, Kp, ya);
  return hipGetLastError();
}

// Zero-K / empty-product epilogue: C = act(beta*C + bias) (alpha*0 contributes nothing).
__global__ void gemm_k0_kernel(GemmParams p, long batch) {
  const long total = p.M * p.N * batch;
  for (long t = blockIdx.x * (long)blockDim.x + threadIdx.x; t < total; t += (long)gridDim.x * blockDim.x) {
    const long z = t / (p.M * p.N);
    const long r = (t / p.N) % p.M;
    const long c = t % p.N;
    float *dst = p.C + z * p.strideC + r * p.ldc + c;
    float v = p.beta != 0.0f ? p.beta * *dst : 0.0f;
    v += p.bias ? p.bias[c] : 0.0f;
    *dst = apply_act(p.act, v, p.act_alpha);
  }
}

// ------------------------------------------------------------------ split-K
// A product with few output tiles and a long K leaves most CUs idle (512 x 4096 x 11008
// fp16: 128 tiles of 128 x 128 for 256 CUs). It runs instead as S slices of K: one launch of
// the aligned kernels computes every slice's partial product P_s = op(A)[:, slice s] op(B)[slice
// s, :] into its own fp32 M x N buffer (slice s is batch index s, through the batch strides),
// then splitk_reduce_kernel writes C = act(alpha (P_0 + P_1 + ... + P_{S-1}) + beta C + bias),
// summing the partials in slice order, so the result does not depend on timing. It differs
// from the one-launch product only in where the K sum is rounded.
// Each thread sums one 16-byte group of four consecutive elements of the M x N partials
// (flat index i .. i+3; the partials' stride PS is a multiple of 4, so every group is aligned,
// and a group past M*N reads only the stride's padding). VST: N, ldc and C allow 16-byte rows,
// so a group lies in one row of C and is stored as a vector; otherwise element by element.
template <bool VST, int ACT>
__global__ void __launch_bounds__(256)
    splitk_reduce_kernel(const float *__restrict__ P, int S, long PS, long M, long N, float *C, long ldc,
                         float alpha, float beta, const float *__restrict__ bias, int act_rt, float act_alpha) {
  const long MN = M * N;
  const int act = ACT == kActRuntime ? act_rt : ACT;
  const long step = (long)gridDim.x * blockDim.x;
  for (long v = blockIdx.x * (long)blockDim.x + threadIdx.x; 4 * v < MN; v += step) {
    const long i = 4 * v;
    // the loads of up to eight partials are issued before their adds, which then run in
    // slice order
    float4_t acc = *reinterpret_cast<const float4_t *>(P + i);
    int k = 1;
    for (; k + 8 <= S; k += 8) {
      float4_t x[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) x[j] = *reinterpret_cast<const float4_t *>(P + (k + j) * PS + i);
#pragma unroll
      for (int j = 0; j < 8; ++j) acc += x[j];
    }
    for (; k + 4 <= S; k += 4) {
      float4_t x[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) x[j] = *reinterpret_cast<const float4_t *>(P + (k + j) * PS + i);
#pragma unroll
      for (int j = 0; j < 4; ++j) acc += x[j];
    }
    for (; k < S; ++k) acc += *reinterpret_cast<const float4_t *>(P + k * PS + i);
    if constexpr (VST) {
      const long r = i / N, c = i - r * N;
      float *dst = C + r * ldc + c;
      const float4_t old = beta != 0.0f ? *reinterpret_cast<const float4_t *>(dst) : float4_t{0.f, 0.f, 0.f, 0.f};
      float4_t o;
#pragma unroll
      for (int e = 0; e < 4; ++e)
        o[e] = apply_act(act, alpha * acc[e] + beta * old[e] + (bias ? bias[c + e] : 0.0f), act_alpha);
      *reinterpret_cast<float4_t *>(dst) = o;
    } else {
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        if (i + e >= MN) break;
        const long r = (i + e) / N, c = (i + e) - r * N;
        float *dst = C + r * ldc + c;
        float x = alpha * acc[e];
        if (beta != 0.0f) x += beta * *dst;
        *dst = apply_act(act, x + (bias ? bias[c] : 0.0f), act_alpha);
      }
    }
  }
}

// The partials' stride: M x N rounded up to a multiple of 4 floats.
inline long splitk_stride(long M, long N) { return (M * N + 3) / 4 * 4; }

hipError_t launch_splitk_reduce(const float *P, int S, const GemmParams &p, hipStream_t s) {
  const bool vst = p.N % 4 == 0 && p.ldc % 4 == 0 && ((uintptr_t)p.C & 15) == 0;
  const long groups = (p.M * p.N + 3) / 4;
  const dim3 grid((unsigned)std::min<long>((groups + 255) / 256, 4096)), block(256);
  const long PS = splitk_stride(p.M, p.N);
  auto go = [&](auto v, auto a) {
    hipLaunchKernelGGL((splitk_reduce_kernel<decltype(v)::value, decltype(a)::value>), grid, block, 0, s, P, S, PS,
                       p.M, p.N, p.C, p.ldc, p.alpha, p.beta, p.bias, p.act, p.act_alpha);
  };
  auto pick = [&](auto v) {
    switch (p.act) {
      case -1: go(v, ActCode<-1>{}); break;
      case 0: go(v, ActCode<0>{}); break;
      case 7: go(v, ActCode<7>{}); break;
      default: go(v, ActCode<kActRuntime>{}); break;
    }
  };
  if (vst) pick(std::true_type{});
  else pick(std::false_type{});
  return hipGetLastError();
}

// The slice count S for a batch-1 product on the aligned path (1: no split). Candidates
// divide K into slices of a whole number of 64-element steps, at least 512 long; each is
// priced in microseconds as its partial launch plus the reduce, and the cheapest is taken
// when it beats one launch by the margin. The partial launch's price is the tile model of
// the aligned kernels (rounds of tiles times their per-round time) at batch S and the slice
// length. fp16: cost x (Ks / 1024 x 24.9 + 13.8) us, with the cost of the 256 x 256 and
// 128 x 128 tiles; the constants are a fit to the partial launches of nine shapes from
// 64 x 4096 x 4096 to 2048 x 2048 x 8192 at S = 1..16. The 128 x 192 and 128 x 96 tiles
// (K-contiguous B only) are left out so that all four transpose layouts choose the same S
// and stay bit-identical. fp32: 219.6 us per 1024 of K per round of 256 x 256 tiles, scaled
// by the fp32 ring's cost (1.1x for one 64 x 64 workgroup per CU). The reduce: 2.5 us plus
// its HBM bytes at 5 TB/s. fp16 splits only products of fewer than 512 tiles of 128 x 128
// (one round of the two-per-CU tiles), the range its model was checked on: there the split
// won or tied on every shape measured (2048 x 2048 x 16384: 167 -> 129 us; 2048 x 2048 x 8192:
// 90 -> 81 us); fp32 takes the model's word.
int choose_split(int dtype, long M, long N, long K, bool beta) {
  if (K < 1024 || K % 64) return 1;
  const bool f16 = dtype == GN_F16;
  const long tiles128 = ((M + 127) / 128) * ((N + 127) / 128);
  if (f16 && tiles128 >= 512) return 1;
  auto gemm_us = [&](long S) {
    const double ks = (double)(K / S) / 1024.0;
    if (f16) return f16_best<false>(M, N, S).cost * (ks * 24.9 + 13.8);
    // one 64 x 64 workgroup per CU (4 waves, one per SIMD) runs about 10% below two or more
    // co-resident ones (128 x 8192 x 8192: 142.6 us in one launch, 127.9 us for the partial
    // launch at S = 2)
    const long tiles64 = ((M + 63) / 64) * ((N + 63) / 64) * S;
    return 219.6 * f32_ring_costs(M, N, S).best() / 65536.0 * ks * (tiles64 <= 256 ? 1.1 : 1.0);
  };
  auto reduce_us = [&](long S) { return 2.5 + (double)(S + 1 + (beta ? 1 : 0)) * (double)(M * N) * 4.0 / 5.0e6; };
  const double whole = gemm_us(1);
  double best = whole * (f16 ? 0.9 : 0.95);
  int pick = 1;
  for (long S = 2; S <= 32; ++S) {
    if (K % (64 * S) || K / S < 512) continue;
    const double t = gemm_us(S) + reduce_us(S);
    if (t < best) best = t, pick = (int)S;
  }
  return pick;
}

}  // namespace

bool act_supported(int act) { return act == -1 || act == 0 || act == 1 || act == 2 || (act >= 4 && act <= 7); }

int launch_gemm(const GemmDesc &d, hipStream_t s, CError *err) {
  if (d.dtype != GN_F32 && d.dtype != GN_F16) return set_error(err, -1, "gemm: unsupported dtype %d", d.dtype);
  if (d.M < 0 || d.N < 0 || d.K < 0 || d.batch < 1) return set_error(err, -1, "gemm: negative size");
  if (!act_supported(d.act)) return set_error(err, -1, "gemm: unsupported activation %d", d.act);
  if (d.M == 0 || d.N == 0) return 0;
  if (!d.C) return set_error(err, -1, "gemm: NULL C");
  if (d.K > 0 && (!d.A || !d.B)) return set_error(err, -1, "gemm: NULL operand");
  const long a_cols = d.ta ? d.M : d.K, b_cols = d.tb ? d.K : d.N;  // stored row lengths
  if ((d.K > 0 && (d.lda < a_cols || d.ldb < b_cols)) || d.ldc < d.N)
    return set_error(err, -1, "gemm: leading dimension smaller than row length");
  const long tiles = ((d.M + 63) / 64) * ((d.N + 63) / 64);
  if (tiles > (1L << 30)) return set_error(err, -1, "gemm: problem too large for the grid");

  GemmParams p{};
  p.A = d.A; p.B = d.B; p.C = d.C; p.bias = d.bias;
  p.M = d.M; p.N = d.N; p.K = d.K;
  p.lda = d.lda; p.ldb = d.ldb; p.ldc = d.ldc;
  p.strideA = d.strideA; p.strideB = d.strideB; p.strideC = d.strideC;
  p.alpha = d.alpha; p.beta = d.beta; p.act = d.act; p.act_alpha = d.act_alpha;

  hipError_t e;
  if (d.K == 0) {
    hipLaunchKernelGGL(gemm_k0_kernel, dim3(1024), dim3(256), 0, s, p, d.batch);
    e = hipGetLastError();
  } else {
    const size_t esz = d.dtype == GN_F16 ? 2 : 4;
    const long epv = 16 / (long)esz;
    auto aligned = [&](const void *ptr, long ld, long stride) {
      return ((uintptr_t)ptr % 16 == 0) && (ld % epv == 0) && (d.batch == 1 || stride % epv == 0);
    };
    // Vector path needs every contiguous extent (K for K-contiguous, M/N otherwise)
    // to be a multiple of the vector length.
    const long a_contig = d.ta ? d.M : d.K, b_contig = d.tb ? d.K : d.N;
    const bool vec = aligned(d.A, d.lda, d.strideA) && aligned(d.B, d.ldb, d.strideB) && a_contig % epv == 0 &&
                     b_contig % epv == 0;
    // The batch index is blockIdx.z (at most 65535 per launch): larger batches run as
    // consecutive launches over chunks of the batch, each with offset operands.
    constexpr long kMaxZ = 65535;
    // Unaligned operands of a large enough product are first packed into zero-padded,
    // K-contiguous copies (row pitch K rounded up to 64) in the stream's scratch, and the
    // aligned path runs on them. Only the operands that fail the alignment test are packed;
    // the product keeps its K, and a 16-byte block of a packed row that straddles K reads the
    // padding's zeros, while the aligned kernels mask an unpacked operand's rows at or past K
    // (per copy in the fp16 ring, by the K-tail split of the fp32 path). The result is the
    // aligned path's on the same values. Products the small-product kernel takes are not
    // packed (its loads need no alignment); the element-wise-load kernel stays for the other
    // products below 2^24 multiply-adds, for scratch beyond 4 GiB, and under HIP graph capture
    // (the scratch may need an allocation).
    const long Kp = (d.K + 63) / 64 * 64;
    const bool a_ok = aligned(d.A, d.lda, d.strideA) && a_contig % epv == 0;
    const bool b_ok = aligned(d.B, d.ldb, d.strideB) && b_contig % epv == 0;
    // NN products of 1-4 rows on the GEMV kernel, which needs only W aligned (X is read element
    // by element)
    const bool gemv = b_ok && !d.ta && !d.tb && gemv_nn(d.M, d.N, d.K, d.batch, d.dtype == GN_F16);
    const size_t pack_bytes =
        (size_t)((a_ok ? 0 : d.M) + (b_ok ? 0 : d.N)) * (size_t)Kp * esz * (size_t)std::min(kMaxZ, d.batch);
    const bool big = (double)d.M * d.N * d.K >= (double)(1L << 24);
    const long pack_grid_y = (a_ok ? 0 : (d.M + 63) / 64) + (b_ok ? 0 : (d.N + 63) / 64);
    const bool small = gemv || (d.dtype == GN_F32 ? f32_small_tile(d.M, d.N, d.K, d.batch, d.ta, d.tb)
                                          : f16_small_tile(d.M, d.N, d.K, d.batch, d.ta, d.tb)) != 0;
    bool pack = !vec && big && !small && pack_bytes <= ((size_t)4 << 30) && pack_grid_y <= 65535;
    // Split-K (choose_split) for a batch-1 product on the aligned path, packed or not, whose
    // operands suit the DMA ring; the partial products take S x M x N floats of the scratch
    // (each M x N rounded up to a multiple of 4), ahead of the packed copies.
    const long k_aligned = (!a_ok && !b_ok) ? Kp : d.K;  // the K the aligned kernels see
    int S = 1;
    if (d.batch == 1 && big && !small && (vec || pack) && (a_ok ? d.lda : Kp) < (1L << 21) && (b_ok ? d.ldb : Kp) < (1L << 21))
      S = choose_split(d.dtype, d.M, d.N, k_aligned, d.beta != 0.0f);
    const size_t part_bytes = S > 1 ? ((size_t)S * splitk_stride(d.M, d.N) * sizeof(float) + 255) / 256 * 256 : 0;
    if (part_bytes > ((size_t)1 << 30)) S = 1;
    if (pack || S > 1) {  // the scratch may need an allocation, which graph capture must not see
      hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
      if (hipStreamIsCapturing(s, &cap) != hipSuccess || cap != hipStreamCaptureStatusNone) pack = false, S = 1;
    }
    const size_t ws_bytes = (pack ? pack_bytes : 0) + (S > 1 ? part_bytes : 0);
    std::unique_lock<std::mutex> lk;
    char *ws = nullptr;
    if (ws_bytes) {
      ws = static_cast<char *>(stream_scratch(s, ws_bytes, lk, err));
      if (!ws) return -3;
    }
    e = hipSuccess;
    for (long z0 = 0; z0 < d.batch && e == hipSuccess; z0 += kMaxZ) {
      GemmParams q = p;
      q.A = static_cast<const char *>(d.A) + z0 * d.strideA * (long)esz;
      q.B = static_cast<const char *>(d.B) + z0 * d.strideB * (long)esz;
      q.C = d.C + z0 * d.strideC;
      const long nb = std::min(kMaxZ, d.batch - z0);
      if (gemv) {
        e = d.dtype == GN_F16 ? launch_gemv<_Float16>(q, s) : launch_gemv<float>(q, s);
        continue;
      }
      if (!pack && S == 1) {
        e = vec ? dispatch<true>(d, q, nb, s) : dispatch<false>(d, q, nb, s);
        continue;
      }
      GemmDesc dp = d;
      char *next = ws + (S > 1 ? part_bytes : 0);
      char *a_dst = next, *b_dst = next + (a_ok ? 0 : (size_t)nb * d.M * Kp * esz);
      if (!a_ok && !b_ok) {  // one launch for both
        e = esz == 2 ? launch_pack2<_Float16>({static_cast<const _Float16 *>(q.A), reinterpret_cast<_Float16 *>(a_dst),
                                               d.M, d.lda, d.strideA}, d.ta,
                                              {static_cast<const _Float16 *>(q.B), reinterpret_cast<_Float16 *>(b_dst),
                                               d.N, d.ldb, d.strideB}, !d.tb, d.K, Kp, nb, s)
                     : launch_pack2<float>({static_cast<const float *>(q.A), reinterpret_cast<float *>(a_dst), d.M, d.lda,
                                            d.strideA}, d.ta,
                                           {static_cast<const float *>(q.B), reinterpret_cast<float *>(b_dst), d.N, d.ldb,
                                            d.strideB}, !d.tb, d.K, Kp, nb, s);
      } else if (!a_ok) {
        e = esz == 2 ? launch_pack<_Float16>(q.A, d.M, d.K, d.lda, d.strideA, d.ta, a_dst, Kp, nb, s)
                     : launch_pack<float>(q.A, d.M, d.K, d.lda, d.strideA, d.ta, a_dst, Kp, nb, s);
      } else if (!b_ok) {
        e = esz == 2 ? launch_pack<_Float16>(q.B, d.N, d.K, d.ldb, d.strideB, !d.tb, b_dst, Kp, nb, s)
                     : launch_pack<float>(q.B, d.N, d.K, d.ldb, d.strideB, !d.tb, b_dst, Kp, nb, s);
      }
      if (!a_ok) {
        q.A = a_dst;
        q.lda = Kp;
        q.strideA = d.M * Kp;
        dp.ta = false;
      }
      if (!b_ok) {
        q.B = b_dst;
        q.ldb = Kp;
        q.strideB = d.N * Kp;
        dp.tb = true;
      }
      if (!a_ok && !b_ok) q.K = Kp;  // both padded with zeros: whole K-tile pairs, no K tail
      if (e != hipSuccess) break;
      if (S == 1) {
        e = dispatch<true>(dp, q, nb, s);
        continue;
      }
      // slice s of K is batch index s: A and B advance by the slice along K, the partial
      // products are S consecutive M x N buffers; alpha, beta, bias and the activation wait
      // for the reduce
      GemmParams r = q;
      const long ks = q.K / S;
      r.K = ks;
      r.alpha = 1.0f;
      r.beta = 0.0f;
      r.bias = nullptr;
      r.act = -1;
      r.C = reinterpret_cast<float *>(ws);
      r.ldc = d.N;
      r.strideC = splitk_stride(d.M, d.N);
      r.strideA = dp.ta ? ks * q.lda : ks;
      r.strideB = dp.tb ? ks : ks * q.ldb;
      e = dispatch<true>(dp, r, S, s);
      if (e == hipSuccess) e = launch_splitk_reduce(r.C, S, q, s);
    }
    stream_scratch_trim(s, lk);
  }
  if (e != hipSuccess) return hip_error(err, -6, "gemm launch", e);
  return 0;
}

}  // namespace gn
