// ring_model.cpp — CPU model of every DMA copy the ring GEMM kernels issue
// (go-nngpu_amd/csrc/gemm.hip: ring_mainloop / ring_mainloop_f32), through the same plan
// functions the kernels call (go-nngpu_amd/csrc/ring_plan.h).
//
// For each ring configuration the dispatch launches (tile, waves, ring slots, dtype), each
// operand layout (K-contiguous or MN-contiguous), and a set of shapes within the kernels'
// preconditions (16-byte vectors: leading dimensions and every contiguous extent multiples of
// 8 halves or 4 floats; fp32 K a multiple of 32; leading dimensions below 2^21), it walks
// every tile along the operand's M (or N), every wave, chunk and lane, and every K-tile pair
// from 0 to np + NS (the ring's refills run NS - 1 pairs ahead, past the end of K). For each
// pair it checks that the live copies (offset below the record count, pair live) read only
// elements of the operand (row < rows, the copy's 16 bytes within the row's valid extent)
// and together cover exactly the tile's part of the pair's K-tiles, each element once; dead
// copies read zeros and touch nothing.
//
// --plant f32-dead-pairs-live treats the fp32 pairs past K as live, the plan before dead
// pairs went through zero-record descriptors (its refills read past the end of K); --plant
// f16-no-kmask drops the fp16 ring's per-copy K mask. Either must report violations.
// --list prints the configurations modelled. Exit 0: no violation; 1: violations.
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <map>
#include <string>
#include <vector>

#include "../../go-nngpu_amd/csrc/ring_plan.h"

namespace {

using namespace gn::ring;

struct Config {
  bool f16;
  int BM, BN, WM, WN, NS;
  bool tb_only;  // the dispatch launches it only for a K-contiguous B (TB)
};

// gemm.hip: launch_f16_tile (256x256 2x4; 128x128 2x4 and 2x2; 128x192 2x4 with three
// slots and 128x96 2x2, TB only) and launch_f32_ring_best (256x256 2x4 for NN, 4x2 for the
// other layouts; 128x128 2x2, 2x4 or 4x2; 64x64 2x2). gemm_f16_ring_mf32_kernel (the 32x32x16 NN
// variant) issues the same copies as the fp16 256x256 2x4 two-slot ring. The test runner checks
// this table against the launches in gemm.hip.
const Config kConfigs[] = {
    {true, 256, 256, 2, 4, 2, false}, {true, 128, 128, 2, 4, 2, false}, {true, 128, 128, 2, 2, 2, false},
    {true, 128, 192, 2, 4, 3, true},  {true, 128, 96, 2, 2, 2, true},   {false, 256, 256, 2, 4, 2, false},
    {false, 256, 256, 4, 2, 2, false}, {false, 128, 128, 2, 2, 2, false}, {false, 128, 128, 2, 4, 2, false},
    {false, 128, 128, 4, 2, 2, false}, {false, 64, 64, 2, 2, 2, false},
};

bool g_plant_f32_dead_live = false, g_plant_f16_no_kmask = false;
long g_checked = 0, g_violations = 0;
std::map<std::string, long> g_kinds;  // violations by kind

void violation(const char *what, const Config &cf, char op, bool kcontig, long MN, long K, long ld, long t0, long pp,
               int wave, int chunk, int lane) {
  if (g_violations < 20)
    std::printf("VIOLATION %s: %s %dx%d w%dx%d ns%d op %c %s MN=%ld K=%ld ld=%ld tile@%ld pair %ld wave %d chunk %d "
                "lane %d\n",
                what, cf.f16 ? "f16" : "f32", cf.BM, cf.BN, cf.WM, cf.WN, cf.NS, op,
                kcontig ? "K-contiguous" : "MN-contiguous", MN, K, ld, t0, pp, wave, chunk, lane);
  ++g_violations;
  ++g_kinds[what];
}

// One operand: A (op 'A', tile extent BM, layout K-contiguous unless TA) or B (op 'B', BN,
// K-contiguous when TB). MN = M or N, the extent the tiles run along.
void check_operand(const Config &cf, char op, bool kcontig, long MN, long K, long ld) {
  const int esz = cf.f16 ? 2 : 4, epv = 16 / esz, BK = cf.f16 ? 32 : 16;
  const int BT = op == 'A' ? cf.BM : cf.BN;  // the tile's extent along MN
  const int NW = cf.WM * cf.WN;
  const int OP = BT * BK * esz;         // bytes of one K-tile of the operand
  const int C = 2 * OP / 1024;          // 1 KiB chunks per pair
  const int IP = C / NW;                // chunks per wave
  const int RB = BT * esz;              // bytes of one k row of an MN-contiguous tile
  // storage: K-contiguous = MN rows of K (pitch ld); MN-contiguous = K rows of MN
  const long rows = kcontig ? MN : K, cols = kcontig ? K : MN;
  const long nk = (K + BK - 1) / BK, np = nk + 1 >= 2 ? (nk + 1) / 2 : 1;
  const long step = pair_step_bytes(kcontig, BK, ld, esz);
  const long ntiles = (MN + BT - 1) / BT;
  std::vector<unsigned char> seen((size_t)BT * 2 * BK);
  for (long t = 0; t < ntiles; ++t) {
    const long t0 = t * BT;
    const long base = base_elems(kcontig, t0, ld) * esz;  // bytes from the operand's start
    const long lim = MN - t0;
    for (long pp = 0; pp < np + cf.NS + 1; ++pp) {
      std::fill(seen.begin(), seen.end(), 0);
      const int krem = f16_krem(K, pp);
      const bool pair_live = f32_pair_live(pp, np) || g_plant_f32_dead_live;
      for (int w = 0; w < NW; ++w)
        for (int i = 0; i < IP; ++i) {
          const int c = w * IP + i;
          for (int lane = 0; lane < 64; ++lane) {
            unsigned off;
            if (cf.f16) {
              const Copy cp = plan_f16(kcontig, c, C, RB, ld, lim, lane);
              off = g_plant_f16_no_kmask ? cp.vo : f16_offset(cp, krem);
            } else {
              off = plan_f32(kcontig, c, C, RB, ld, lim, lane);
              if (!pair_live) continue;  // a zero-record descriptor: reads zeros
            }
            if (off >= kNumRecords) continue;  // reads zeros, touches no memory
            ++g_checked;
            const long byte = base + pp * step + (long)off;
            if (byte < 0 || byte % 16) {
              violation("misaligned or negative copy", cf, op, kcontig, MN, K, ld, t0, pp, w, c, lane);
              continue;
            }
            const long e = byte / esz, r = e / ld, col = e % ld;
            if (r >= rows || col + epv > cols) {
              violation(r >= rows || (r == rows - 1 && col + epv > cols) ? "copy outside the operand"
                                                                          : "copy outside the valid elements",
                        cf, op, kcontig, MN, K, ld, t0, pp, w, c, lane);
              continue;
            }
            // tile-relative position: (MN index within the tile, k within the pair)
            const long mn = kcontig ? r - t0 : col - t0, k = kcontig ? col - pp * 2 * BK : r - pp * 2 * BK;
            const long mn_len = kcontig ? 1 : epv, k_len = kcontig ? epv : 1;
            if (mn < 0 || mn + mn_len > BT || k < 0 || k + k_len > 2 * BK) {
              violation("copy outside the tile's pair", cf, op, kcontig, MN, K, ld, t0, pp, w, c, lane);
              continue;
            }
            for (long a = 0; a < mn_len; ++a)
              for (long b = 0; b < k_len; ++b) {
                unsigned char &s = seen[(size_t)(mn + a) * 2 * BK + (size_t)(k + b)];
                if (s) violation("element copied twice", cf, op, kcontig, MN, K, ld, t0, pp, w, c, lane);
                s = 1;
              }
          }
        }
      // every valid element of the tile's part of the pair, and only those, was copied
      const long mn_valid = lim < BT ? lim : BT;
      const long k_lo = pp * 2 * BK, k_valid = K - k_lo < 0 ? 0 : (K - k_lo > 2 * BK ? 2 * BK : K - k_lo);
      for (long a = 0; a < BT; ++a)
        for (long b = 0; b < 2 * BK; ++b) {
          const bool want = a < mn_valid && b < k_valid;
          if ((bool)seen[(size_t)a * 2 * BK + (size_t)b] != want) {
            violation(want ? "element never copied" : "element outside the matrix copied", cf, op, kcontig, MN, K, ld,
                      t0, pp, -1, -1, -1);
            a = BT;  // one report per pair
            break;
          }
        }
    }
  }
}

}  // namespace

int main(int argc, char **argv) {
  for (int i = 1; i < argc; ++i) {
    if (!std::strcmp(argv[i], "--list")) {
      for (const Config &cf : kConfigs)
        std::printf("%s %d %d %d %d %d%s\n", cf.f16 ? "f16" : "f32", cf.BM, cf.BN, cf.WM, cf.WN, cf.NS,
                    cf.tb_only ? " tb" : "");
      return 0;
    }
    if (!std::strcmp(argv[i], "--plant") && i + 1 < argc) {
      const std::string p = argv[++i];
      if (p == "f32-dead-pairs-live") g_plant_f32_dead_live = true;
      else if (p == "f16-no-kmask") g_plant_f16_no_kmask = true;
      else {
        std::fprintf(stderr, "unknown plant %s\n", p.c_str());
        return 2;
      }
    }
  }
  for (const Config &cf : kConfigs) {
    const int epv = cf.f16 ? 8 : 4;
    for (char op : {'A', 'B'}) {
      const int BT = op == 'A' ? cf.BM : cf.BN;
      for (bool kcontig : {true, false}) {
        if (cf.tb_only && op == 'B' && !kcontig) continue;
        // MN extents: ragged around the tile (MN-contiguous extents stay vector multiples)
        std::vector<long> mns = {(long)epv, 8L * epv, (long)BT - epv, (long)BT, (long)BT + epv, 2L * BT + 5 * epv};
        if (kcontig) mns.insert(mns.end(), {1L, 37L, (long)BT - 1, (long)BT + 3});
        // K: one to three pairs and tails (fp16); whole pairs for fp32 (its tail runs elsewhere)
        // (an MN-contiguous fp16 operand takes any K: a layout with both operands MN-contiguous
        // has no K alignment)
        std::vector<long> ks;
        if (cf.f16) ks = {8, 56, 64, 72, 128, 136, 200};
        else ks = {32, 64, 96, 128};
        if (cf.f16 && !kcontig) ks.insert(ks.end(), {1L, 37L, 99L, 129L});
        for (long MN : mns)
          for (long K : ks) {
            const long contig = kcontig ? K : MN;  // the extent along a stored row
            const long lds_[] = {contig, contig + epv, (1L << 21) - epv};
            for (long ld : lds_) {
              if (ld < contig || ld % epv) continue;
              check_operand(cf, op, kcontig, MN, K, ld);
            }
          }
      }
    }
  }
  for (const auto &k : g_kinds) std::printf("violations of kind \"%s\": %ld\n", k.first.c_str(), k.second);
  std::printf("ring model: %ld live copies checked, %ld violations\n", g_checked, g_violations);
  return g_violations ? 1 : 0;
}
