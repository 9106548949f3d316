// ring_plan.h — the copy plan of the DMA-ring GEMM kernels (gemm.hip): which 16 bytes of an
// operand each lane copies into LDS for a K-tile pair, and which copies are dead.
//
// Plain constexpr functions (HIP-Clang compiles them for the device as well), so the
// kernels and the CPU model of every copy (tests/ring_model/ring_model.cpp, run by
// tests/test_ring_model.py) use the same arithmetic.
//
// A ring kernel keeps one raw buffer descriptor per operand. It starts at the tile's first
// row (K-contiguous operand) or column (MN-contiguous operand) and advances by one K-tile
// pair per pair issued; lane `lane` of chunk c copies 16 bytes at descriptor base + offset.
// An offset at or beyond the descriptor's record count reads zeros and touches no memory:
// the plan gives rows or columns past the matrix kOutOfRange, the fp16 ring masks copies of k
// at or past K the same way (per copy, every pair), and the fp32 ring, whose K is a multiple
// of a pair, issues the pairs past K through descriptors with a record count of 0.
#pragma once

namespace gn {
namespace ring {

constexpr unsigned kNumRecords = 0x7ffffff0u;  // record count of a live descriptor
constexpr unsigned kOutOfRange = 0x80000000u;  // an offset beyond it: the copy reads zeros

// K-contiguous tiles: a 1 KiB chunk holds rows 8c..8c+7 of the pair's two K-tiles (128
// bytes each). Lane L copies octet kc8_octet(r, L & 7) of row r = 8c + (L >> 3), which the
// hardware writes to slot L: octet o of row r sits in slot kc8_slot(r, o).
constexpr int kc8_slot(int r, int o) { return 8 * (r & 7) + (o ^ ((r >> 1) & 7)); }
constexpr int kc8_octet(int r, int j) { return j ^ ((r >> 1) & 7); }
// 32-byte block XOR of k row k of an fp16 MN-contiguous tile: 2 (k & 3) + ((k >> 3) & 1). The
// rows a half-wave's ds_read_b64_tr_b16 touches get 8 distinct blocks of one 256-byte bank
// row: k0 + 0..3 and k0 + 8..11 at one column block (16 x 16 x 32 fragments), and k0 + 0..3 at
// two adjacent column blocks (32 x 32 x 16 fragments).
constexpr int hsw(int k) { return ((k & 3) << 1) | ((k >> 3) & 1); }
// 16-byte block XOR of k row k of an fp32 MN-contiguous tile.
constexpr int msw32(int k) { return ((k >> 2) & 1) << 2; }

// One lane's copy: byte offset from the pair's descriptor base, and (fp16) the first k of
// the pair it covers.
struct Copy {
  unsigned vo;
  int kl;
};

// fp16 ring (K-tiles of 32 halves, pairs of 64). K-contiguous: chunk c covers rows 8c..8c+7
// and the pair's 64 k; lim is the rows left in the matrix from the tile's first (M - m0 or
// N - n0). MN-contiguous: chunk c belongs to K-tile h = c / (nchunks / 2) and holds k rows
// cl * (1024 / rb_bytes).. of it (cl = c % (nchunks / 2)), rb_bytes per k row, 32-byte blocks
// XOR-swizzled by hsw(k); lim is the columns left.
constexpr Copy plan_f16(bool kcontig, int c, int nchunks, int rb_bytes, long ld, long lim, int lane) {
  if (kcontig) {
    const int row = 8 * c + (lane >> 3), q = kc8_octet(row, lane & 7);
    return {lim > row ? (unsigned)((long)row * ld * 2 + 16 * q) : kOutOfRange, 8 * q};
  }
  const int h = c / (nchunks / 2), cl = c % (nchunks / 2);
  const int gpr = rb_bytes / 16;
  const int k = cl * (1024 / rb_bytes) + lane / gpr, qp = lane % gpr;
  const int q = 2 * ((qp >> 1) ^ hsw(k)) + (qp & 1);
  return {lim > 8 * q ? (unsigned)((long)(32 * h + k) * ld * 2 + 16 * q) : kOutOfRange, 32 * h + k};
}

// The k of pair pp that remain in K (0..64): an fp16 copy is live only when its kl is below.
constexpr int f16_krem(long K, long pp) {
  const long r = K - pp * 64;
  return (int)(r < 0 ? 0 : (r > 64 ? 64 : r));
}
constexpr unsigned f16_offset(const Copy &cp, int krem) { return cp.kl < krem ? cp.vo : kOutOfRange; }

// fp32 ring (K-tiles of 16 floats, pairs of 32): the same chunking, 16-byte blocks of an
// MN-contiguous k row swizzled by msw32(k).
constexpr unsigned plan_f32(bool kcontig, int c, int nchunks, int rb_bytes, long ld, long lim, int lane) {
  if (kcontig) {
    const int row = 8 * c + (lane >> 3), q = kc8_octet(row, lane & 7);
    return lim > row ? (unsigned)((long)row * ld * 4 + 16 * q) : kOutOfRange;
  }
  const int h = c / (nchunks / 2), cl = c % (nchunks / 2);
  const int bpr = rb_bytes / 16;
  const int k = cl * (1024 / rb_bytes) + lane / bpr, b = (lane % bpr) ^ msw32(k);
  return lim > 4 * b ? (unsigned)((long)(16 * h + k) * ld * 4 + 16 * b) : kOutOfRange;
}
// Pairs at or past np = K / 32 go through a descriptor with a record count of 0.
constexpr bool f32_pair_live(long pp, long np) { return pp < np; }

// An operand's descriptor base, in elements from its start, for a tile whose first row (or
// column) is t0; and its advance per pair, in bytes (bk: elements per K-tile).
constexpr long base_elems(bool kcontig, long t0, long ld) { return kcontig ? t0 * ld : t0; }
constexpr long pair_step_bytes(bool kcontig, int bk, long ld, int esz) {
  return kcontig ? 2L * bk * esz : 2L * bk * ld * esz;
}

}  // namespace ring
}  // namespace gn
