// Asynchronous MFMA tile product for gfx950: LDS-DMA operand ring +
// transposing LDS reads.
//
// Computes acc += A^T B for one BM x BN output tile where both operands are
// stored with the contraction axis k as the strided axis (A: [K, M], B: [K, N],
// the layout of every per-sample weight gradient g_b^T x_b).  Four waves split
// the tile 2 x 2; each wave owns (BM/2) x (BN/2) outputs as blocks of 32x32
// v_mfma_f32_32x32x16_{bf16,f16} accumulators.
//
//  * Global -> LDS: buffer_load_dwordx4 ... lds (16 bytes per lane straight into
//    LDS, no VGPR staging).  A BK(k) x R tile of 16-bit values is rows of
//    CPR = R/8 logical chunks of 16 bytes, stored in LDS rows of RS = CPR
//    rounded up to a multiple of 16 chunks (256 bytes: every row starts on
//    the same bank).  Lane l of a wave's load j fills the next 64 slots in
//    order, i.e. slot -> row k = slot / RS, physical chunk p = slot % RS, and
//    the lane loads logical chunk c = p ^ swz(k) of that row.  The XOR (with
//    0, 4, 8 or 12) stays inside each aligned group of 16 chunks, so it maps
//    [0, CPR) into [0, RS); it puts the 4 rows x 4 chunks that half a wave
//    reads in one transposing read onto 16 distinct 16-byte bank groups.
//    Slots whose logical chunk is >= CPR (only when R is not a multiple of
//    128) are padding: their offset lies past the buffer's records, so the
//    load writes zeros and reads no memory.  The buffer resource's record
//    count is the sample's K*ld*2 bytes, so rows past K read as zeros
//    (columns past M/N may carry the next row's values; callers ignore those
//    rows/columns).
//  * S LDS stages, each a separate __shared__ object so that the compiler's
//    wait-count pass can tell the stage being filled from the one being read:
//    while stage kt is consumed, the loads of the next S-2 k-tiles are in flight
//    and waits are explicit s_waitcnt vmcnt(n).
//  * LDS -> MFMA: ds_read_b64_tr_b16.  In a group of 16 lanes, lane r fetches 4
//    consecutive 16-bit values at its address and lane i receives value i%4 of
//    the fetches of lanes i/4, 4+i/4, 8+i/4, 12+i/4.  With lane r pointing at
//    row k0 + r/4, column m0 + 4(r%4), lane i thus holds rows k0..k0+3 of
//    column m0 + i: two such reads give the 8 consecutive k-values one lane
//    contributes to a 32x32x16 MFMA operand.
#pragma once

#include "fdp_common.hpp"

namespace fdp {
namespace dma {

#define FDP_LDS __attribute__((address_space(3)))

typedef __attribute__((__vector_size__(4 * sizeof(short)))) short i16x4;

constexpr int kBK = 64;
constexpr uint32_t kRsrcWord3 = 0x00020000u;  // raw buffer, 32-bit records

__device__ __forceinline__ int swz(int k) { return (k & 3) << 2; }

// LDS row of a tile R values wide, in 16-byte chunks (see above).
__host__ __device__ constexpr int row_chunks(int R) { return (R / 8 + 15) / 16 * 16; }
// Offset of a padding slot: past any buffer's records (< 2^31 bytes) even
// after the k-tile and column offsets (< 2^31) are added, without wrapping.
constexpr uint32_t kPadOffset = 0x80000000u;

// Rows of a k-contiguous tile (below) rounded up so that every wave issues
// whole 1 KB loads: rows of BK 16-bit values, NW waves.
__host__ __device__ constexpr int kc_rows(int R, int BK, int NW) {
  return (R + (NW * 1024) / (BK * 2) - 1) / ((NW * 1024) / (BK * 2)) * ((NW * 1024) / (BK * 2));
}

// Tile geometry: BM x BN outputs, WGM x WGN waves (default 2 x 2), each
// (BM/WGM) x (BN/WGN); k-tiles of BK rows (a multiple of 16) per LDS stage.
// AKC / BKC: operand A / B is stored with k contiguous ([R, K] rows, e.g. a
// layer's grad_output [tokens, out] as the first operand of dX = g W) instead
// of k-strided; such a tile is kept in LDS as rows of BK k-values (below).
template <int BM_, int BN_, int BK_ = kBK, int WGM_ = 2, int WGN_ = 2, bool AKC_ = false,
          bool BKC_ = false>
struct Geom {
  static constexpr int BM = BM_;
  static constexpr int BN = BN_;
  static constexpr int BK = BK_;
  static constexpr int WGM = WGM_;
  static constexpr int WGN = WGN_;
  static constexpr bool AKC = AKC_;
  static constexpr bool BKC = BKC_;
  static constexpr int NW = WGM * WGN;    // waves per workgroup
  static constexpr int KS = BK / 16;      // 16-deep MFMA k-steps per k-tile
  static constexpr int WM = BM / WGM;     // wave tile rows
  static constexpr int WN = BN / WGN;     // wave tile columns
  static constexpr int FI = WM / 32;      // 32-row MFMA blocks per wave
  static constexpr int FJ = WN / 32;      // 32-column MFMA blocks per wave
  static constexpr int ROW_A = row_chunks(BM) * 16;  // LDS bytes per k-row of a k-strided A tile
  static constexpr int ROW_B = row_chunks(BN) * 16;
  static constexpr int TILE_A = AKC ? kc_rows(BM, BK, NW) * BK * 2 : BK * ROW_A;
  static constexpr int TILE_B = BKC ? kc_rows(BN, BK, NW) * BK * 2 : BK * ROW_B;
  static constexpr int STAGE = TILE_A + TILE_B;
  static constexpr int LOADS_A = TILE_A / (NW * 64 * 16);  // per wave per k-tile
  static constexpr int LOADS_B = TILE_B / (NW * 64 * 16);
  static constexpr int LOADS = LOADS_A + LOADS_B;
  static_assert(LOADS_A * NW * 64 * 16 == TILE_A && LOADS_B * NW * 64 * 16 == TILE_B,
                "each wave issues whole 1 KB loads");
  static_assert(BM % 32 == 0 && BN % 32 == 0 && WM % 32 == 0 && WN % 32 == 0, "32x32 blocks");
  static_assert(!(AKC || BKC) || BK == 32 || BK == 64, "k-contiguous tiles: rows of 4 or 8 chunks");
};

// k-contiguous tile in LDS: row r (one m or n) holds the k-tile's BK = 32 or
// 64 values as 4 or 8 chunks of 16 bytes, logical chunk c at physical chunk
// c ^ kc_swz<BK>(r).  An MFMA fragment is one ds_read_b128 per lane (rows
// w0 + lane % 32, chunk 2 ks + lane / 32); the swizzle puts any 16 (and any 8)
// consecutive rows' reads of one chunk on distinct 16-byte bank groups.
template <int BK>
__host__ __device__ constexpr int kc_swz(int r) {
  return BK == 32 ? ((r >> 1) ^ (r >> 2)) & 3 : ((r >> 1) ^ ((r & 1) << 2)) & 7;
}

// One operand's per-thread load state: L buffer loads per k-tile of BK rows.
//
// The loads are issued with inline asm rather than the LDS-DMA builtin: the
// compiler cannot always tell the stage being filled from the one being read
// and then inserts a full vmcnt(0) drain before the reads.  Outside the
// compiler's view, every wait on these loads is the explicit wait_tiles()
// below (its own vmcnt waits stay correct: they only become stronger).
template <int L, int BK = kBK>
struct Operand {
  u32x4 rsrc;        // raw buffer descriptor of the sample's operand
  uint32_t voff[L];  // byte offsets of this thread's loads for k-tile 0, column 0
  uint32_t col;      // byte offset of the tile's first column (uniform)
  uint32_t step;     // bytes per k-tile (BK rows)

  // base: the sample's operand [K, ld] (16-bit); R: tile width; r0: first column.
  template <int R>
  __device__ inline void init(const uint16_t* base, int64_t ld, int64_t K, int64_t r0) {
    constexpr int CPR = R / 8;              // logical 16-byte chunks per row
    constexpr int RS = row_chunks(R);       // physical chunks per LDS row
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    retarget(base, ld, K);
#pragma unroll
    for (int j = 0; j < L; ++j) {
      const int slot = (wave * L + j) * 64 + lane;
      const int k = slot / RS;
      const int c = (slot % RS) ^ swz(k);
      voff[j] = c < CPR ? static_cast<uint32_t>((int64_t(k) * ld + 8 * c) * 2) : kPadOffset;
    }
    retile(r0);
    step = static_cast<uint32_t>(BK * ld * 2);
  }
  // Two samples' R-wide tiles side by side in one LDS row of 2R values: logical
  // chunks [0, R/8) from the sample at `base`, [R/8, R/4) from the one `ds`
  // elements further on (one buffer record over both).  Rows past K of the
  // first sample would read the second's rows: callers need K % BK == 0.
  template <int R>
  __device__ inline void init_pair(const uint16_t* base, int64_t ld, int64_t K, int64_t r0,
                                   int64_t ds) {
    constexpr int CPR = R / 8;
    constexpr int RS = row_chunks(2 * R);
    static_assert(RS == 2 * CPR, "the two samples fill the LDS row");
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const uint64_t a = reinterpret_cast<uint64_t>(base);
    rsrc = u32x4{static_cast<uint32_t>(a), static_cast<uint32_t>(a >> 32) & 0xffffu,
                 static_cast<uint32_t>((ds + K * ld) * 2), kRsrcWord3};
#pragma unroll
    for (int j = 0; j < L; ++j) {
      const int slot = (wave * L + j) * 64 + lane;
      const int k = slot / RS;
      const int c = (slot % RS) ^ swz(k);
      const int64_t e = (c < CPR ? 0 : ds) + int64_t(k) * ld + 8 * (c < CPR ? c : c - CPR);
      voff[j] = static_cast<uint32_t>(e * 2);
    }
    retile(r0);
    step = static_cast<uint32_t>(BK * ld * 2);
  }
  // Operand stored [rows, K] with K contiguous (row stride ld, a multiple of 8
  // elements): the tile's R rows from r0, as rows of BK values (kc_swz
  // layout above); slots of the tile's padding rows (R and up) read nothing.
  // Rows past `rows` read as zeros (the record ends there).  A row's values
  // past K would be the next row's: callers keep K a multiple of BK.
  template <int R>
  __device__ inline void init_kc(const uint16_t* base, int64_t ld, int64_t rows, int64_t r0) {
    static_assert(BK == 32 || BK == 64, "rows of 4 or 8 chunks");
    constexpr int CPK = BK / 8;  // 16-byte chunks per row
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const uint64_t a = reinterpret_cast<uint64_t>(base);
    rsrc = u32x4{static_cast<uint32_t>(a), static_cast<uint32_t>(a >> 32) & 0xffffu,
                 static_cast<uint32_t>(rows * ld * 2), kRsrcWord3};
#pragma unroll
    for (int j = 0; j < L; ++j) {
      const int slot = (wave * L + j) * 64 + lane;
      const int r = slot / CPK;
      const int c = (slot % CPK) ^ kc_swz<BK>(r);
      voff[j] = r < R ? static_cast<uint32_t>((int64_t(r) * ld + 8 * c) * 2) : kPadOffset;
    }
    col = static_cast<uint32_t>(r0 * ld * 2);
    step = static_cast<uint32_t>(BK * 2);
  }
  // The same tile of another sample (same ld, K and columns).  Records past
  // K*ld*2 bytes read as zero.
  __device__ __forceinline__ void retarget(const uint16_t* base, int64_t ld, int64_t K) {
    const uint64_t a = reinterpret_cast<uint64_t>(base);
    rsrc = u32x4{static_cast<uint32_t>(a), static_cast<uint32_t>(a >> 32) & 0xffffu,
                 static_cast<uint32_t>(K * ld * 2), kRsrcWord3};
  }
  // Another tile (first column r0) of the same operand.
  __device__ __forceinline__ void retile(int64_t r0) { col = static_cast<uint32_t>(r0 * 2); }

  // buffer_load_dwordx4 ... lds: lane l of load j writes 16 bytes to
  // tile + (wave*L + j)*1024 + 16*l; M0 holds the wave's LDS address for the
  // load and is restored afterwards (the compiler may keep a value in it).
  __device__ __forceinline__ void issue(FDP_LDS char* tile, int kt) const {
    const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t lds = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(tile)) + wave * L * 1024;
    const uint32_t add = step * static_cast<uint32_t>(kt) + col;
    u32x4 r;
#pragma unroll
    for (int w = 0; w < 4; ++w) r[w] = static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(rsrc[w]));
#pragma unroll
    for (int j = 0; j < L; ++j) {
      uint32_t saved;
      asm volatile(
          "s_mov_b32 %0, m0\n\t"
          "s_mov_b32 m0, %1\n\t"
          "buffer_load_dwordx4 %2, %3, 0 offen lds\n\t"
          "s_mov_b32 m0, %0"
          : "=&s"(saved)
          : "s"(lds + j * 1024), "v"(voff[j] + add), "s"(r)
          : "memory");
    }
  }
};

// Byte offset (inside a tile of row width R, k-step 0) of this lane's
// transposing read for MFMA rows w0 + 32i .. +31, k sub-group h.
template <int R>
__device__ __forceinline__ uint32_t frag_off(int w0, int i, int h) {
  const int lane = threadIdx.x & 63;
  const int g = lane >> 4, r = lane & 15;
  const int m = w0 + 32 * i + 16 * (g & 1) + 4 * (r & 3);
  const int k = 8 * (g >> 1) + 4 * h + (r >> 2);
  return static_cast<uint32_t>(k * (row_chunks(R) * 16) + (((m >> 3) ^ swz(k)) * 16) +
                               ((m >> 2) & 1) * 8);
}

// Byte offset inside a k-contiguous tile of this lane's plain read for MFMA
// rows w0 + 32i .. +31 at k-step 0 (8 k-values: chunk lane / 32).  Chunk
// 2 ks + h of a row sits at physical chunk (2 ks) ^ (h ^ kc_swz(r)), and a
// row is 64 or 128 bytes, so k-step ks reads at this offset ^ (ks << 5).
template <int BK>
__device__ __forceinline__ uint32_t kc_frag_off(int w0, int i) {
  const int lane = threadIdx.x & 63;
  const int r = w0 + 32 * i + (lane & 31);
  return static_cast<uint32_t>(r * (BK * 2) + (((lane >> 5) ^ kc_swz<BK>(r)) * 16));
}

// Per operand two offsets per fragment: the two transposing half reads of
// k-step 0 (k-strided tile; later k-steps add 16 rows), or the plain read of
// k-step 0 (k-contiguous tile; [1] unused).
template <class G>
struct FragOffsets {
  uint32_t a[G::FI][2], b[G::FJ][2];
  __device__ __forceinline__ void init(int wm, int wn) {
#pragma unroll
    for (int i = 0; i < G::FI; ++i)
#pragma unroll
      for (int h = 0; h < 2; ++h)
        a[i][h] = G::AKC ? kc_frag_off<G::BK>(wm, i) : frag_off<G::BM>(wm, i, h);
#pragma unroll
    for (int j = 0; j < G::FJ; ++j)
#pragma unroll
      for (int h = 0; h < 2; ++h)
        b[j][h] = (G::BKC ? kc_frag_off<G::BK>(wn, j) : frag_off<G::BN>(wn, j, h)) + G::TILE_A;
  }
};

__device__ __forceinline__ uint4 read_frag(const FDP_LDS char* stage, uint32_t o0, uint32_t o1) {
  const i16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      reinterpret_cast<FDP_LDS i16x4*>(const_cast<FDP_LDS char*>(stage) + o0));
  const i16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      reinterpret_cast<FDP_LDS i16x4*>(const_cast<FDP_LDS char*>(stage) + o1));
  uint4 v;
  v.x = uint32_t(uint16_t(lo[0])) | (uint32_t(uint16_t(lo[1])) << 16);
  v.y = uint32_t(uint16_t(lo[2])) | (uint32_t(uint16_t(lo[3])) << 16);
  v.z = uint32_t(uint16_t(hi[0])) | (uint32_t(uint16_t(hi[1])) << 16);
  v.w = uint32_t(uint16_t(hi[2])) | (uint32_t(uint16_t(hi[3])) << 16);
  return v;
}

// One lane's 16 bytes of a k-contiguous tile (ds_read_b128).
__device__ __forceinline__ uint4 read_plain(const FDP_LDS char* stage, uint32_t o) {
  const u32x4 v = *reinterpret_cast<const FDP_LDS u32x4*>(stage + o);
  return make_uint4(v[0], v[1], v[2], v[3]);
}

template <class DT>
__device__ __forceinline__ f32x16 mfma16(uint4 a, uint4 b, f32x16 c) {
  if constexpr (DT::code == FDP_BF16) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a),
                                                   __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
  } else {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a),
                                                  __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
  }
}

// Fragments of one 16-deep k-step.
template <class G>
struct Frags {
  uint4 a[G::FI], b[G::FJ];
  __device__ __forceinline__ void load(const FDP_LDS char* st, const FragOffsets<G>& fo, int ks) {
#pragma unroll
    for (int j = 0; j < G::FJ; ++j) {
      if constexpr (G::BKC)
        b[j] = read_plain(st, fo.b[j][0] ^ (ks << 5));
      else
        b[j] = read_frag(st, fo.b[j][0] + ks * 16 * G::ROW_B, fo.b[j][1] + ks * 16 * G::ROW_B);
    }
#pragma unroll
    for (int i = 0; i < G::FI; ++i) {
      if constexpr (G::AKC)
        a[i] = read_plain(st, fo.a[i][0] ^ (ks << 5));
      else
        a[i] = read_frag(st, fo.a[i][0] + ks * 16 * G::ROW_A, fo.a[i][1] + ks * 16 * G::ROW_A);
    }
  }
};

// One BK-deep k-tile of the wave's sub-tile from LDS stage `st`.
template <class DT, class G>
__device__ __forceinline__ void compute_stage(const FDP_LDS char* st, const FragOffsets<G>& fo,
                                              f32x16 (&acc)[G::FI][G::FJ]) {
#pragma unroll
  for (int ks = 0; ks < G::KS; ++ks) {
    Frags<G> f;
    f.load(st, fo, ks);
#pragma unroll
    for (int i = 0; i < G::FI; ++i)
#pragma unroll
      for (int j = 0; j < G::FJ; ++j) acc[i][j] = mfma16<DT>(f.a[i], f.b[j], acc[i][j]);
  }
}

// The same, handing each k-step's fragments to fh(ks, frags) after its MFMAs.
template <class DT, class G, class FH>
__device__ __forceinline__ void compute_stage_f(const FDP_LDS char* st, const FragOffsets<G>& fo,
                                                f32x16 (&acc)[G::FI][G::FJ], const FH& fh) {
#pragma unroll
  for (int ks = 0; ks < G::KS; ++ks) {
    Frags<G> f;
    f.load(st, fo, ks);
#pragma unroll
    for (int i = 0; i < G::FI; ++i)
#pragma unroll
      for (int j = 0; j < G::FJ; ++j) acc[i][j] = mfma16<DT>(f.a[i], f.b[j], acc[i][j]);
    fh(ks, f);
  }
}

// s_waitcnt vmcnt(n) with the other counters left alone (gfx9 encoding).
template <int N>
__device__ __forceinline__ void wait_vm() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 0xf) | (0x7 << 4) | (0xf << 8) | ((N >> 4) << 14));
}
// Wait until at most `tiles` k-tiles (L loads each) of this thread's loads are
// outstanding (stores issued in between only make the wait stronger).
// (Counts above the 6-bit vmcnt field are clamped: a smaller count only makes
// the wait stronger.)
template <int L>
__device__ __forceinline__ void wait_tiles(int tiles) {
  switch (tiles) {
    case 0: wait_vm<0>(); break;
    case 1: wait_vm<(L < 63 ? L : 63)>(); break;
    case 2: wait_vm<(2 * L < 63 ? 2 * L : 63)>(); break;
    default: wait_vm<(3 * L < 63 ? 3 * L : 63)>(); break;
  }
}

// Workgroup barrier that also completes this wave's LDS reads and keeps the
// compiler from moving memory operations across it.  (A __syncthreads() would
// add a vmcnt(0) wait for the in-flight LDS-DMA loads, serialising the ring.)
__device__ __forceinline__ void barrier() {
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

// The S stages live in separate __shared__ objects owned by the kernel.
struct Stages {
  FDP_LDS char* s[4];
  __device__ __forceinline__ FDP_LDS char* get(int i) const {
    switch (i) {
      case 0: return s[0];
      case 1: return s[1];
      case 2: return s[2];
      default: return s[3];
    }
  }
};

// Per-thread state of one (tile, sample) product.
template <class G>
struct Job {
  Operand<G::LOADS_A, G::BK> a;
  Operand<G::LOADS_B, G::BK> b;
  __device__ __forceinline__ void init(const uint16_t* pa, int64_t lda, const uint16_t* pb,
                                       int64_t ldb, int64_t K, int64_t m0, int64_t n0) {
    a.template init<G::BM>(pa, lda, K, m0);
    b.template init<G::BN>(pb, ldb, K, n0);
  }
  __device__ __forceinline__ void retarget(const uint16_t* pa, int64_t lda, const uint16_t* pb,
                                           int64_t ldb, int64_t K) {
    a.retarget(pa, lda, K);
    b.retarget(pb, ldb, K);
  }
  __device__ __forceinline__ void retile(int64_t m0, int64_t n0) {
    a.retile(m0);
    b.retile(n0);
  }
  __device__ __forceinline__ void issue(FDP_LDS char* stage, int kt) const {
    a.issue(stage, kt);
    b.issue(stage + G::TILE_A, kt);
  }
};

// Per-thread state of two samples' products of one output tile, loaded side
// by side (Operand::init_pair): the A tile's rows hold both samples' BM/2
// columns, the B tile's both samples' BN/2.
template <class G>
struct PairJob {
  Operand<G::LOADS_A, G::BK> a;
  Operand<G::LOADS_B, G::BK> b;
  // pa/pb: the first sample's operands; dsa/dsb: elements to the second's
  __device__ __forceinline__ void init(const uint16_t* pa, int64_t lda, int64_t dsa,
                                       const uint16_t* pb, int64_t ldb, int64_t dsb, int64_t K,
                                       int64_t m0, int64_t n0) {
    a.template init_pair<G::BM / 2>(pa, lda, K, m0, dsa);
    b.template init_pair<G::BN / 2>(pb, ldb, K, n0, dsb);
  }
  __device__ __forceinline__ void issue(FDP_LDS char* stage, int kt) const {
    a.issue(stage, kt);
    b.issue(stage + G::TILE_A, kt);
  }
};

// acc += A_tile^T B_tile over nk k-tiles with an S-stage ring (S in {2, 3, 4}).
template <class DT, class G, int S>
__device__ inline void gemm(const Job<G>& job, int nk, const FragOffsets<G>& fo, const Stages& st,
                            f32x16 (&acc)[G::FI][G::FJ]) {
  static_assert(S >= 2 && S <= 4, "stages");
  wait_vm<0>();  // no older vector-memory operation may confuse the counting below
#pragma unroll
  for (int s = 0; s < S - 1; ++s)
    if (s < nk) job.issue(st.get(s), s);
  for (int base = 0; base < nk; base += S) {
#pragma unroll
    for (int s = 0; s < S; ++s) {
      const int kt = base + s;
      if (kt < nk) {
        const int ahead = nk - 1 - kt;
        wait_tiles<G::LOADS>(ahead < S - 2 ? ahead : S - 2);
        barrier();
        if (kt + S - 1 < nk) job.issue(st.get((s + S - 1) % S), kt + S - 1);
        compute_stage<DT, G>(st.get(s), fo, acc);
      }
    }
  }
  barrier();  // every wave is done reading before the ring is reused
}

struct NoHook {
  __device__ __forceinline__ void operator()(int) const {}
};
struct NoFragHook {
  template <class F>
  __device__ __forceinline__ void operator()(int, int, const F&) const {}
};

// acc += A_tile^T B_tile over nk k-tiles with an S-stage ring, fragments
// double-buffered in registers: the LDS reads of k-step s+1 (the next k-tile's
// first step at a k-tile's end, after its wait and barrier) are issued before
// the MFMAs of step s, and scheduling groups interleave one MFMA with the DS
// reads of the next step.  The refill of the stage a k-tile frees (k-tile
// kt + S) is issued after that k-tile's last MFMAs rather than right after
// the barrier: the waves leave the barrier straight into matrix work (on the
// wide kernel's cfg2 call 57.1-57.5 against 59.8-59.9 us per call).  KS must
// be even (fragment buffers alternate).
// hook(kt) runs at the start of every k-tile kt: VALU work placed there
// (reading no memory) overlaps the matrix cores' work of the other wave of
// the SIMD.  fhook(kt, ks, frags) runs after the MFMAs of k-step ks are
// issued, with that step's operand fragments (VALU work on them overlaps
// the MFMAs in flight).
// J: Job<G> (one sample) or PairJob<G> (two samples side by side).
template <class DT, class G, int S, class J, class Hook = NoHook, class FragHook = NoFragHook>
__device__ inline void gemm_pipe(const J& job, int nk, const FragOffsets<G>& fo,
                                 const Stages& st, f32x16 (&acc)[G::FI][G::FJ],
                                 const Hook& hook = Hook(), const FragHook& fhook = FragHook()) {
  static_assert(S >= 2 && S <= 4, "stages");
  static_assert(G::KS % 2 == 0, "an even number of k-steps per k-tile");
  wait_vm<0>();
#pragma unroll
  for (int s = 0; s < S - 1; ++s)
    if (s < nk) job.issue(st.get(s), s);
  if (nk <= 0) return;
  wait_tiles<G::LOADS>(nk - 1 < S - 2 ? nk - 1 : S - 2);
  barrier();
  if (S - 1 < nk) job.issue(st.get(S - 1), S - 1);
  Frags<G> f[2];
  f[0].load(st.get(0), fo, 0);
  for (int base = 0; base < nk; base += S) {
#pragma unroll
    for (int s = 0; s < S; ++s) {
      const int kt = base + s;
      if (kt < nk) {
        hook(kt);
#pragma unroll
        for (int ks = 0; ks < G::KS; ++ks) {
          const int cur = ks & 1;
          if (ks + 1 < G::KS) {
            f[cur ^ 1].load(st.get(s), fo, ks + 1);
          } else if (kt + 1 < nk) {
            const int ahead = nk - 2 - kt;
            wait_tiles<G::LOADS>(ahead < S - 2 ? ahead : S - 2);
            barrier();
            f[cur ^ 1].load(st.get((s + 1) % S), fo, 0);
          }
#pragma unroll
          for (int i = 0; i < G::FI; ++i)
#pragma unroll
            for (int j = 0; j < G::FJ; ++j) acc[i][j] = mfma16<DT>(f[cur].a[i], f[cur].b[j], acc[i][j]);
          constexpr int nm = G::FI * G::FJ, nr = 2 * (G::FI + G::FJ);
          constexpr int per = (nr + nm - 1) / nm;
#pragma unroll
          for (int t = 0; t < nm; ++t) {
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);    // one MFMA
            __builtin_amdgcn_sched_group_barrier(0x100, per, 0);  // then DS reads
          }
          // the freed stage's refill goes out behind this step's MFMAs
          if (ks + 1 == G::KS && kt + S < nk) job.issue(st.get(s), kt + S);
          fhook(kt, ks, f[cur]);
        }
      }
    }
  }
  barrier();  // every wave is done reading before the ring is reused
}

}  // namespace dma
}  // namespace fdp
