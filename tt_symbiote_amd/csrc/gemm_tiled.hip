// Tiled bf16 GEMMs for prefill-size problems (MFMA-bound): dense projections and the grouped
// expert GEMMs over ragged, expert-sorted rows.
//
// Reference: the projections of TTNNBailingMoEAttention (ttnn_attention.py:2001-2011) at
// sequence length > 1, and the expert sparse_matmuls of TTNNExperts.forward
// (ttnn_moe.py:1250-1289) with the shared expert (ttnn_moe.py:656-675), for prefill batches.
//
// Design (gfx950). What bounds these kernels was measured, not assumed: a wave-wide load of
// 16 rows x 64 bytes (a 32-column step of K-major rows) reaches ~30 B/clk per CU from L2, one of
// 8 rows x 128 bytes ~50 B/clk, while LDS reads (~190 B/clk) and back-to-back MFMAs (94% of
// peak) have room; and the chip clocks down to 2.0-2.25 GHz under these kernels. Two tile
// shapes (and a thin variant of the first):
//   gemm_tile_kernel / gemm_tile_persistent (dense projections; grouped gate/up and down on a
//     persistent grid while the segment list has at most 512 entries): 256 x 256 tiles, one
//     workgroup of 8 waves per CU, each wave a 64 x 128 block (4 x 8 v_mfma_f32_16x16x32_bf16
//     tiles). The K loop moves 64 columns per step (128-byte rows: whole cache lines) through two
//     64 KB LDS stages; each step is computed in two 32-column halves whose fragment reads
//     overlap the other half's MFMAs, with one barrier per step. In the persistent kernels a
//     tile of at most 64 valid rows runs thin_tile instead: three 40 KB stages (64 A rows and
//     256 B rows each), two steps of lookahead.
//   gemm_tile128_kernel (router logits, N = E = 256: few tiles; grouped down projection over
//     longer segment lists): 128 x 256 tiles, two workgroups of 8 waves per CU, each
//     wave a 64 x 64 block; 32 columns per step through a 3-stage 72 KB ring. The second
//     workgroup covers a tile's prologue (segment lookup, first loads) and epilogue, which a
//     one-workgroup shape leaves bare at 16 steps.
// Operand tiles go from global memory straight into LDS (global_load_lds_dwordx4, no register
// staging). A wave-wide LDS-DMA instruction writes 1 KB contiguously: lane l takes row l / c,
// 16-byte slot l % c (c = chunks per row), fetching global chunk (l % c) ^ swz(row), so that
// chunk j of row r sits in slot j ^ swz(r) and the rows of an MFMA fragment read fall in
// distinct banks. Workgroups are ordered so that each XCD's L2 sees a contiguous run of tiles.
// The MFMAs compute transposed 16 x 16 tiles, so a lane ends with 4 consecutive columns of one
// row; bf16 outputs of the 256 x 256 tiles go back out through LDS as whole 128-byte lines
// (store_block_lds), fp32 outputs and the 128 x 256 tiles write 16 (fp32) or 8 (bf16) bytes per
// lane directly.
//   DENSE:   out[M, N] = A[M, K] . W[N, K]^T (+ bias) (+ residual fp32 or bf16), bf16 or
//            fp32 out.
//   GATE_UP: rows of a segment gather x[sorted_tokens[row]]; the B tile holds 128 gate rows and
//            the matching 128 up rows of the expert, so each wave's block pairs 64 gate with 64
//            up columns and the epilogue writes h = silu(gate) * up (bf16).
//   DOWN:    rows of a segment are h rows (contiguous); y = h . W_down^T (fp32 or bf16).
// Rows past a tile's valid rows and columns past N repeat the last row / column in the loads
// (always in bounds) and are not stored; in the 256-row tiles, 64-row bands wholly past the
// valid rows skip their MFMAs (and their A loads).
// Grouped modes: the workgroup's row tile is found from the device-side segment list (each
// segment owns ceil(count / tile rows) consecutive row tiles); workgroups past the last tile
// exit.
#include <type_traits>

#include "common.h"

namespace sym {

constexpr int kMaxGemmSegments = 4096;  // grid bound on segments (y range)

enum TileMode { kDense = 0, kGateUp = 1, kDown = 2 };

struct TileArgs {
  const uint16_t* a;        // DENSE/DOWN: rows [., K]; GATE_UP: x [T, K]
  const uint16_t* w;        // DENSE: [N, K]; GATE_UP: [S, 2I, K]; DOWN: [S, N, K]
  const uint16_t* bias;     // DENSE, optional [N]
  const float* residual;    // DENSE, optional [M, N] fp32
  const uint16_t* residual_bf16;  // DENSE with out_f32, optional [M, N] bf16 (store_block)
  const int32_t* sorted_tokens;
  const int32_t* seg_expert;
  const int32_t* seg_offset;
  const int32_t* seg_count;
  const int32_t* n_segments;
  int max_segments;         // grouped modes: entries of the seg_* arrays (>= *n_segments)
  int M, N, K;              // GATE_UP: N = I (h columns); DOWN: N = H
  uint16_t* out_bf16;
  float* out_f32;
  long long w_zstride;      // DENSE: grid z selects weight plane w + z * w_zstride ...
  long long out_zstride;    // ... and output plane out + z * out_zstride (elements)
  int full_rt;              // DENSE with tail_rows > 0: row tiles 0 .. full_rt - 1 have TM rows,
  int tail_rows;            // the rows from full_rt * TM on tiles of tail_rows (one plane)
  int* tickets;             // gemm_tile_persistent: the caller's 8 per-XCD tile counters
};

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// dma16 (common.h) moves 16 bytes per lane from global memory into LDS; the kernels below wait
// for it explicitly (SYM_TILE_SYNC) before the barrier that publishes a stage.

// Wait until at most N of this wave's vector-memory loads are outstanding (the LDS-DMA of later
// steps) and for this wave's LDS reads, then the workgroup barrier. The asm is a compiler memory
// barrier, so no LDS access moves across it; a plain __syncthreads would also wait for every DMA
// in flight.
#define SYM_TILE_SYNC(N) \
  asm volatile("s_waitcnt vmcnt(" #N ")\n\ts_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory")

// Tile t of n for the workgroup with linear id lin, or -1. Workgroups are dispatched to the 8
// XCDs round-robin by linear id (lin % 8), and each XCD has its own L2: XCD x takes the
// contiguous range of tiles [x n / 8, (x + 1) n / 8) in dispatch order, so the column tiles of a
// row tile (same A rows) and the row tiles of an expert (same weights) meet in one L2.
__device__ __forceinline__ int xcd_tile(int lin, int n) {
  const int x = lin & 7, j = lin >> 3;
  const int q = n >> 3, r = n & 7;
  if (j >= q + (x < r ? 1 : 0)) return -1;
  return x * q + min(x, r) + j;
}

// The tile of workgroup lin (nx column tiles per row tile). DENSE: row tiles of TM rows of
// p.M; grouped modes: each segment owns ceil(seg_count / TM) consecutive row tiles, found by
// every wave scanning the segment list (prefix sums by lane shuffles; no LDS, no barrier, all
// waves agree): once for the number of row tiles, then up to the segment holding the row tile.
// The counts, offsets and experts of 512 segments at a time load together with n_segments (the
// first 512 speculatively, bounded by max_segments), so that a tile with at most 512 segments
// in the list waits for one round trip. Returns false past the last tile (the grouped grids
// are sized for the worst case). Results are wave-uniform.
struct TileLoc {
  int row0, rows, e, ct, z;  // first row, valid rows, expert, column tile, weight plane
};
template <int MODE, int TM>
__device__ __forceinline__ bool locate_tile(const TileArgs& p, int lane, TileLoc& loc) {
  const int nx = gridDim.x;
  const int lin = (blockIdx.z * gridDim.y + blockIdx.y) * nx + blockIdx.x;
  loc.e = 0;
  loc.z = 0;
  if constexpr (MODE == kDense) {
    const int nxy = nx * gridDim.y;
    if (p.tail_rows > 0) {
      // whole tiles first, then the tail's smaller tiles, each range in its XCD runs
      const int nfull = p.full_rt * nx;
      const bool full = lin < nfull;
      const int t = full ? xcd_tile(lin, nfull) : xcd_tile(lin - nfull, nxy - nfull);
      const int gy = t / nx;
      loc.ct = t - gy * nx;
      loc.row0 = full ? gy * TM : p.full_rt * TM + gy * p.tail_rows;
      loc.rows = min(full ? TM : p.tail_rows, p.M - loc.row0);
      return true;
    }
    const int t = xcd_tile(lin, nxy * gridDim.z);  // the grid holds exactly the tiles
    loc.z = t / nxy;
    const int gy = (t - loc.z * nxy) / nx;
    loc.ct = t - loc.z * nxy - gy * nx;
    loc.row0 = gy * TM;
    loc.rows = min(TM, p.M - loc.row0);
    return true;
  } else {
    constexpr int kBatch = 8;  // 64-segment chunks per batch
    int cnt[kBatch], off[kBatch], exp[kBatch];
    auto load = [&](int b) {
#pragma unroll
      for (int c = 0; c < kBatch; ++c) {
        const int s = (b * kBatch + c) * 64 + lane;
        const bool in = s < p.max_segments;
        cnt[c] = in ? p.seg_count[s] : 0;
        off[c] = in ? p.seg_offset[s] : 0;
        exp[c] = in ? p.seg_expert[s] : 0;
      }
    };
    load(0);
    const int nseg = p.n_segments[0];
    const int nbatch = (nseg + 64 * kBatch - 1) / (64 * kBatch);
    auto tiles = [&](int b, int c) {
      return (b * kBatch + c) * 64 + lane < nseg ? (cnt[c] + TM - 1) / TM : 0;
    };
    int ntile = 0;
    for (int b = 0; b < nbatch; ++b) {
      if (b > 0) load(b);
#pragma unroll
      for (int c = 0; c < kBatch; ++c) ntile += tiles(b, c);
    }
#pragma unroll
    for (int off2 = 32; off2 > 0; off2 >>= 1) ntile += __shfl_xor(ntile, off2);
    const int t = xcd_tile(lin, ntile * nx);
    if (t < 0) return false;
    const int g = t / nx;
    loc.ct = __builtin_amdgcn_readfirstlane(t - g * nx);
    int found = 0, run = 0;
    for (int b = 0; b < nbatch && !found; ++b) {
      if (nbatch > 1) load(b);  // one batch: the values are still in registers
#pragma unroll
      for (int c = 0; c < kBatch; ++c) {
        const int nt = tiles(b, c);
        int x = nt;
#pragma unroll
        for (int o = 1; o < 64; o <<= 1) {
          const int y = __shfl_up(x, o);
          if (lane >= o) x += y;
        }
        const int s0 = run + x - nt;
        const unsigned long long hit = __ballot(nt > 0 && s0 <= g && g < s0 + nt);
        if (!found && hit) {
          const int l = __ffsll((long long)hit) - 1;
          const int rt = g - __shfl(s0, l);
          // wave-uniform (the compiler cannot see it through the lane shuffles)
          loc.e = __builtin_amdgcn_readfirstlane(__shfl(exp[c], l));
          loc.row0 = __builtin_amdgcn_readfirstlane(__shfl(off[c], l) + rt * TM);
          loc.rows = __builtin_amdgcn_readfirstlane(min(TM, __shfl(cnt[c], l) - rt * TM));
          found = 1;
        }
        run += __shfl(x, 63);
      }
    }
    return found;  // (always true: g < ntile)
  }
}

// Output-plane and weight-matrix bases of a tile: DENSE plane z; GATE_UP / DOWN expert e.
template <int MODE>
__device__ __forceinline__ const uint16_t* tile_weights(TileArgs& p, const TileLoc& loc) {
  if constexpr (MODE == kDense) {
    if (p.out_f32) p.out_f32 += loc.z * p.out_zstride;
    else p.out_bf16 += loc.z * p.out_zstride;
    return p.w + loc.z * p.w_zstride;
  } else if constexpr (MODE == kGateUp) {
    return p.w + (size_t)loc.e * 2 * p.N * p.K;
  } else {
    return p.w + (size_t)loc.e * p.N * p.K;
  }
}

// Byte offset of B row br (0 .. TN - 1) of column tile ct within the tile's weight matrix.
// GATE_UP: TN / 2 gate rows then the matching TN / 2 up rows. Rows past N repeat the last one.
template <int MODE, int TN>
__device__ __forceinline__ uint32_t b_row_offset(const TileArgs& p, int ct, int br) {
  uint32_t brow;
  if constexpr (MODE == kGateUp) {
    const int col = min(ct * (TN / 2) + (br % (TN / 2)), p.N - 1);
    brow = (uint32_t)(br < TN / 2 ? col : p.N + col);
  } else {
    brow = (uint32_t)min(ct * TN + br, p.N - 1);
  }
  return brow * (uint32_t)p.K * 2u;
}

// Byte offset of A row r (< rows) of the tile: GATE_UP gathers x[sorted_tokens[row]].
template <int MODE>
__device__ __forceinline__ uint32_t a_row_offset(const TileArgs& p, const TileLoc& loc, int r) {
  uint32_t arow;
  if constexpr (MODE == kGateUp) arow = (uint32_t)p.sorted_tokens[loc.row0 + r];
  else arow = (uint32_t)(loc.row0 + r);
  return arow * (uint32_t)p.K * 2u;
}

// Epilogue of one wave's 64 x (16 NJ) block. The MFMAs take the B fragment as their first
// operand and A as their second, i.e. compute transposed 16 x 16 tiles: lane l holds row l%16,
// columns 4*(l/16) .. +3 of each.
// GATE_UP: tiles j < NJ/2 are gate columns col0 + 16 j .., tiles j + NJ/2 the matching up
// columns; h = silu(gate) * up. Otherwise tile j is columns col0 + 16 j ..
// The 4 output values of tile (i, j) held by this lane, for output row orow and first column
// col (col < N): GATE_UP h, DENSE plus bias and residual, DOWN as computed.
template <int MODE, int NJ>
__device__ __forceinline__ void tile_values(const TileArgs& p, const floatx4 (&acc)[4][NJ], int i,
                                            int j, size_t orow, int col, float (&v)[4]) {
  if constexpr (MODE == kGateUp) {
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      // silu(g) = g / (1 + 2^(-g log2(e))) by v_exp_f32 and v_rcp_f32 (about 1 ulp each;
      // h is rounded to bf16 next). g -> -inf: 1 / inf = 0; g -> +inf: 1 / 1.
      const float g = acc[i][j][q], u = acc[i][j + NJ / 2][q];
      const float e = __builtin_amdgcn_exp2f(g * -1.44269504f);
      v[q] = g * __builtin_amdgcn_rcpf(1.0f + e) * u;
    }
  } else {
#pragma unroll
    for (int q = 0; q < 4; ++q) v[q] = acc[i][j][q];
    if constexpr (MODE == kDense) {
      if (p.bias) {
        const uint2 b = *reinterpret_cast<const uint2*>(p.bias + col);
        v[0] += bf16_lo(b.x); v[1] += bf16_hi(b.x); v[2] += bf16_lo(b.y); v[3] += bf16_hi(b.y);
      }
      if (p.residual) {
        const float4 rr = *reinterpret_cast<const float4*>(p.residual + orow * p.N + col);
        v[0] += rr.x; v[1] += rr.y; v[2] += rr.z; v[3] += rr.w;
      }
    }
  }
}

// Direct epilogue: each (i, j) tile as one 8-byte (bf16) or 16-byte (fp32) write per lane, i.e.
// an instruction writes 32 or 64 bytes into each of 16 rows.
template <int MODE, int NJ>
__device__ __forceinline__ void store_block(const TileArgs& p, const floatx4 (&acc)[4][NJ],
                                            const TileLoc& loc, int rbase, int col0, int lane) {
  const int r16 = lane & 15, kq = lane >> 4;
  constexpr int NT = MODE == kGateUp ? NJ / 2 : NJ;  // output tiles per 16-row sub-tile
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int r = rbase + i * 16 + r16;
    if (r >= loc.rows) continue;
    const size_t orow = (size_t)(loc.row0 + r);
    // a bf16 residual: the sub-tile's loads all go out before its stores (a load after a store
    // to memory that may alias it would wait for its own round trip)
    uint2 rb[MODE == kDense ? NT : 1];
    if constexpr (MODE == kDense) {
      if (p.residual_bf16) {
#pragma unroll
        for (int j = 0; j < NT; ++j) {
          const int col = min(col0 + j * 16 + kq * 4, p.N - 4);
          rb[j] = *reinterpret_cast<const uint2*>(p.residual_bf16 + orow * p.N + col);
        }
      }
    }
#pragma unroll
    for (int j = 0; j < NT; ++j) {
      const int col = col0 + j * 16 + kq * 4;
      if (col >= p.N) continue;  // N % 16 == 0: the 4 columns are all valid or all not
      float v[4];
      tile_values<MODE, NJ>(p, acc, i, j, orow, col, v);
      if constexpr (MODE == kDense) {
        if (p.residual_bf16) {
          v[0] += bf16_lo(rb[j].x); v[1] += bf16_hi(rb[j].x);
          v[2] += bf16_lo(rb[j].y); v[3] += bf16_hi(rb[j].y);
        }
      }
      if (MODE != kGateUp && p.out_f32)
        *reinterpret_cast<float4*>(p.out_f32 + orow * p.N + col) =
            make_float4(v[0], v[1], v[2], v[3]);
      else
        *reinterpret_cast<uint2*>(p.out_bf16 + orow * p.N + col) =
            make_uint2(pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3]));
    }
  }
}

// Epilogue through LDS (bf16 outputs): the wave's 64-row block (COLS = 128 columns, or 64 h
// columns in GATE_UP) goes into the wave's own LDS region `buf` (64 x COLS bf16) in the MFMA
// layout and comes back out as whole rows, so that a store instruction writes 1 KB of whole
// 128-byte lines (4 rows x 256 B or 8 rows x 128 B) instead of 32 bytes into each of 16 rows:
// the direct epilogue's partial lines made the tile's stores its most expensive phase after the
// K loop. The region is row-major with its 16-byte chunks XOR-swizzled by row (chunk c of row r
// at c ^ (r % 16) for 16 chunks per row, c ^ ((r / 2) % 8) for 8), so the 8-byte writes of 16
// rows and the 16-byte reads of whole rows are both free of bank conflicts. LDS operations of a
// wave complete in order, so no barrier is needed between the writes and the reads; the caller
// guarantees that no other wave touches `buf` meanwhile.
template <int MODE, int NJ>
__device__ __forceinline__ void store_block_lds(const TileArgs& p, const floatx4 (&acc)[4][NJ],
                                                const TileLoc& loc, int rbase, int col0,
                                                int lane, uint16_t* buf) {
  constexpr int NT = MODE == kGateUp ? NJ / 2 : NJ;
  constexpr int COLS = NT * 16;   // columns of the wave's block
  constexpr int CH = COLS / 8;    // 16-byte chunks per row (16 or 8)
  constexpr int RPI = 64 / CH;    // rows per 1 KB store instruction (4 or 8)
  // the lane index through an opaque copy: the per-lane addresses below are then computed here,
  // not hoisted out of a persistent kernel's tile loop, where they would hold registers across
  // the K loop
  asm volatile("" : "+v"(lane));
  const int r16 = lane & 15, kq = lane >> 4;
  auto slot = [](int row, int ch) {
    const int sw = CH == 16 ? (row & 15) : ((row >> 1) & 7);
    return row * COLS + (ch ^ sw) * 8;
  };
  const int nrows = min(64, loc.rows - rbase);  // valid rows of the block (wave-uniform)
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    if (i * 16 >= nrows) break;
    const int row = i * 16 + r16;
    const size_t orow = (size_t)(loc.row0 + rbase + row);
#pragma unroll
    for (int j = 0; j < NT; ++j) {
      const int col = col0 + j * 16 + kq * 4;
      if (row >= nrows || col >= p.N) continue;
      float v[4];
      tile_values<MODE, NJ>(p, acc, i, j, orow, col, v);
      *reinterpret_cast<uint2*>(buf + slot(row, 2 * j + (kq >> 1)) + (kq & 1) * 4) =
          make_uint2(pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3]));
    }
  }
  const int rl = lane / CH, ch = lane % CH;
  const int col = col0 + ch * 8;
#pragma unroll
  for (int it = 0; it < 64 / RPI; ++it) {
    if (it * RPI >= nrows) break;
    const int row = it * RPI + rl;
    const uint4 v = *reinterpret_cast<const uint4*>(buf + slot(row, ch));
    if (row < nrows && col < p.N)
      *reinterpret_cast<uint4*>(p.out_bf16 + (size_t)(loc.row0 + rbase + row) * p.N + col) = v;
  }
}

// ================================================================================================
// 256 x 256 tiles (dense projections, router logits, grouped gate/up): 8 waves of 64 x 128, one
// workgroup per CU, 64-column steps through two 64 KB LDS stages. Per step a CU moves 64 KB from
// L2 in whole 128-byte lines for 4 M MACs.
// ================================================================================================
namespace big {
constexpr int kTM = 256, kTN = 256, kTK = 64;
constexpr int kWavesN = 2, kWaves = 8, kThreads = 512;
constexpr int kWC = kTN / kWavesN, kNJ = kWC / 16;  // 128 columns (8 MFMA tiles) per wave
constexpr int kAStage = kTM * kTK, kBStage = kTN * kTK, kStage = kAStage + kBStage;  // bf16
constexpr int kRowsPerDma = 8;  // one wave-wide LDS-DMA instruction: 8 rows x 128 bytes
constexpr int kARows = kTM / kWaves, kBRows = kTN / kWaves;  // rows DMA'd per wave and step
constexpr int kADma = kARows / kRowsPerDma, kBDma = kBRows / kRowsPerDma;  // 4 + 4
static_assert(kADma == 4 && kBDma == 4, "the prologue wait counts");
// LDS slot of 16-byte chunk c (of 8) in row r: c ^ (r % 8), so that the 8 rows of a fragment
// read that share a chunk index fall in distinct banks.
__device__ __forceinline__ int swz(int r) { return r & 7; }
}  // namespace big

// One 256 x 256 tile at loc (p is a copy: tile_weights moves its output pointer to the tile's
// plane). The stages are smem + s * kStage, s = 0, 1 (64 KB each: every fragment read of a stage
// is within the 64 KB immediate offset of an LDS instruction from the stage base).
// hook() runs in every thread after the K loop, before the epilogue (the persistent kernel
// hands out its next tile there, when no operand load of the tile is in flight).
struct NoHook {
  __device__ void operator()() const {}
};
template <int MODE, typename Hook = NoHook>
__device__ __forceinline__ void big_tile(TileArgs p, const TileLoc& loc, uint16_t* smem,
                                         Hook hook = Hook{}) {
  using namespace big;
  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
  const int wm = wave / kWavesN, wn = wave % kWavesN;
  const int r16 = lane & 15, kq = lane >> 4;
  const int K = p.K;

  const uint16_t* wbase = tile_weights<MODE>(p, loc);

  // ---- LDS-DMA sources: this wave fills A rows kARows w .. and B rows kBRows w .. of every
  // stage; lane l takes row + l / 8, slot l % 8, i.e. global chunk slot ^ swz(row). A rows at
  // or past `rows` in groups of kARows are not loaded (their wave skips those instructions and
  // waits for fewer loads; no wave reads those LDS rows for a stored output). Sources are byte
  // offsets from p.a (the host checks that A fits in 4 GB) and from the tile's weight matrix
  // (one expert's, in the grouped modes; the host checks that one fits in 4 GB).
  const int lr = lane >> 3;
  const uint32_t chunk_b = ((lane & 7) ^ swz(lr)) * 16;  // swz(row) == swz(lr)
  const bool a_on = wave * kARows < loc.rows;
  uint32_t a_off[kADma], b_off[kBDma];
#pragma unroll
  for (int i = 0; i < kBDma; ++i)
    b_off[i] = b_row_offset<MODE, kTN>(p, loc.ct, wave * kBRows + lr + kRowsPerDma * i) + chunk_b;
  const int a_dst = wave * kARows * kTK;  // element offset of this wave's first A row
  const int b_dst = kAStage + wave * kBRows * kTK;

  auto issue_a = [&](int kt, uint16_t* stage) {
    const uint32_t k = (uint32_t)kt * (kTK * 2);
    if (a_on) {
#pragma unroll
      for (int i = 0; i < kADma; ++i) dma16(p.a, a_off[i] + k, stage + a_dst + i * 512);
    }
  };
  auto issue_b = [&](int kt, uint16_t* stage) {
    const uint32_t k = (uint32_t)kt * (kTK * 2);
#pragma unroll
    for (int i = 0; i < kBDma; ++i) dma16(wbase, b_off[i] + k, stage + b_dst + i * 512);
  };
  auto issue = [&](int kt, uint16_t* stage) {
    issue_a(kt, stage);
    issue_b(kt, stage);
  };

  // fragment rows of this wave: A rows wm*64 + 16i + r16; B rows b_row(j) + r16 per column
  // tile j. GATE_UP: the first kNJ/2 tiles are gate columns wn*kWC/2 .., the rest the matching
  // up columns (B rows 128 + ...). Lane l reads chunk h*4 + l/16 of its row for the 32-column
  // half h of a step. One per-lane base per operand and half; tile offsets are constants.
  const int a_frag0 = (wm * 64 + r16) * kTK;
  const int b_frag0 = kAStage + ((MODE == kGateUp ? wn * (kWC / 2) : wn * kWC) + r16) * kTK;
  const int slot0 = (kq ^ swz(r16)) * 8, slot1 = ((4 + kq) ^ swz(r16)) * 8;
  auto b_row = [](int j) {
    return MODE == kGateUp ? (j < kNJ / 2 ? 0 : kTN / 2) + (j % (kNJ / 2)) * 16 : j * 16;
  };
  // the wave computes the first ni 16-row sub-tiles of its 64-row band that hold valid rows; a
  // wave whose 64 rows are all past `rows` computes nothing (it still loads and syncs)
  const int ni = min(max((loc.rows - wm * 64 + 15) >> 4, 0), 4);
  const bool m_on = ni > 0;

  floatx4 acc[4][kNJ];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < kNJ; ++j) acc[i][j] = floatx4{0.f, 0.f, 0.f, 0.f};

  // fragments of one 32-column half: [0..3] A rows, [4..] B columns
  constexpr int kNF = 4 + kNJ;
  // NI: sub-tiles of the band computed (A fragments read for those only)
  auto read_frags = [&](auto ni_tag, const uint16_t* stage, int slot, u32x4 (&f)[kNF]) {
    constexpr int NI = decltype(ni_tag)::value;
    const uint16_t* sA = stage + a_frag0 + slot;
    const uint16_t* sB = stage + b_frag0 + slot;
#pragma unroll
    for (int i = 0; i < NI; ++i) f[i] = *reinterpret_cast<const u32x4*>(sA + i * 16 * kTK);
#pragma unroll
    for (int j = 0; j < kNJ; ++j) f[4 + j] = *reinterpret_cast<const u32x4*>(sB + b_row(j) * kTK);
  };
  auto mfmas = [&](auto ni_tag, const u32x4 (&f)[kNF]) {  // transposed tiles (B first), see store_block
    constexpr int NI = decltype(ni_tag)::value;
#pragma unroll
    for (int i = 0; i < NI; ++i)
#pragma unroll
      for (int j = 0; j < kNJ; ++j)
        acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
            __builtin_bit_cast(bf16x8, f[4 + j]), __builtin_bit_cast(bf16x8, f[i]), acc[i][j],
            0, 0, 0);
  };
  // one LDS read between every two MFMAs (the reads feed the other half's MFMAs); the whole
  // band only (partial bands leave the order to the compiler)
  auto interleave = [&](auto ni_tag) {
    if constexpr (decltype(ni_tag)::value == 4) {
#pragma unroll
      for (int i = 0; i < kNF; ++i) {
        __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
        __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);
      }
    }
  };

  // Step kt (64 columns) uses stage kt % 2 and is computed in two halves: the MFMAs of half 0
  // run while half 1's fragments are read; then wait for step kt + 1's stage and barrier (every
  // wave has read all of step kt, so its stage is free), issue step kt + 2 into it, and run the
  // MFMAs of half 1 while half 0 of step kt + 1 is read.
  const int nk = K / kTK;
  auto stage_of = [&](int kt) { return smem + (kt & 1) * kStage; };
  auto loop = [&](auto ni_tag) {
    constexpr bool kMfma = decltype(ni_tag)::value > 0;
    u32x4 fa[kNF], fb[kNF];
    // the weight rows of steps 0 and 1 go first: the A rows may wait for their row indices
    // (GATE_UP gathers them). Step 0 in, step 1's A loads (or, for a wave without A rows, its
    // B loads) may still fly: 4 either way.
    issue_b(0, smem);
    if (nk > 1) issue_b(1, smem + kStage);
#pragma unroll
    for (int i = 0; i < kADma; ++i)
      a_off[i] = a_row_offset<MODE>(p, loc, min(wave * kARows + lr + kRowsPerDma * i, loc.rows - 1)) +
                 chunk_b;
    issue_a(0, smem);
    if (nk > 1) {
      issue_a(1, smem + kStage);
      SYM_TILE_SYNC(4);
    } else {
      SYM_TILE_SYNC(0);
    }
    if constexpr (kMfma) read_frags(ni_tag, smem, slot0, fa);
    for (int kt = 0; kt < nk - 1; ++kt) {
      if constexpr (kMfma) {
        read_frags(ni_tag, stage_of(kt), slot1, fb);
        mfmas(ni_tag, fa);
        interleave(ni_tag);
      }
      SYM_TILE_SYNC(0);
      if (kt + 2 < nk) issue(kt + 2, smem + (kt & 1) * kStage);
      if constexpr (kMfma) {
        read_frags(ni_tag, stage_of(kt + 1), slot0, fa);
        mfmas(ni_tag, fb);
        interleave(ni_tag);
      }
    }
    if constexpr (kMfma) {  // the last step
      read_frags(ni_tag, stage_of(nk - 1), slot1, fb);
      mfmas(ni_tag, fa);
      mfmas(ni_tag, fb);
    }
  };
  switch (ni) {
    case 4: loop(std::integral_constant<int, 4>{}); break;
    case 3: loop(std::integral_constant<int, 3>{}); break;
    case 2: loop(std::integral_constant<int, 2>{}); break;
    case 1: loop(std::integral_constant<int, 1>{}); break;
    default: loop(std::integral_constant<int, 0>{}); break;
  }
  hook();
  const int col0 = MODE == kGateUp ? loc.ct * (kTN / 2) + wn * (kWC / 2) : loc.ct * kTN + wn * kWC;
  if (MODE == kGateUp || p.out_f32 == nullptr) {
    // bf16 out, through the stages: every wave has read its last fragments (and thread 0 has
    // written what the hook writes) before any wave overwrites them; no vmcnt wait, so a vector
    // atomic of the hook still flies
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
    constexpr int kBlockElems = 64 * (MODE == kGateUp ? kWC / 2 : kWC);
    store_block_lds<MODE, kNJ>(p, acc, loc, wm * 64, col0, lane, smem + wave * kBlockElems);
  } else if (m_on) {
    store_block<MODE, kNJ>(p, acc, loc, wm * 64, col0, lane);
  }
}

// ================================================================================================
// Thin tiles: a 256-column tile of at most 64 valid rows (the persistent grouped kernels' tiles
// of small experts under skewed routing). big_tile streams the whole weight tile for them but
// computes one band of four, and each K-step waits a memory round trip with one step of
// lookahead: per-tile timestamps put such tiles at 80% (gate/up) and 69% (down) of a whole
// tile's time. Their A part is a quarter (64 rows), so three stages of 64 + 256 rows (40 KB)
// fit in the 128 KB that big_tile's two stages use: two steps of lookahead. The 8 waves share
// the DMA (1 A instruction and 4 B instructions each per step); waves 0 and 1 compute the 64 x
// 128 blocks of the band, as in big_tile.
// ================================================================================================
namespace thin {
constexpr int kTM = 64;
constexpr int kAStage = kTM * big::kTK;             // bf16 elements (8 KB)
constexpr int kStage = kAStage + big::kBStage;      // 40 KB
constexpr int kStages = 3;
static_assert(kStages * kStage <= 2 * big::kStage, "within big_tile's LDS");
}  // namespace thin

template <int MODE, typename Hook>
__device__ __forceinline__ void thin_tile(TileArgs p, const TileLoc& loc, uint16_t* smem,
                                          Hook hook) {
  using namespace big;
  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  // the lane index through an opaque copy: the per-lane values below are then computed here, not
  // hoisted out of the persistent kernel's tile loop (where big_tile's would be held beside them)
  int lane = tid & 63;
  asm volatile("" : "+v"(lane));
  const int wn = wave % kWavesN;
  const int r16 = lane & 15, kq = lane >> 4;
  const uint16_t* wbase = tile_weights<MODE>(p, loc);

  // DMA: wave w fills A rows 8w .. 8w + 7 (while the tile has rows there) and B rows 32w ..
  // 32w + 31 of each stage, lane l taking row + l / 8, chunk slot (l % 8) ^ swz(row)
  const int lr = lane >> 3;
  const uint32_t chunk_b = ((lane & 7) ^ swz(lr)) * 16;
  const bool a_on = wave * kRowsPerDma < loc.rows;
  uint32_t b_off[kBDma];
#pragma unroll
  for (int i = 0; i < kBDma; ++i)
    b_off[i] = b_row_offset<MODE, kTN>(p, loc.ct, wave * kBRows + lr + kRowsPerDma * i) + chunk_b;
  const int a_dst = wave * kRowsPerDma * kTK;
  const int b_dst = thin::kAStage + wave * kBRows * kTK;
  auto stage_of = [&](int kt) { return smem + (kt % thin::kStages) * thin::kStage; };
  uint32_t a_off = 0;
  auto issue_a = [&](int kt) {
    if (a_on) dma16(p.a, a_off + (uint32_t)kt * (kTK * 2), stage_of(kt) + a_dst);
  };
  auto issue_b = [&](int kt) {
    const uint32_t k = (uint32_t)kt * (kTK * 2);
#pragma unroll
    for (int i = 0; i < kBDma; ++i) dma16(wbase, b_off[i] + k, stage_of(kt) + b_dst + i * 512);
  };
  const int nk = p.K / kTK;
  // wait for step kt, leaving what was issued after it in flight: at kt = 0 (issued B0, B1,
  // A0, A1) step 1's A instruction, or for a wave without A rows step 1's 4 B instructions;
  // later, step kt + 1's 5 (or 4) instructions, issued after all of step kt
  auto sync_step = [&](int kt) {
    if (kt + 1 >= nk) {
      SYM_TILE_SYNC(0);
    } else if (kt == 0) {
      if (a_on) SYM_TILE_SYNC(1);
      else SYM_TILE_SYNC(4);
    } else if (a_on) {
      SYM_TILE_SYNC(5);
    } else {
      SYM_TILE_SYNC(4);
    }
  };

  // waves 0 and 1 compute: A rows 16 i + r16 of the band, B columns as big_tile's band 0
  const bool m_on = wave < kWavesN;
  const int ni = m_on ? min((loc.rows + 15) >> 4, 4) : 0;
  const int a_frag0 = r16 * kTK;
  const int b_frag0 = thin::kAStage + ((MODE == kGateUp ? wn * (kWC / 2) : wn * kWC) + r16) * kTK;
  const int slot0 = (kq ^ swz(r16)) * 8, slot1 = ((4 + kq) ^ swz(r16)) * 8;
  auto b_row = [](int j) {
    return MODE == kGateUp ? (j < kNJ / 2 ? 0 : kTN / 2) + (j % (kNJ / 2)) * 16 : j * 16;
  };
  floatx4 acc[4][kNJ];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < kNJ; ++j) acc[i][j] = floatx4{0.f, 0.f, 0.f, 0.f};
  constexpr int kNF = 4 + kNJ;
  auto read_frags = [&](auto ni_tag, const uint16_t* stage, int slot, u32x4 (&f)[kNF]) {
    constexpr int NI = decltype(ni_tag)::value;
#pragma unroll
    for (int i = 0; i < NI; ++i)
      f[i] = *reinterpret_cast<const u32x4*>(stage + a_frag0 + slot + i * 16 * kTK);
#pragma unroll
    for (int j = 0; j < kNJ; ++j)
      f[4 + j] = *reinterpret_cast<const u32x4*>(stage + b_frag0 + slot + b_row(j) * kTK);
  };
  auto mfmas = [&](auto ni_tag, const u32x4 (&f)[kNF]) {
    constexpr int NI = decltype(ni_tag)::value;
#pragma unroll
    for (int i = 0; i < NI; ++i)
#pragma unroll
      for (int j = 0; j < kNJ; ++j)
        acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
            __builtin_bit_cast(bf16x8, f[4 + j]), __builtin_bit_cast(bf16x8, f[i]), acc[i][j],
            0, 0, 0);
  };
  // Step kt uses stage kt % 3. Iteration kt waits for step kt (step kt + 1 may fly), and the
  // barrier after that wait also means every wave has finished reading step kt - 1, whose
  // stage then receives step kt + 2.
  auto loop = [&](auto ni_tag) {
    constexpr bool kMfma = decltype(ni_tag)::value > 0;
    u32x4 fa[kNF], fb[kNF];
    issue_b(0);
    if (nk > 1) issue_b(1);
    a_off = a_row_offset<MODE>(p, loc, min(wave * kRowsPerDma + lr, loc.rows - 1)) + chunk_b;
    issue_a(0);
    if (nk > 1) issue_a(1);
    for (int kt = 0; kt < nk; ++kt) {
      sync_step(kt);
      if (kt + 2 < nk) {
        issue_a(kt + 2);
        issue_b(kt + 2);
      }
      if constexpr (kMfma) {
        read_frags(ni_tag, stage_of(kt), slot0, fa);
        read_frags(ni_tag, stage_of(kt), slot1, fb);
        mfmas(ni_tag, fa);
        mfmas(ni_tag, fb);
      }
    }
  };
  switch (ni) {
    case 4: loop(std::integral_constant<int, 4>{}); break;
    case 3: loop(std::integral_constant<int, 3>{}); break;
    case 2: loop(std::integral_constant<int, 2>{}); break;
    case 1: loop(std::integral_constant<int, 1>{}); break;
    default: loop(std::integral_constant<int, 0>{}); break;
  }
  hook();
  const int col0 = MODE == kGateUp ? loc.ct * (kTN / 2) + wn * (kWC / 2) : loc.ct * kTN + wn * kWC;
  constexpr int kCols = MODE == kGateUp ? kWC / 2 : kWC;
  if (MODE == kGateUp || p.out_f32 == nullptr) {
    // (as in big_tile: every wave is done with the stages before the epilogue reuses them)
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
    store_block_lds<MODE, kNJ>(p, acc, loc, m_on ? 0 : 64, col0, lane, smem + wave * 64 * kCols);
  } else if (m_on) {
    store_block<MODE, kNJ>(p, acc, loc, 0, col0, lane);
  }
}

template <int MODE>
__global__ __launch_bounds__(big::kThreads) __attribute__((amdgpu_waves_per_eu(2)))
void gemm_tile_kernel(TileArgs p) {
  using namespace big;
  __shared__ __align__(1024) uint16_t smem[2 * kStage];
  TileLoc loc;
  if (!locate_tile<MODE, kTM>(p, threadIdx.x & 63, loc)) return;
  big_tile<MODE>(p, loc, smem);
}

// Segment list of the grouped modes in LDS (at most kPersistSeg segments): the first row tile
// of every segment (segments past the list: the total), the estimated cost of the tiles before
// it (kTileCost), its row count, first row and expert.
constexpr int kPersistSeg = 512;
struct SegTable {
  int pre[kPersistSeg], cpre[kPersistSeg], cnt[kPersistSeg], off[kPersistSeg];
  uint16_t exp[kPersistSeg];
  int total, ctotal;
};

// Estimated cost of a tile: 16 for a 256-row tile of more than thin::kTM rows, less for a thin
// tile (per-tile timestamps at the prefill workload: thin tiles took 0.56 of a whole tile's time
// in gate/up, 0.54 in down, and tiles of 65-256 rows about the same as whole ones). The thin
// costs were then tuned on the kernel time at that workload: gate/up with 11 took 411-412
// against 416-418 us with 9 (8: 422-423, 10: 416); down is fastest with 9 (282 against 283-287
// us with 8, 10 or 11).
constexpr int kTileCost = 16, kThinCostGateUp = 11, kThinCostDown = 9;
template <int MODE>
__device__ __forceinline__ int row_tile_cost(int cnt, int rt, int tm) {
  return cnt - rt * tm <= thin::kTM ? (MODE == kGateUp ? kThinCostGateUp : kThinCostDown)
                                    : kTileCost;
}

// Wave 0 reads the segment list (all loads in flight together with n_segments; lane l owns
// segments 8l .. 8l+7) and scans the row-tile counts of tiles of TM rows into the table.
template <int TM, int MODE>
__device__ __forceinline__ void load_seg_table(const TileArgs& p, SegTable& t, int nx) {
  const int lane = threadIdx.x & 63;
  if (threadIdx.x >= 64) return;
  int c[8], o[8], e[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int sg = lane * 8 + i;
    const bool in = sg < p.max_segments;
    c[i] = in ? p.seg_count[sg] : 0;
    o[i] = in ? p.seg_offset[sg] : 0;
    e[i] = in ? p.seg_expert[sg] : 0;
  }
  const int nseg = p.n_segments[0];
  int pre[8], cpre[8], run = 0, crun = 0;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    pre[i] = run;
    cpre[i] = crun;
    const int nt = lane * 8 + i < nseg ? (c[i] + TM - 1) / TM : 0;
    run += nt;
    // (nt - 1) row tiles of TM rows, then the last one (thin or not)
    crun += nt ? nx * ((nt - 1) * kTileCost + row_tile_cost<MODE>(c[i], nt - 1, TM)) : 0;
  }
  int x = run, cx = crun;  // inclusive scans of the lanes' row-tile counts and costs
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    const int y = __shfl_up(x, d), cy = __shfl_up(cx, d);
    if (lane >= d) {
      x += y;
      cx += cy;
    }
  }
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int sg = lane * 8 + i;
    t.pre[sg] = x - run + pre[i];
    t.cpre[sg] = cx - crun + cpre[i];
    t.cnt[sg] = c[i];
    t.off[sg] = o[i];
    t.exp[sg] = (uint16_t)e[i];
  }
  if (lane == 63) {
    t.total = x;
    t.ctotal = cx;
  }
}

// The first tile (index row tile * nx + column tile, in segment order) whose estimated cost
// before it is at least c: the boundary of an XCD's run of tiles of equal cost. Wave-uniform.
template <int TM, int MODE>
__device__ __forceinline__ int tile_at_cost(const SegTable& t, int c, int nx) {
  if (c <= 0) return 0;
  if (c >= t.ctotal) return t.total * nx;
  int lo = 0, hi = kPersistSeg - 1;  // the last segment whose cost prefix is <= c
  while (lo < hi) {
    const int md = (lo + hi + 1) >> 1;
    if (t.cpre[md] <= c) lo = md;
    else hi = md - 1;
  }
  const int cnt = t.cnt[lo], r = c - t.cpre[lo];
  const int rt = min(r / (nx * kTileCost), (cnt + TM - 1) / TM - 1);
  const int per = row_tile_cost<MODE>(cnt, rt, TM);
  const int ct = (r - rt * nx * kTileCost + per - 1) / per;  // (nx: the next row tile's first)
  return __builtin_amdgcn_readfirstlane((t.pre[lo] + rt) * nx + ct);
}

// Row tile g (of TM rows) of the table: the last segment whose first row tile is <= g (binary
// search, the same in every lane).
template <int TM>
__device__ __forceinline__ TileLoc seg_tile(const SegTable& t, int g, int ct) {
  int lo = 0, hi = kPersistSeg - 1;
  while (lo < hi) {
    const int md = (lo + hi + 1) >> 1;
    if (t.pre[md] <= g) lo = md;
    else hi = md - 1;
  }
  const int rt = g - t.pre[lo];
  TileLoc loc;
  loc.e = __builtin_amdgcn_readfirstlane((int)t.exp[lo]);
  loc.row0 = __builtin_amdgcn_readfirstlane(t.off[lo] + rt * TM);
  loc.rows = __builtin_amdgcn_readfirstlane(min(TM, t.cnt[lo] - rt * TM));
  loc.ct = __builtin_amdgcn_readfirstlane(ct);
  loc.z = 0;
  return loc;
}

// Tile tickets of gemm_tile_persistent: one counter per XCD in the caller's workspace
// (kTicketBytes), zero before the launch. The workgroup that draws an XCD's last ticket resets
// its counter, so a launch leaves the workspace zeroed for the next launch that uses it; launches
// that may overlap in time (different streams) take different workspaces.
constexpr size_t kTicketBytes = 8 * sizeof(int);

// Grouped modes of the 256 x 256 tiles on a persistent grid (one workgroup per CU, a multiple
// of 8): the segment list is read and scanned once per workgroup into LDS and each tile then
// finds its segment there. gemm_tile_kernel's per-tile lookup is a memory round trip behind
// the other workgroups' operand loads that no second workgroup on the CU hides; here only a
// workgroup's first tile pays it. Workgroups are dispatched to the XCDs round-robin by id, so
// XCD x = blockIdx.x % 8 owns a contiguous run of tiles (the column tiles of a row tile and the
// row tiles of an expert meet in its L2): the x-th of 8 runs of equal estimated cost
// (kTileCost), since with thin tiles, runs of equal tile count left the XCDs' ends 56 us
// (gate/up) and 34 us (down) apart under skewed routing. Its W = gridDim.x / 8
// workgroups take the run's first W tiles in order and then draw the rest from the XCD's
// ticket counter: tiles of a segment's last rows are shorter, and a static share would leave
// the workgroups that drew several whole tiles last. Thread 0 draws one tile ahead (the ticket
// for the tile after the current one is drawn at the current one's hook, or at the start), so
// the fetch-add has a whole tile to return. Tickets 0 .. run - 1 are drawn, one per tile of
// the run (a ticket past the run ends the drawing workgroup); whoever reads run - 1 is the
// last to touch the counter and resets it.
template <int MODE>
__global__ __launch_bounds__(big::kThreads) __attribute__((amdgpu_waves_per_eu(2)))
void gemm_tile_persistent(TileArgs p, int nx) {
  using namespace big;
  __shared__ __align__(1024) uint16_t smem[2 * kStage];
  __shared__ SegTable tab;
  __shared__ int s_next;
  load_seg_table<kTM, MODE>(p, tab, nx);
  __syncthreads();
  const int x = blockIdx.x & 7, wpx = gridDim.x >> 3;
  // this XCD's tiles: the x-th eighth of the estimated cost
  const long long ctot = tab.ctotal;
  const int run0 = tile_at_cost<kTM, MODE>(tab, (int)(ctot * x / 8), nx);
  const int run = tile_at_cost<kTM, MODE>(tab, (int)(ctot * (x + 1) / 8), nx) - run0;
  // a per-lane (to the compiler: divergent) address, so the fetch-add is issued as it stands
  // and its result is waited for only where it is used
  int zero = 0;
  asm volatile("" : "+v"(zero));
  int* ticket = p.tickets + x + zero;
  int i = blockIdx.x >> 3;  // index in the run
  int pend = 0;             // thread 0: the ticket drawn for the tile after the current one
  if (threadIdx.x == 0 && i < run)
    pend = __hip_atomic_fetch_add(ticket, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  while (i < run) {
    const int t = run0 + i;
    const int g = t / nx;
    const TileLoc loc = seg_tile<kTM>(tab, g, t - g * nx);
    // (every wave passed the barrier after the previous tile's epilogue, whose LDS reads of the
    // stages had completed: this tile's DMA may refill them)
    auto hook = [&]() {
      if (threadIdx.x == 0) {
        const int nxt = wpx + pend;
        if (pend == run - 1)
          __hip_atomic_store(ticket, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (nxt < run)
          pend = __hip_atomic_fetch_add(ticket, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        s_next = nxt;
      }
    };
    if (loc.rows <= thin::kTM) thin_tile<MODE>(p, loc, smem, hook);
    else big_tile<MODE>(p, loc, smem, hook);
    __syncthreads();
    i = __builtin_amdgcn_readfirstlane(s_next);
  }
}

// ================================================================================================
// 128 x 256 tiles (grouped down projection, K = I is short; router logits, N = E is narrow): 8
// waves of 64 x 64, two workgroups per CU (while one waits at a barrier or on its prologue, the other computes), 32-column steps
// through a 3-stage 72 KB LDS ring; a step's fragment reads are all issued before its MFMAs.
// ================================================================================================
namespace mid {
constexpr int kTM = 128, kTN = 256, kTK = 32;
constexpr int kWavesN = 4, kWaves = 8, kThreads = 512;
constexpr int kWC = kTN / kWavesN, kNJ = kWC / 16;  // 64 columns (4 MFMA tiles) per wave
constexpr int kAStage = kTM * kTK, kBStage = kTN * kTK, kStage = kAStage + kBStage;  // bf16
constexpr int kRowsPerDma = 16;  // one wave-wide LDS-DMA instruction: 16 rows x 64 bytes
constexpr int kARows = kTM / kWaves, kBRows = kTN / kWaves;
constexpr int kADma = kARows / kRowsPerDma, kBDma = kBRows / kRowsPerDma;  // 1 + 2
static_assert(kADma == 1 && kBDma == 2, "the wait counts");
// LDS slot of 16-byte chunk c (of 4) in row r: c ^ ((r / 2) % 4): the 16 rows of a fragment
// read (one chunk each, two rows per 128 bytes) fall in distinct banks.
__device__ __forceinline__ int swz(int r) { return (r >> 1) & 3; }
}  // namespace mid

template <int MODE>
__global__ __launch_bounds__(mid::kThreads) __attribute__((amdgpu_waves_per_eu(4)))
void gemm_tile128_kernel(TileArgs p) {
  using namespace mid;
  __shared__ __align__(1024) uint16_t smem[3 * kStage];

  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
  const int wm = wave / kWavesN, wn = wave % kWavesN;
  const int r16 = lane & 15, kq = lane >> 4;
  const int K = p.K;

  TileLoc loc;
  if (!locate_tile<MODE, kTM>(p, lane, loc)) return;
  const uint16_t* wbase = tile_weights<MODE>(p, loc);

  // LDS-DMA sources as in gemm_tile_kernel, 16 rows x 64 bytes per instruction (every wave
  // loads its rows: the wait counts are fixed)
  const int lr = lane >> 2;
  const uint32_t chunk_b = ((lane & 3) ^ swz(lr)) * 16;
  const uint32_t a_off = a_row_offset<MODE>(p, loc, min(wave * kARows + lr, loc.rows - 1)) + chunk_b;
  uint32_t b_off[kBDma];
#pragma unroll
  for (int i = 0; i < kBDma; ++i)
    b_off[i] = b_row_offset<MODE, kTN>(p, loc.ct, wave * kBRows + lr + kRowsPerDma * i) + chunk_b;
  const int a_dst = wave * kARows * kTK;
  const int b_dst = kAStage + wave * kBRows * kTK;
  auto issue = [&](int kt, uint16_t* stage) {
    const uint32_t k = (uint32_t)kt * (kTK * 2);
    dma16(p.a, a_off + k, stage + a_dst);
#pragma unroll
    for (int i = 0; i < kBDma; ++i) dma16(wbase, b_off[i] + k, stage + b_dst + i * 512);
  };

  const int a_frag0 = (wm * 64 + r16) * kTK + (kq ^ swz(r16)) * 8;
  const int b_frag0 = kAStage + ((MODE == kGateUp ? wn * (kWC / 2) : wn * kWC) + r16) * kTK +
                      (kq ^ swz(r16)) * 8;
  auto b_row = [](int j) {
    return MODE == kGateUp ? (j < kNJ / 2 ? 0 : kTN / 2) + (j % (kNJ / 2)) * 16 : j * 16;
  };

  floatx4 acc[4][kNJ];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < kNJ; ++j) acc[i][j] = floatx4{0.f, 0.f, 0.f, 0.f};

  // MFMAs of one step over the first NI 16-row sub-tiles of the wave's 64-row band
  auto compute = [&](auto ni_tag, const uint16_t* stage) {
    constexpr int NI = decltype(ni_tag)::value;
    u32x4 fa[NI], fb[kNJ];
#pragma unroll
    for (int i = 0; i < NI; ++i)
      fa[i] = *reinterpret_cast<const u32x4*>(stage + a_frag0 + i * 16 * kTK);
#pragma unroll
    for (int j = 0; j < kNJ; ++j)
      fb[j] = *reinterpret_cast<const u32x4*>(stage + b_frag0 + b_row(j) * kTK);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int i = 0; i < NI; ++i)
#pragma unroll
      for (int j = 0; j < kNJ; ++j)
        acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
            __builtin_bit_cast(bf16x8, fb[j]), __builtin_bit_cast(bf16x8, fa[i]), acc[i][j],
            0, 0, 0);
  };

  // Step k: wait for its stage (the DMA of step k + 1 may still be in flight), barrier (every
  // wave is also done with step k - 1's stage), issue step k + 2 into that stage, MFMAs. Step k
  // uses stage k % 3. In a segment's last tile a wave computes only the 16-row sub-tiles of its
  // 64-row band that hold valid rows (none when the band lies wholly past them) and keeps the
  // loads and barriers: the sub-tile count is a template parameter, so no K loop carries a
  // branch.
  const int nk = K / kTK;
  const int ni = min(max((loc.rows - wm * 64 + 15) >> 4, 0), 4);
  issue(0, smem);
  if (nk > 1) issue(1, smem + kStage);
  auto loop = [&](auto ni_tag) {
    int cur = 0;  // stage of step kt (element offset)
    for (int kt = 0; kt < nk; ++kt) {
      if (kt + 1 >= nk) SYM_TILE_SYNC(0);
      else SYM_TILE_SYNC(3);  // step kt + 1's three loads may still fly
      const int nxt = cur == 0 ? 2 * kStage : cur - kStage;  // stage of step kt + 2
      if (kt + 2 < nk) issue(kt + 2, smem + nxt);
      if constexpr (decltype(ni_tag)::value > 0) compute(ni_tag, smem + cur);
      cur = cur == 2 * kStage ? 0 : cur + kStage;
    }
  };
  switch (ni) {
    case 4: loop(std::integral_constant<int, 4>{}); break;
    case 3: loop(std::integral_constant<int, 3>{}); break;
    case 2: loop(std::integral_constant<int, 2>{}); break;
    case 1: loop(std::integral_constant<int, 1>{}); break;
    default: loop(std::integral_constant<int, 0>{}); break;
  }
  if (ni == 0) return;

  const int col0 = MODE == kGateUp ? loc.ct * (kTN / 2) + wn * (kWC / 2) : loc.ct * kTN + wn * kWC;
  store_block<MODE, kNJ>(p, acc, loc, wm * 64, col0, lane);
}

}  // namespace sym

using namespace sym;

// The kernel addresses A and one weight matrix with 32-bit byte offsets.
static bool fits_4g(long long rows, long long cols) { return rows * cols * 2 < (1ll << 32); }
// Operands move in 16-byte pieces (A, W, fp32 outputs and residuals) and 8-byte pieces (bf16
// outputs, bias).
static bool aligned(const void* ptr, uintptr_t n) { return ((uintptr_t)ptr & (n - 1)) == 0; }

// Row tiling of a dense GEMM on the 256 x 256 tiles (one workgroup per CU, dispatched in
// order). A tile of 128 valid rows computes its two 64-row bands with one wave per SIMD instead of
// two, in about 0.55 of a whole tile's time; when the whole tiles leave a last round mostly idle
// (or a single round uses few CUs), the rows past full_rt whole row tiles go in 128-row tiles.
// Estimated makespans in whole-tile times: the tail's tiles start on the CUs the last round of
// whole tiles leaves free and on every CU after it. tail_rows = 0 keeps the uniform tiling.
static void dense_tail_split(int M, int nx, int cus, int& full_rt, int& tail_rows) {
  constexpr double kHalf = 0.55;
  const int rt = (M + big::kTM - 1) / big::kTM;
  const int tiles = rt * nx;
  const double uniform = (double)((tiles + cus - 1) / cus);
  full_rt = 0;
  tail_rows = 0;
  double best = uniform;
  for (int rounds = 0; rounds * cus <= tiles; ++rounds) {
    const int f = std::min(rt, rounds * cus / nx);  // whole row tiles
    const int tail = M - f * big::kTM;
    if (tail <= 0) break;
    const int jobs = (tail + 127) / 128 * nx;
    const int a = f * nx, r1 = a / cus, busy = a - r1 * cus;  // CUs busy in the last round
    // tail tiles done by time t (in kHalf steps) from the start of that round
    int steps = 0;
    for (long long done = 0; done < jobs;) {
      ++steps;
      const double t = steps * kHalf;
      done = (long long)(cus - busy) * steps +
             (busy > 0 && t > 1.0 ? (long long)busy * (int)((t - 1.0) / kHalf + 1e-9) : 0);
    }
    const double est = r1 + std::max(steps * kHalf, busy > 0 ? 1.0 : 0.0);
    if (est < best - 1e-9) {
      best = est;
      full_rt = f;
      tail_rows = 128;
    }
  }
}

static int gemm_dense(const char* what, const void* a, const void* w, const void* bias,
                      const float* residual, const void* residual_bf16, int M, int N, int K,
                      void* out, int out_fp32, void* stream) {
  SYM_REQUIRE(M >= 0, SYM_ERR_INVALID, "%s: M=%d < 0", what, M);
  if (M == 0) return SYM_OK;
  SYM_REQUIRE(a && w && out, SYM_ERR_INVALID, "%s: null pointer argument", what);
  SYM_REQUIRE(N > 0 && N % 16 == 0, SYM_ERR_UNSUPPORTED,
              "%s: N=%d must be a positive multiple of 16", what, N);
  SYM_REQUIRE(K > 0 && K % big::kTK == 0, SYM_ERR_UNSUPPORTED,
              "%s: K=%d must be a positive multiple of %d", what, K, big::kTK);
  namespace C = big;
  SYM_REQUIRE((M + C::kTM - 1) / C::kTM <= 65535, SYM_ERR_UNSUPPORTED, "%s: M=%d too large",
              what, M);
  SYM_REQUIRE(fits_4g(M, K) && fits_4g(N, K), SYM_ERR_UNSUPPORTED,
              "%s: a [%d, %d] or w [%d, %d] is 4 GB or more", what, M, K, N, K);
  SYM_REQUIRE(aligned(a, 16) && aligned(w, 16) && aligned(out, 16) && aligned(residual, 16) &&
                  aligned(residual_bf16, 8) && aligned(bias, 8),
              SYM_ERR_INVALID, "%s: a, w, out and an fp32 residual must be 16-byte aligned, "
              "bias and a bf16 residual 8-byte aligned", what);
  TileArgs p{};
  p.a = (const uint16_t*)a;
  p.w = (const uint16_t*)w;
  p.bias = (const uint16_t*)bias;
  p.residual = residual;
  p.residual_bf16 = (const uint16_t*)residual_bf16;
  p.M = M;
  p.N = N;
  p.K = K;
  p.out_bf16 = out_fp32 ? nullptr : (uint16_t*)out;
  p.out_f32 = out_fp32 ? (float*)out : nullptr;
  const int nx = (N + C::kTN - 1) / C::kTN;
  int rt = (M + C::kTM - 1) / C::kTM;
  dense_tail_split(M, nx, sym_host::cu_count(), p.full_rt, p.tail_rows);
  if (p.tail_rows > 0) rt = p.full_rt + (M - p.full_rt * C::kTM + p.tail_rows - 1) / p.tail_rows;
  (void)hipGetLastError();
  hipLaunchKernelGGL((gemm_tile_kernel<kDense>), dim3(nx, rt), dim3(C::kThreads), 0,
                     (hipStream_t)stream, p);
  return sym_host::check_launch("gemm_tile_kernel");
}

extern "C" int sym_gemm_bf16(const void* a, const void* w, const void* bias, const float* residual,
                             int M, int N, int K, void* out, int out_fp32, void* stream) {
  return gemm_dense("gemm_bf16", a, w, bias, residual, nullptr, M, N, K, out, out_fp32, stream);
}

extern "C" int sym_gemm_bf16_res_bf16(const void* a, const void* w, const void* bias,
                                      const void* residual, int M, int N, int K, float* out,
                                      void* stream) {
  SYM_REQUIRE(M <= 0 || residual, SYM_ERR_INVALID, "gemm_bf16_res_bf16: null residual");
  return gemm_dense("gemm_bf16_res_bf16", a, w, bias, nullptr, residual, M, N, K, out, 1,
                    stream);
}

// Router logits for prefill-size T on MFMA. The fp32 gate weight w [E, H] comes as three bf16
// planes [3, E, H] with w = hi + mid + lo exactly (24 mantissa bits = 3 x 8); x is bf16, so each
// product x * plane is exact in fp32 and parts[z] = x . plane_z^T (fp32 accumulation) are the
// three partial logits, summed (hi + mid) + lo by sym_moe_route_permute (n_logit_parts = 3).
extern "C" int sym_moe_router_logits_split(const void* x, const void* w_planes, int T, int H,
                                           int E, float* parts, void* stream) {
  SYM_REQUIRE(T >= 0, SYM_ERR_INVALID, "moe_router_logits_split: T=%d < 0", T);
  if (T == 0) return SYM_OK;
  SYM_REQUIRE(x && w_planes && parts, SYM_ERR_INVALID,
              "moe_router_logits_split: null pointer argument");
  SYM_REQUIRE(E > 0 && E % 16 == 0, SYM_ERR_UNSUPPORTED,
              "moe_router_logits_split: E=%d must be a positive multiple of 16", E);
  SYM_REQUIRE(H > 0 && H % big::kTK == 0, SYM_ERR_UNSUPPORTED,
              "moe_router_logits_split: H=%d must be a positive multiple of %d", H, big::kTK);
  // 128 x 256 tiles, two workgroups per CU: with N = E = 256 columns and three planes, 256-row
  // tiles would leave more than half of the CUs idle at T ~ 10k
  namespace C = mid;
  SYM_REQUIRE((T + C::kTM - 1) / C::kTM <= 65535, SYM_ERR_UNSUPPORTED,
              "moe_router_logits_split: T=%d too large", T);
  SYM_REQUIRE(fits_4g(T, H) && fits_4g(E, H), SYM_ERR_UNSUPPORTED,
              "moe_router_logits_split: x [%d, %d] is 4 GB or more", T, H);
  SYM_REQUIRE(aligned(x, 16) && aligned(w_planes, 16) && aligned(parts, 16), SYM_ERR_INVALID,
              "moe_router_logits_split: x, w_planes and parts must be 16-byte aligned");
  TileArgs p{};
  p.a = (const uint16_t*)x;
  p.w = (const uint16_t*)w_planes;
  p.M = T;
  p.N = E;
  p.K = H;
  p.out_f32 = parts;
  p.w_zstride = (long long)E * H;
  p.out_zstride = (long long)T * E;
  (void)hipGetLastError();
  hipLaunchKernelGGL((gemm_tile128_kernel<kDense>),
                     dim3((E + C::kTN - 1) / C::kTN, (T + C::kTM - 1) / C::kTM, 3), dim3(C::kThreads),
                     0, (hipStream_t)stream, p);
  return sym_host::check_launch("gemm_tile128_kernel");
}

static int check_grouped(const char* what, int T, int H, int I, int rows, int max_segments) {
  SYM_REQUIRE(fits_4g(T, H) && fits_4g(rows, I) && fits_4g(2 * (long long)I, H), SYM_ERR_UNSUPPORTED,
              "%s: an operand (x [%d, %d], h [%d, %d] or one expert's weights) is 4 GB or more",
              what, T, H, rows, I);
  SYM_REQUIRE(T >= 0 && rows >= 0, SYM_ERR_INVALID, "%s: T=%d rows=%d", what, T, rows);
  // gate/up steps through H 64 columns at a time, down through I 32 at a time; h rows are
  // written in 128-byte pieces
  SYM_REQUIRE(H > 0 && H % big::kTK == 0, SYM_ERR_UNSUPPORTED, "%s: H=%d must be a multiple of %d",
              what, H, big::kTK);
  SYM_REQUIRE(I > 0 && I % big::kTK == 0, SYM_ERR_UNSUPPORTED, "%s: I=%d must be a multiple of %d",
              what, I, big::kTK);
  SYM_REQUIRE(max_segments >= 1 && max_segments <= kMaxGemmSegments, SYM_ERR_INVALID,
              "%s: max_segments=%d out of range", what, max_segments);
  SYM_REQUIRE((long long)rows / mid::kTM + max_segments <= 65535, SYM_ERR_UNSUPPORTED,
              "%s: %d rows too many", what, rows);
  return SYM_OK;
}

// The tile-ticket workspace of the grouped tiled GEMMs (zeroed once by the caller, left zeroed
// by every launch).
static int check_tickets(const char* what, const void* workspace, size_t workspace_bytes) {
  SYM_REQUIRE(workspace_bytes >= kTicketBytes, SYM_ERR_WORKSPACE,
              "%s: workspace of %zu bytes, %zu needed", what, workspace_bytes, kTicketBytes);
  SYM_REQUIRE(workspace && aligned(workspace, 4), SYM_ERR_INVALID,
              "%s: workspace must be a non-null 4-byte aligned device pointer", what);
  return SYM_OK;
}

extern "C" size_t sym_moe_tiled_workspace_bytes(void) { return kTicketBytes; }

extern "C" int sym_moe_gate_up_tiled(const void* x, int T, int H, int I, int rows,
                                     const int32_t* sorted_tokens, const int32_t* seg_expert,
                                     const int32_t* seg_offset, const int32_t* seg_count,
                                     const int32_t* n_segments, int max_segments,
                                     const void* w_gate_up, void* h, void* workspace,
                                     size_t workspace_bytes, void* stream) {
  int rc = check_grouped("moe_gate_up_tiled", T, H, I, rows, max_segments);
  if (!rc) rc = check_tickets("moe_gate_up_tiled", workspace, workspace_bytes);
  if (rc || rows == 0 || T == 0) return rc;
  SYM_REQUIRE(x && sorted_tokens && seg_expert && seg_offset && seg_count && n_segments &&
                  w_gate_up && h,
              SYM_ERR_INVALID, "moe_gate_up_tiled: null pointer argument");
  SYM_REQUIRE(aligned(x, 16) && aligned(w_gate_up, 16) && aligned(h, 16), SYM_ERR_INVALID,
              "moe_gate_up_tiled: x, w_gate_up and h must be 16-byte aligned");
  TileArgs p{};
  p.a = (const uint16_t*)x;
  p.w = (const uint16_t*)w_gate_up;
  p.sorted_tokens = sorted_tokens;
  p.seg_expert = seg_expert;
  p.seg_offset = seg_offset;
  p.seg_count = seg_count;
  p.n_segments = n_segments;
  p.max_segments = max_segments;
  p.M = rows;
  p.N = I;
  p.K = H;
  p.out_bf16 = (uint16_t*)h;
  p.tickets = (int*)workspace;
  (void)hipGetLastError();
  namespace C = big;
  const int nx = (I + C::kTN / 2 - 1) / (C::kTN / 2);
  if (max_segments <= kPersistSeg) {
    // one workgroup per CU, a multiple of 8 (one run of tiles per XCD)
    const int grid = std::max(8, sym_host::cu_count() / 8 * 8);
    hipLaunchKernelGGL((gemm_tile_persistent<kGateUp>), dim3(grid), dim3(C::kThreads), 0,
                       (hipStream_t)stream, p, nx);
    return sym_host::check_launch("gemm_tile_persistent");
  }
  hipLaunchKernelGGL((gemm_tile_kernel<kGateUp>), dim3(nx, rows / C::kTM + max_segments),
                     dim3(C::kThreads), 0, (hipStream_t)stream, p);
  return sym_host::check_launch("gemm_tile_kernel");
}

extern "C" int sym_moe_down_tiled(const void* h, int T, int H, int I, int rows,
                                  const int32_t* seg_expert, const int32_t* seg_offset,
                                  const int32_t* seg_count, const int32_t* n_segments,
                                  int max_segments, const void* w_down, void* y, int y_bf16,
                                  void* workspace, size_t workspace_bytes, void* stream) {
  int rc = check_grouped("moe_down_tiled", T, H, I, rows, max_segments);
  if (!rc) rc = check_tickets("moe_down_tiled", workspace, workspace_bytes);
  if (rc || rows == 0 || T == 0) return rc;
  SYM_REQUIRE(h && seg_expert && seg_offset && seg_count && n_segments && w_down && y,
              SYM_ERR_INVALID, "moe_down_tiled: null pointer argument");
  SYM_REQUIRE(aligned(h, 16) && aligned(w_down, 16) && aligned(y, 16), SYM_ERR_INVALID,
              "moe_down_tiled: h, w_down and y must be 16-byte aligned");
  TileArgs p{};
  p.a = (const uint16_t*)h;
  p.w = (const uint16_t*)w_down;
  p.seg_expert = seg_expert;
  p.seg_offset = seg_offset;
  p.seg_count = seg_count;
  p.n_segments = n_segments;
  p.max_segments = max_segments;
  p.M = rows;
  p.N = H;
  p.K = I;
  if (y_bf16) p.out_bf16 = (uint16_t*)y;
  else p.out_f32 = (float*)y;
  p.tickets = (int*)workspace;
  (void)hipGetLastError();
  if (max_segments <= kPersistSeg) {
    const int grid = std::max(8, sym_host::cu_count() / 8 * 8);
    hipLaunchKernelGGL((gemm_tile_persistent<kDown>), dim3(grid), dim3(big::kThreads), 0,
                       (hipStream_t)stream, p, (H + big::kTN - 1) / big::kTN);
    return sym_host::check_launch("gemm_tile_persistent");
  }
  namespace C = mid;
  hipLaunchKernelGGL((gemm_tile128_kernel<kDown>),
                     dim3((H + C::kTN - 1) / C::kTN, rows / C::kTM + max_segments),
                     dim3(C::kThreads), 0, (hipStream_t)stream, p);
  return sym_host::check_launch("gemm_tile128_kernel");
}
