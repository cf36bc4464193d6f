// Grouped SwiGLU expert GEMMs over ragged per-expert row counts, and the weighted combine.
//
// Reference semantics: TTNNExperts.forward (ttnn_moe.py:1159-1343): per expert
// h = silu(x W1^T) * (x W3^T), y = h W2^T, then combine sum_k w_k y_k (ttnn_moe.py:1307-1335);
// shared expert TTNNGlm4MoeMLP (ttnn_moe.py:656-675) added at ttnn_moe.py:1487-1490.
//
// Design for gfx950 at decode sizes (about 1-6 rows per routed expert, T rows for the shared
// expert): the kernels are weight-streaming. A wave owns 16 output columns of one segment
// (expert) and a range of the reduction dimension, so every weight byte is read from HBM
// exactly once per step, and it issues its loads in batches so that enough bytes are in flight
// to cover HBM latency even in the last partial round of workgroups. The 16 weight rows form the B operand of v_mfma_f32_16x16x32_bf16:
// lane l streams 32 contiguous bytes of row (l % 16) per 64-wide K step (4 lanes cover 128
// contiguous bytes of a row), and the rows of the segment (tokens, gathered through
// sorted_tokens) form the A operand; rows past the segment repeat its last row and their outputs are dropped. Both operands use the
// same lane -> K mapping, so the K order inside a step is free to follow memory order. Up to
// MT row tiles (16 rows each) are accumulated per pass over the weights.
// Segments live on the device: a grid of a fixed size per kernel and batch (24 to 56 workgroups
// per CU, the constants below) strides over the live tiles (*n_segments of them times the tiles
// per segment), so no host synchronization is needed.
#include "common.h"

namespace sym {

constexpr int kGemmThreads = 256;  // 4 waves; each wave owns 16 output columns
// 16-column tiles per wave of the down projection: one tile needs 90 + 4 registers (5 waves per
// SIMD), two need 124 + 8 (3 per SIMD); 62.1 against 65.3 us at batch 32.
constexpr int kDownNT = 1;
constexpr int kColsPerWG = 4 * 16 * kDownNT;  // down projection: 4 waves x 16 * kDownNT columns
constexpr int kColsPerWG8 = 128;              // fp8 down projection: 4 waves x 32 columns

__device__ __forceinline__ uint4 ld16(const uint16_t* p) {
  return *reinterpret_cast<const uint4*>(p);
}

// Segment of a tile of the grid-stride loops below.
struct SegInfo {
  int e, row0, cnt;
};
// The grid-stride loops below walk the live tiles from the last one down: the last segment is the
// shared expert, whose T rows take the most passes, so its tiles start first instead of forming
// the kernel's tail. Metadata is read with scalar loads written out in asm (the compiler would
// otherwise wait between dependent loads it could issue together, or sink a prefetch to its
// use); their destinations are early-clobber, so that no load overwrites the address of a later
// one before it issues. The live segment count comes first, then the segments of a workgroup's
// first two tiles in one round trip; a third or later tile (only at large batches) reads its
// segment when it starts.
__device__ __forceinline__ int load_segment_count(const int32_t* n_segments) {
  int nseg;
  asm volatile("s_load_dword %0, %1, 0x0\n\ts_waitcnt lgkmcnt(0)"
               : "=&s"(nseg)
               : "s"(n_segments)
               : "memory");
  return nseg;
}
__device__ __forceinline__ void load_two_segments(const int32_t* seg_expert,
                                                  const int32_t* seg_offset,
                                                  const int32_t* seg_count, int seg0, int seg1,
                                                  SegInfo& m0, SegInfo& m1) {
  asm volatile(
      "s_load_dword %0, %6, 0x0\n\t"
      "s_load_dword %1, %7, 0x0\n\t"
      "s_load_dword %2, %8, 0x0\n\t"
      "s_load_dword %3, %9, 0x0\n\t"
      "s_load_dword %4, %10, 0x0\n\t"
      "s_load_dword %5, %11, 0x0\n\t"
      "s_waitcnt lgkmcnt(0)"
      : "=&s"(m0.e), "=&s"(m0.row0), "=&s"(m0.cnt), "=&s"(m1.e), "=&s"(m1.row0), "=&s"(m1.cnt)
      : "s"(seg_expert + seg0), "s"(seg_offset + seg0), "s"(seg_count + seg0),
        "s"(seg_expert + seg1), "s"(seg_offset + seg1), "s"(seg_count + seg1)
      : "memory");
}
__device__ __forceinline__ SegInfo load_segment(const int32_t* seg_expert,
                                                const int32_t* seg_offset,
                                                const int32_t* seg_count, int seg) {
  SegInfo m;
  asm volatile(
      "s_load_dword %0, %3, 0x0\n\t"
      "s_load_dword %1, %4, 0x0\n\t"
      "s_load_dword %2, %5, 0x0\n\t"
      "s_waitcnt lgkmcnt(0)"
      : "=&s"(m.e), "=&s"(m.row0), "=&s"(m.cnt)
      : "s"(seg_expert + seg), "s"(seg_offset + seg), "s"(seg_count + seg)
      : "memory");
  return m;
}
// Declares ntiles, m0 and m1 in a kernel with the arguments seg_expert, seg_offset, seg_count,
// n_segments and tiles_per_seg: the workgroup's k-th tile is ntiles - 1 - (blockIdx.x + k *
// gridDim.x); m0 / m1 hold the segments of its first two (an index clamped at 0 for a tile past
// the live ones: read, not used).
#define SYM_FIRST_SEGMENTS(ntiles, m0, m1)                                                     \
  const int ntiles = load_segment_count(n_segments) * tiles_per_seg;                         \
  SegInfo m0, m1;                                                                            \
  load_two_segments(                                                                         \
      seg_expert, seg_offset, seg_count,                                                     \
      __builtin_amdgcn_readfirstlane(max(ntiles - 1 - (int)blockIdx.x, 0) / tiles_per_seg),  \
      __builtin_amdgcn_readfirstlane(max(ntiles - 1 - (int)(blockIdx.x + gridDim.x), 0) /   \
                                     tiles_per_seg),                                         \
      m0, m1)
// The segment of the it-th tile of this workgroup, tile wt.
#define SYM_TILE_SEGMENT(it, wt, m0, m1)                       \
  ((it) == 0   ? (m0)                                          \
   : (it) == 1 ? (m1)                                          \
               : load_segment(seg_expert, seg_offset, seg_count, \
                              __builtin_amdgcn_readfirstlane((wt) / tiles_per_seg)))

// Lane -> k mapping inside a 64-wide K step (the same for both MFMA operands, so any mapping
// is exact): lane group kq = l / 16 takes k = kKLane * kq + 0..7 for the first MFMA and the same
// + kKHalf for the second.
constexpr int kKLane = 16, kKHalf = 8;   // a lane's two loads are 32 contiguous bytes

// One pass of gate/up over 16 rows of a segment, for this wave's K-step range [s_beg, s_end)
// (a multiple of U steps). Per batch of U K-steps: the weight loads, then the activation loads,
// then the MFMAs, kept in that order by scheduling barriers. The 16 token indices of the pass
// are read with scalar loads after the first weight batch is issued: waiting for them (lgkmcnt)
// does not wait for the weights in flight (vmcnt).
template <int U>
__device__ __forceinline__ void gate_up_pass(const uint16_t* __restrict__ x, int H,
                                             const int32_t* __restrict__ tok_rows, int rows,
                                             const uint16_t* __restrict__ wg,
                                             const uint16_t* __restrict__ wu, int s_beg, int s_end,
                                             int r16, int kq, floatx4& accg, floatx4& accu) {
  accg = floatx4{0.f, 0.f, 0.f, 0.f};
  accu = floatx4{0.f, 0.f, 0.f, 0.f};
  // the lane's token (rows past the pass read its last row, in bounds; their outputs are
  // dropped), loaded before the weights: waiting for it does not wait for them
  const int tok = tok_rows[min(r16, rows - 1)];
  __builtin_amdgcn_sched_barrier(0);
  const uint16_t* xr = x + kq * kKLane;
  for (int st = s_beg; st < s_end; st += U) {
    uint4 bg[U][2], bu[U][2], a[U][2];
#pragma unroll
    for (int s = 0; s < U; ++s) {
      const int k = (st + s) << 6;
      bg[s][0] = ld16(wg + k);
      bg[s][1] = ld16(wg + k + kKHalf);
      bu[s][0] = ld16(wu + k);
      bu[s][1] = ld16(wu + k + kKHalf);
    }
    __builtin_amdgcn_sched_barrier(0);
    if (st == s_beg) xr += (size_t)tok * H;
#pragma unroll
    for (int s = 0; s < U; ++s) {
      const int k = (st + s) << 6;
      a[s][0] = ld16(xr + k);
      a[s][1] = ld16(xr + k + kKHalf);
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int s = 0; s < U; ++s) {
      accg = mfma16x16x32(a[s][0], bg[s][0], accg);
      accg = mfma16x16x32(a[s][1], bg[s][1], accg);
      accu = mfma16x16x32(a[s][0], bu[s][0], accu);
      accu = mfma16x16x32(a[s][1], bu[s][1], accu);
    }
  }
}

// Partial accumulators of the 4 waves -> LDS -> sum, SwiGLU, bf16 h rows of the pass.
template <int MT>
__device__ __forceinline__ void gate_up_epilogue(float (*s_red)[MT][2][4][64],
                                                 const floatx4 (&accg)[MT],
                                                 const floatx4 (&accu)[MT], int wave, int lane,
                                                 int rows, size_t h_row0, int I, int col0,
                                                 uint16_t* __restrict__ h) {
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      s_red[wave][mt][0][i][lane] = accg[mt][i];
      s_red[wave][mt][1][i][lane] = accu[mt][i];
    }
  __syncthreads();
  // thread -> element i of lane l's 16x16 fragment: row 4*(l/16)+i, column l%16
  const int l = threadIdx.x & 63;
  const int i = threadIdx.x >> 6;
  const int row = 4 * (l >> 4) + i;
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    const float g = (s_red[0][mt][0][i][l] + s_red[1][mt][0][i][l]) +
                    (s_red[2][mt][0][i][l] + s_red[3][mt][0][i][l]);
    const float u = (s_red[0][mt][1][i][l] + s_red[1][mt][1][i][l]) +
                    (s_red[2][mt][1][i][l] + s_red[3][mt][1][i][l]);
    const int r = mt * 16 + row;
    if (r < rows) {
      const float hv = g / (1.0f + expf(-g)) * u;
      h[(h_row0 + r) * I + col0 + (l & 15)] = f32_to_bf16(hv);
    }
  }
  __syncthreads();
}

// gate/up + SwiGLU. One workgroup per (segment, 16 columns of h); its 4 waves split the
// reduction over H into contiguous K-step ranges and reduce through LDS. The segment's metadata
// (count, expert, offset, row count) is loaded in one round trip before the exit test; rows are
// processed in passes of 16 (a routed expert at decode has a few rows; the shared expert's
// second pass finds its weight rows in L2).
constexpr size_t kGateUpLds = sizeof(float) * 4 * 2 * 4 * 64;  // moe_gate_up_kernel's static LDS
template <int U>
__global__ __launch_bounds__(kGemmThreads) void moe_gate_up_kernel(
    const uint16_t* __restrict__ x, int H, int I, const int32_t* __restrict__ sorted_tokens,
    const int32_t* __restrict__ seg_expert, const int32_t* __restrict__ seg_offset,
    const int32_t* __restrict__ seg_count, const int32_t* __restrict__ n_segments,
    const uint16_t* __restrict__ w_gu, uint16_t* __restrict__ h, int tiles_per_seg) {
  __shared__ float s_red[4][1][2][4][64];  // kGateUpLds bytes
  // the grid strides over the live tiles (segments * tiles_per_seg), from the last one down
  SYM_FIRST_SEGMENTS(ntiles, m0, m1);
  int it = 0;
  for (int ws = blockIdx.x; ws < ntiles; ws += gridDim.x, ++it) {
    const int wt = ntiles - 1 - ws;
    const int seg = wt / tiles_per_seg;
    const SegInfo m = SYM_TILE_SEGMENT(it, wt, m0, m1);
    const int e = m.e, row0 = m.row0, cnt = m.cnt;
    const int tile = wt - seg * tiles_per_seg;
    const int col0 = tile * 16;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    const int r16 = lane & 15;
    const int kq = lane >> 4;
    const int nsteps = H >> 6;
    const int s_beg = (wave * nsteps) >> 2;
    const int s_end = ((wave + 1) * nsteps) >> 2;
    const uint16_t* wg = w_gu + ((size_t)e * 2 * I + col0 + r16) * (size_t)H + kq * kKLane;
    const uint16_t* wu = wg + (size_t)I * H;

    for (int mb = 0; mb < cnt; mb += 16) {
      const int rows = min(16, cnt - mb);
      floatx4 accg[1], accu[1];
      gate_up_pass<U>(x, H, sorted_tokens + row0 + mb, rows, wg, wu, s_beg, s_end, r16, kq,
                      accg[0], accu[0]);
      gate_up_epilogue<1>(s_red, accg, accu, wave, lane, rows, (size_t)row0 + mb, I, col0, h);
    }
  }
}

// One pass of the down projection over MT row tiles: this wave's NT 16-column tiles (sharing
// the activation fragments) over the full reduction dim I, in batches of U K-steps (weights
// first, then activations, then MFMAs).
template <int MT, int U, int NT = 2>
__device__ __forceinline__ void down_pass(const uint16_t* __restrict__ hrow, int I, int rows,
                                          const uint16_t* __restrict__ wd0,
                                          const uint16_t* __restrict__ wd1, int r16, int kq,
                                          floatx4 (&acc0)[MT], floatx4 (&acc1)[MT]) {
  const int nsteps = I >> 6;
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    acc0[mt] = floatx4{0.f, 0.f, 0.f, 0.f};
    acc1[mt] = floatx4{0.f, 0.f, 0.f, 0.f};
  }
  for (int st = 0; st < nsteps; st += U) {
    uint4 b0[U][2], b1[U][2], a[MT][U][2];
#pragma unroll
    for (int s = 0; s < U; ++s) {
      const int k = (st + s) << 6;
      b0[s][0] = ld16(wd0 + k);
      b0[s][1] = ld16(wd0 + k + kKHalf);
      if constexpr (NT == 2) {
        b1[s][0] = ld16(wd1 + k);
        b1[s][1] = ld16(wd1 + k + kKHalf);
      }
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      const uint16_t* hr = hrow + (size_t)min(mt * 16 + r16, rows - 1) * I + kq * kKLane;
#pragma unroll
      for (int s = 0; s < U; ++s) {
        const int k = (st + s) << 6;
        a[mt][s][0] = ld16(hr + k);
        a[mt][s][1] = ld16(hr + k + kKHalf);
      }
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int s = 0; s < U; ++s)
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        acc0[mt] = mfma16x16x32(a[mt][s][0], b0[s][0], acc0[mt]);
        acc0[mt] = mfma16x16x32(a[mt][s][1], b0[s][1], acc0[mt]);
        if constexpr (NT == 2) {
          acc1[mt] = mfma16x16x32(a[mt][s][0], b1[s][0], acc1[mt]);
          acc1[mt] = mfma16x16x32(a[mt][s][1], b1[s][1], acc1[mt]);
        }
      }
  }
}

template <int MT, int NT = 2>
__device__ __forceinline__ void down_store(const floatx4 (&acc0)[MT], const floatx4 (&acc1)[MT],
                                           int rows, float* __restrict__ yrow, int H, int r16,
                                           int kq) {
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int r = mt * 16 + kq * 4 + i;
      if (r < rows) {
        float* yr = yrow + (size_t)r * H + r16;
        yr[0] = acc0[mt][i];
        if constexpr (NT == 2) yr[16] = acc1[mt][i];
      }
    }
}

// down projection. One wave per (segment, 16 * kDownNT output columns); segment metadata in one
// round trip before the exit test; rows in passes of 16.
template <int U>
__global__ __launch_bounds__(kGemmThreads) void moe_down_kernel(
    const uint16_t* __restrict__ hbuf, int H, int I, const int32_t* __restrict__ seg_expert,
    const int32_t* __restrict__ seg_offset, const int32_t* __restrict__ seg_count,
    const int32_t* __restrict__ n_segments, const uint16_t* __restrict__ w_d,
    float* __restrict__ y, int tiles_per_seg) {
  // the grid strides over the live tiles; waves are independent (no LDS), so a wave whose
  // columns lie past H just moves on
  SYM_FIRST_SEGMENTS(ntiles, m0, m1);
  int it = 0;
  for (int ws = blockIdx.x; ws < ntiles; ws += gridDim.x, ++it) {
    const int wt = ntiles - 1 - ws;
    const int seg = wt / tiles_per_seg;
    const SegInfo m = SYM_TILE_SEGMENT(it, wt, m0, m1);
    const int e = m.e, row0 = m.row0, cnt = m.cnt;
    const int tile = wt - seg * tiles_per_seg;
    const int wave = threadIdx.x >> 6;
    const int lane = threadIdx.x & 63;
    const int col0 = (tile * 4 + wave) * (16 * kDownNT);
    if (col0 >= H) continue;
    const int r16 = lane & 15;
    const int kq = lane >> 4;
    const uint16_t* wd0 = w_d + ((size_t)e * H + col0 + r16) * (size_t)I + kq * kKLane;
    const uint16_t* wd1 = wd0 + (size_t)16 * I;

    for (int mb = 0; mb < cnt; mb += 16) {
      const int rows = min(16, cnt - mb);
      floatx4 acc0[1], acc1[1];
      down_pass<1, U, kDownNT>(hbuf + (size_t)(row0 + mb) * I, I, rows, wd0, wd1, r16, kq, acc0,
                               acc1);
      down_store<1, kDownNT>(acc0, acc1, rows, y + (size_t)(row0 + mb) * H + col0, H, r16, kq);
    }
  }
}

// down projection for I <= 512 (NS = I / 64 K-steps), one wave per (segment, 16 output
// columns) as moe_down_kernel, with two changes that double the weight bytes a wave has in
// flight at the same occupancy:
//  * a wave requests its 16 columns' weights over the whole of I at the start of the tile (NS x
//    32 bytes per lane, one round trip per tile instead of one per batch of 4 K-steps), and
//    keeps them in registers for every 16-row pass of the segment;
//  * the segment's h rows (the A operand, shared by the workgroup's waves) are copied once
//    per pass into LDS by LDS-DMA, wave w moving rows 8w .. 8w+7 (clamped to the last row, so
//    rows past the segment hold copies of it), and read back per K-step right before the
//    MFMAs: no registers for A, and half the L2 reads of h.
// The h DMA is issued before the weights, so waiting for it (vmcnt) leaves the weights in
// flight. A workgroup is kDownWaves = 2 waves (32 columns): small workgroups that drift apart
// keep a CU streaming through each other's barriers and stores (batch 32, 3 resident per CU:
// down 53.9-54.0 us against 56.8-57.1 for 4-wave workgroups at 2 per CU; 8-wave workgroups
// 58.2-58.6 at 2 per CU and 64.2-64.4 at 1 per CU; 1-wave workgroups at 6 per CU 54.4-54.6).
constexpr int kDownLdsSlot = 1024 + 16;  // bytes per staged row: 16 rows of an A read fall in
                                         // distinct banks (row stride 260 dwords)
constexpr size_t kDownLds = 16 * kDownLdsSlot;  // moe_down_lds_kernel's static LDS
constexpr int kDownWaves = 2;                     // waves (16 columns each) per workgroup
template <int NS>
__global__ __launch_bounds__(64 * kDownWaves) void moe_down_lds_kernel(
    const uint16_t* __restrict__ hbuf, int H, int I, const int32_t* __restrict__ seg_expert,
    const int32_t* __restrict__ seg_offset, const int32_t* __restrict__ seg_count,
    const int32_t* __restrict__ n_segments, const uint16_t* __restrict__ w_d,
    float* __restrict__ y, int tiles_per_seg) {
  static_assert(NS >= 1 && NS * 128 <= 1024, "one LDS-DMA instruction per staged row");
  __shared__ __align__(16) uint16_t s_h[16 * kDownLdsSlot / 2];
  SYM_FIRST_SEGMENTS(ntiles, m0, m1);
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const int r16 = lane & 15;
  const int kq = lane >> 4;
  // a lane's chunk of a staged row (lanes past the row re-read its last 16 bytes and write
  // them past the row's end inside its slot, never read)
  const uint32_t dma_off = (uint32_t)min(lane * 16, NS * 128 - 16);
  const uint16_t* a_frag = s_h + (r16 * kDownLdsSlot + kq * 32) / 2;
  int it = 0;
  for (int ws = blockIdx.x; ws < ntiles; ws += gridDim.x, ++it) {
    const int wt = ntiles - 1 - ws;
    const int seg = wt / tiles_per_seg;
    const SegInfo m = SYM_TILE_SEGMENT(it, wt, m0, m1);
    const int e = m.e, row0 = m.row0, cnt = m.cnt;
    const int tile = wt - seg * tiles_per_seg;
    const int col0 = (tile * kDownWaves + wave) * 16;
    const uint16_t* wd = w_d + ((size_t)e * H + col0 + r16) * (size_t)I + kq * kKLane;
    uint4 b[NS][2];
    for (int mb = 0; mb < cnt; mb += 16) {
      const int rows = min(16, cnt - mb);
      // every wave is done with the previous pass's rows before they are replaced
      asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
      const uint16_t* hb = hbuf + (size_t)(row0 + mb) * I;
      constexpr int kRowsPerWave = 16 / kDownWaves;
#pragma unroll
      for (int j = 0; j < kRowsPerWave; ++j) {
        const int r = __builtin_amdgcn_readfirstlane(min(wave * kRowsPerWave + j, rows - 1));
        dma16(hb + (size_t)r * I, dma_off, s_h + (wave * kRowsPerWave + j) * (kDownLdsSlot / 2));
      }
      if (mb == 0) {
#pragma unroll
        for (int s = 0; s < NS; ++s) {
          b[s][0] = ld16(wd + (s << 6));
          b[s][1] = ld16(wd + (s << 6) + kKHalf);
        }
        // this wave's rows have landed (the NS x 2 weight loads issued after them may still be
        // in flight), then every wave's
        asm volatile("s_waitcnt vmcnt(%0)\n\ts_barrier" ::"n"(2 * NS) : "memory");
      } else {
        asm volatile("s_waitcnt vmcnt(0)\n\ts_barrier" ::: "memory");
      }
      floatx4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int s = 0; s < NS; ++s) {
        const uint4 a0 = *reinterpret_cast<const uint4*>(a_frag + s * 64);
        const uint4 a1 = *reinterpret_cast<const uint4*>(a_frag + s * 64 + kKHalf);
        acc = mfma16x16x32(a0, b[s][0], acc);
        acc = mfma16x16x32(a1, b[s][1], acc);
      }
      float* yrow = y + (size_t)(row0 + mb) * H + col0;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int r = kq * 4 + i;
        if (r < rows) yrow[(size_t)r * H + r16] = acc[i];
      }
    }
  }
}

// ---------------------------------------------------------------------------------------------
// fp8 e4m3fn expert weights with one fp32 scale per 128 x 128 block (w = q * scale): the same
// grouped GEMMs, dequantized in-kernel. A K-step is 128 wide, one scale block: lane l streams
// 32 contiguous weight bytes of row l % 16 (4 lanes cover the 128 bytes of a row in the block),
// converts them exactly to bf16 and runs four v_mfma_f32_16x16x32_bf16 with the activations at
// the same k (MFMA j takes the lane's elements 8j .. 8j+7). The 16 rows of a wave lie in one
// 128-row block, so the block scale is wave-uniform: each step's MFMA sum is scaled once in
// fp32 and added to the accumulator. Weights in HBM are half the bf16 bytes; the products are
// exact fp8 x bf16 values, so the result equals the bf16 GEMM over dequantized weights up to
// fp32 summation order (the weights are never rounded to bf16 after scaling).
__device__ __forceinline__ floatx4 mfma_fp8_step(const uint4 (&a)[4], const uint4 (&w)[2],
                                                 floatx4 acc, float scale) {
  floatx4 t = {0.f, 0.f, 0.f, 0.f};
  t = mfma16x16x32(a[0], fp8x8_to_bf16x8(w[0].x, w[0].y), t);
  t = mfma16x16x32(a[1], fp8x8_to_bf16x8(w[0].z, w[0].w), t);
  t = mfma16x16x32(a[2], fp8x8_to_bf16x8(w[1].x, w[1].y), t);
  t = mfma16x16x32(a[3], fp8x8_to_bf16x8(w[1].z, w[1].w), t);
#pragma unroll
  for (int i = 0; i < 4; ++i) acc[i] = fmaf(scale, t[i], acc[i]);
  return acc;
}

__device__ __forceinline__ uint4 ld16b(const uint8_t* p) {
  return *reinterpret_cast<const uint4*>(p);
}

// gate/up over 16 rows of a segment, K-steps [s_beg, s_end) of 128 (a multiple of U); sg / su
// point at the scales of this wave's gate / up row block, one per K-step.
template <int U>
__device__ __forceinline__ void gate_up_pass_fp8(const uint16_t* __restrict__ x, int H,
                                                 const int32_t* __restrict__ tok_rows, int rows,
                                                 const uint8_t* __restrict__ wg,
                                                 const uint8_t* __restrict__ wu,
                                                 const float* __restrict__ sg,
                                                 const float* __restrict__ su, int s_beg,
                                                 int s_end, int r16, int kq, floatx4& accg,
                                                 floatx4& accu) {
  accg = floatx4{0.f, 0.f, 0.f, 0.f};
  accu = floatx4{0.f, 0.f, 0.f, 0.f};
  // the lane's token, loaded before the weights (see gate_up_pass)
  const int tok = tok_rows[min(r16, rows - 1)];
  __builtin_amdgcn_sched_barrier(0);
  const uint16_t* xr = x + kq * 32;
  for (int st = s_beg; st < s_end; st += U) {
    uint4 bg[U][2], bu[U][2], a[U][4];
    float cg[U], cu[U];
#pragma unroll
    for (int s = 0; s < U; ++s) {
      cg[s] = sg[st + s];
      cu[s] = su[st + s];
    }
#pragma unroll
    for (int s = 0; s < U; ++s) {
      const int k = (st + s) << 7;
      bg[s][0] = ld16b(wg + k);
      bg[s][1] = ld16b(wg + k + 16);
      bu[s][0] = ld16b(wu + k);
      bu[s][1] = ld16b(wu + k + 16);
    }
    __builtin_amdgcn_sched_barrier(0);
    if (st == s_beg) xr += (size_t)tok * H;
#pragma unroll
    for (int s = 0; s < U; ++s) {
      const int k = (st + s) << 7;
#pragma unroll
      for (int j = 0; j < 4; ++j) a[s][j] = ld16(xr + k + 8 * j);
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int s = 0; s < U; ++s) {
      accg = mfma_fp8_step(a[s], bg[s], accg, cg[s]);
      accu = mfma_fp8_step(a[s], bu[s], accu, cu[s]);
    }
  }
}

// gate/up + SwiGLU with fp8 weights: w_gu [E+1, 2I, H] e4m3fn bytes, s_gu [E+1, 2I/128, H/128].
// Workgroup = (segment, 16 columns of h) as in moe_gate_up_kernel. It launches with two 128-wide
// K-steps per load batch (U = 2, 108 VGPRs, 4 waves per SIMD): 99.2 against 101.5 us for U = 1
// at batch 128 (U = 4 needs 190 registers, 2 waves per SIMD).
template <int U>
__global__ __launch_bounds__(kGemmThreads) void moe_gate_up_fp8_kernel(
    const uint16_t* __restrict__ x, int H, int I, const int32_t* __restrict__ sorted_tokens,
    const int32_t* __restrict__ seg_expert, const int32_t* __restrict__ seg_offset,
    const int32_t* __restrict__ seg_count, const int32_t* __restrict__ n_segments,
    const uint8_t* __restrict__ w_gu, const float* __restrict__ s_gu, uint16_t* __restrict__ h,
    int tiles_per_seg) {
  __shared__ float s_red[4][1][2][4][64];
  // the grid strides over the live tiles (as moe_gate_up_kernel)
  SYM_FIRST_SEGMENTS(ntiles, m0, m1);
  int it = 0;
  for (int ws = blockIdx.x; ws < ntiles; ws += gridDim.x, ++it) {
    const int wt = ntiles - 1 - ws;
    const int seg = wt / tiles_per_seg;
    const SegInfo m = SYM_TILE_SEGMENT(it, wt, m0, m1);
    const int e = m.e, row0 = m.row0, cnt = m.cnt;
    const int tile = wt - seg * tiles_per_seg;
    const int col0 = tile * 16;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    const int r16 = lane & 15;
    const int kq = lane >> 4;
    const int nsteps = H >> 7;
    const int s_beg = (wave * nsteps) >> 2;
    const int s_end = ((wave + 1) * nsteps) >> 2;
    const uint8_t* wg = w_gu + ((size_t)e * 2 * I + col0 + r16) * (size_t)H + kq * 32;
    const uint8_t* wu = wg + (size_t)I * H;
    const int rb = (2 * I) >> 7;  // row blocks per expert
    const float* sg = s_gu + ((size_t)e * rb + (col0 >> 7)) * nsteps;
    const float* su = s_gu + ((size_t)e * rb + ((I + col0) >> 7)) * nsteps;

    for (int mb = 0; mb < cnt; mb += 16) {
      const int rows = min(16, cnt - mb);
      floatx4 accg[1], accu[1];
      gate_up_pass_fp8<U>(x, H, sorted_tokens + row0 + mb, rows, wg, wu, sg, su, s_beg, s_end, r16,
                          kq, accg[0], accu[0]);
      gate_up_epilogue<1>(s_red, accg, accu, wave, lane, rows, (size_t)row0 + mb, I, col0, h);
    }
  }
}

// down projection with fp8 weights: w_d [E+1, H, I] e4m3fn bytes, s_d [E+1, H/128, I/128]. One
// wave per (segment, 32 output columns), all of I in batches of U K-steps of 128.
template <int U>
__global__ __launch_bounds__(kGemmThreads) void moe_down_fp8_kernel(
    const uint16_t* __restrict__ hbuf, int H, int I, const int32_t* __restrict__ seg_expert,
    const int32_t* __restrict__ seg_offset, const int32_t* __restrict__ seg_count,
    const int32_t* __restrict__ n_segments, const uint8_t* __restrict__ w_d,
    const float* __restrict__ s_d, float* __restrict__ y, int tiles_per_seg) {
  // the grid strides over the live tiles (as moe_down_kernel)
  SYM_FIRST_SEGMENTS(ntiles, m0, m1);
  int it = 0;
  for (int ws = blockIdx.x; ws < ntiles; ws += gridDim.x, ++it) {
    const int wt = ntiles - 1 - ws;
    const int seg = wt / tiles_per_seg;
    const SegInfo m = SYM_TILE_SEGMENT(it, wt, m0, m1);
    const int e = m.e, row0 = m.row0, cnt = m.cnt;
    const int tile = wt - seg * tiles_per_seg;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    const int col0 = (tile * 4 + wave) * 32;
    if (col0 >= H) continue;
    const int r16 = lane & 15;
    const int kq = lane >> 4;
    const int nsteps = I >> 7;
    const uint8_t* wd0 = w_d + ((size_t)e * H + col0 + r16) * (size_t)I + kq * 32;
    const uint8_t* wd1 = wd0 + (size_t)16 * I;
    const float* sd = s_d + ((size_t)e * (H >> 7) + (col0 >> 7)) * nsteps;

    for (int mb = 0; mb < cnt; mb += 16) {
      const int rows = min(16, cnt - mb);
      const uint16_t* hr = hbuf + (size_t)(row0 + mb + min(r16, rows - 1)) * I + kq * 32;
      floatx4 acc0[1] = {{0.f, 0.f, 0.f, 0.f}}, acc1[1] = {{0.f, 0.f, 0.f, 0.f}};
      for (int st = 0; st < nsteps; st += U) {
        uint4 b0[U][2], b1[U][2], a[U][4];
        float c[U];
#pragma unroll
        for (int s = 0; s < U; ++s) c[s] = sd[st + s];
#pragma unroll
        for (int s = 0; s < U; ++s) {
          const int k = (st + s) << 7;
          b0[s][0] = ld16b(wd0 + k);
          b0[s][1] = ld16b(wd0 + k + 16);
          b1[s][0] = ld16b(wd1 + k);
          b1[s][1] = ld16b(wd1 + k + 16);
        }
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int s = 0; s < U; ++s) {
          const int k = (st + s) << 7;
#pragma unroll
          for (int j = 0; j < 4; ++j) a[s][j] = ld16(hr + k + 8 * j);
        }
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int s = 0; s < U; ++s) {
          acc0[0] = mfma_fp8_step(a[s], b0[s], acc0[0], c[s]);
          acc1[0] = mfma_fp8_step(a[s], b1[s], acc1[0], c[s]);
        }
      }
      down_store<1>(acc0, acc1, rows, y + (size_t)(row0 + mb) * H + col0, H, r16, kq);
    }
  }
}

// The conversion of fp8x8_to_bf16x8 into registers that do not overlap the source: with the
// builtins the compiler converts each weight register in place, which makes it reserve twice
// the weight registers for a whole tile of loads in flight (196 instead of about 100).
__device__ __forceinline__ uint4 fp8x8_to_bf16x8_apart(uint32_t w0, uint32_t w1) {
  uint4 r;
  asm("v_cvt_scalef32_pk_bf16_fp8 %0, %4, 1.0\n\t"
      "v_cvt_scalef32_pk_bf16_fp8 %1, %4, 1.0 op_sel:[1,0,0]\n\t"
      "v_cvt_scalef32_pk_bf16_fp8 %2, %5, 1.0\n\t"
      "v_cvt_scalef32_pk_bf16_fp8 %3, %5, 1.0 op_sel:[1,0,0]"
      : "=&v"(r.x), "=&v"(r.y), "=&v"(r.z), "=&v"(r.w)
      : "v"(w0), "v"(w1));
  return r;
}

// mfma_fp8_step with the weights converted by fp8x8_to_bf16x8_apart
__device__ __forceinline__ floatx4 mfma_fp8_step_apart(const uint4 (&a)[4], const uint4 (&w)[2],
                                                       floatx4 acc, float scale) {
  floatx4 t = {0.f, 0.f, 0.f, 0.f};
  t = mfma16x16x32(a[0], fp8x8_to_bf16x8_apart(w[0].x, w[0].y), t);
  t = mfma16x16x32(a[1], fp8x8_to_bf16x8_apart(w[0].z, w[0].w), t);
  t = mfma16x16x32(a[2], fp8x8_to_bf16x8_apart(w[1].x, w[1].y), t);
  t = mfma16x16x32(a[3], fp8x8_to_bf16x8_apart(w[1].z, w[1].w), t);
#pragma unroll
  for (int i = 0; i < 4; ++i) acc[i] = fmaf(scale, t[i], acc[i]);
  return acc;
}

// down projection with fp8 weights for I <= 512 (NS = I / 128 K-steps of 128), laid out as
// moe_down_lds_kernel: one wave per (segment, 16 output columns); the wave requests its columns'
// weight bytes over the whole of I (NS x 32 bytes per lane) and the NS block scales at the start
// of the tile and keeps them for every pass; the segment's h rows are staged in LDS by LDS-DMA
// once per pass for the workgroup's 4 waves and read back per K-step. Twice the weight bytes in
// flight per wave of the U = 1 kernel (32 columns, one K-step per batch), at 84 instead of 88
// registers (5 waves per SIMD). 32 columns per wave here need 136 registers (3 waves per
// SIMD), or spill when held to 128.
constexpr int kColsPerWG8Lds = 64;  // 4 waves x 16 columns
template <int NS>
__global__ __launch_bounds__(kGemmThreads) void moe_down_fp8_lds_kernel(
    const uint16_t* __restrict__ hbuf, int H, int I, const int32_t* __restrict__ seg_expert,
    const int32_t* __restrict__ seg_offset, const int32_t* __restrict__ seg_count,
    const int32_t* __restrict__ n_segments, const uint8_t* __restrict__ w_d,
    const float* __restrict__ s_d, float* __restrict__ y, int tiles_per_seg) {
  static_assert(NS >= 1 && NS * 256 <= 1024, "one LDS-DMA instruction per staged row");
  __shared__ __align__(16) uint16_t s_h[16 * kDownLdsSlot / 2];
  SYM_FIRST_SEGMENTS(ntiles, m0, m1);
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const int r16 = lane & 15;
  const int kq = lane >> 4;
  const uint32_t dma_off = (uint32_t)min(lane * 16, NS * 256 - 16);
  // a lane's A fragments of K-step st: 4 x 8 bf16 at k = 128 st + 32 kq + 8 j (the k order of
  // the weight bytes it holds)
  const uint16_t* a_frag = s_h + (r16 * kDownLdsSlot + kq * 64) / 2;
  int it = 0;
  for (int ws = blockIdx.x; ws < ntiles; ws += gridDim.x, ++it) {
    const int wt = ntiles - 1 - ws;
    const int seg = wt / tiles_per_seg;
    const SegInfo m = SYM_TILE_SEGMENT(it, wt, m0, m1);
    const int e = m.e, row0 = m.row0, cnt = m.cnt;
    const int tile = wt - seg * tiles_per_seg;
    const int col0 = (tile * 4 + wave) * 16;
    const uint8_t* wd = w_d + ((size_t)e * H + col0 + r16) * (size_t)I + kq * 32;
    const float* sd = s_d + ((size_t)e * (H >> 7) + (col0 >> 7)) * NS;
    uint4 b[NS][2];
    float c[NS];
    for (int mb = 0; mb < cnt; mb += 16) {
      const int rows = min(16, cnt - mb);
      // every wave is done with the previous pass's rows before they are replaced
      asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
      const uint16_t* hb = hbuf + (size_t)(row0 + mb) * I;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int r = __builtin_amdgcn_readfirstlane(min(wave * 4 + j, rows - 1));
        dma16(hb + (size_t)r * I, dma_off, s_h + (wave * 4 + j) * (kDownLdsSlot / 2));
      }
      if (mb == 0) {
#pragma unroll
        for (int st = 0; st < NS; ++st) c[st] = sd[st];
#pragma unroll
        for (int st = 0; st < NS; ++st) {
          b[st][0] = ld16b(wd + (st << 7));
          b[st][1] = ld16b(wd + (st << 7) + 16);
        }
        // this wave's rows have landed (the 2 NS weight loads issued after them may still be in
        // flight), then every wave's
        asm volatile("s_waitcnt vmcnt(%0)\n\ts_barrier" ::"n"(2 * NS) : "memory");
      } else {
        asm volatile("s_waitcnt vmcnt(0)\n\ts_barrier" ::: "memory");
      }
      floatx4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int st = 0; st < NS; ++st) {
        uint4 a[4];
#pragma unroll
        for (int j = 0; j < 4; ++j)
          a[j] = *reinterpret_cast<const uint4*>(a_frag + st * 128 + 8 * j);
        acc = mfma_fp8_step_apart(a, b[st], acc, c[st]);
        // one step's fragments and conversions live at a time
        __builtin_amdgcn_sched_barrier(0);
      }
      float* yrow = y + (size_t)(row0 + mb) * H + col0;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int r = kq * 4 + i;
        if (r < rows) yrow[(size_t)r * H + r16] = acc[i];
      }
    }
  }
}

// 8 consecutive values of a y row (fp32, or bf16 widened exactly)
__device__ __forceinline__ void load_y8(const float* p, float (&f)[8]) {
  const float4 a = reinterpret_cast<const float4*>(p)[0], b = reinterpret_cast<const float4*>(p)[1];
  f[0] = a.x; f[1] = a.y; f[2] = a.z; f[3] = a.w;
  f[4] = b.x; f[5] = b.y; f[6] = b.z; f[7] = b.w;
}
__device__ __forceinline__ void load_y8(const uint16_t* p, float (&f)[8]) {
  unpack8(*reinterpret_cast<const uint4*>(p), f);
}

// Top-k assignments whose row indices, weights and y rows are loaded in one batch: the row
// loads depend on the indices, so a batch costs two round trips instead of two per assignment.
constexpr int kCombineBatch = 8;

template <typename YT>
__global__ __launch_bounds__(256) void moe_combine_kernel(
    const YT* __restrict__ y, const int32_t* __restrict__ inv_perm,
    const float* __restrict__ topk_w, int K, int H, int shared_row0,
    const float* __restrict__ residual, uint16_t* __restrict__ out) {
  const int t = blockIdx.x;
  const int32_t* ip = inv_perm + (size_t)t * K;
  const float* tw = topk_w + (size_t)t * K;
  const int stride = gridDim.y * blockDim.x * 8;
  for (int c = (blockIdx.y * blockDim.x + threadIdx.x) * 8; c < H; c += stride) {
    // the shared expert's row and the residual do not depend on the routing: issued first
    float sh[8], rs[8];
    if (shared_row0 >= 0) load_y8(y + (size_t)(shared_row0 + t) * H + c, sh);
    if (residual) load_y8(residual + (size_t)t * H + c, rs);
    float acc[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) acc[i] = 0.f;
    for (int k0 = 0; k0 < K; k0 += kCombineBatch) {
      // indices past K repeat the last assignment's (in-bounds) row; they are not accumulated
      int row[kCombineBatch];
      float wk[kCombineBatch];
#pragma unroll
      for (int j = 0; j < kCombineBatch; ++j) {
        const int k = min(k0 + j, K - 1);
        row[j] = ip[k];
        wk[j] = tw[k];
      }
      float f[kCombineBatch][8];
#pragma unroll
      for (int j = 0; j < kCombineBatch; ++j) load_y8(y + (size_t)row[j] * H + c, f[j]);
      // assignments added in k order, as one at a time
#pragma unroll
      for (int j = 0; j < kCombineBatch; ++j)
        if (k0 + j < K)
#pragma unroll
          for (int i = 0; i < 8; ++i) acc[i] += wk[j] * f[j][i];
    }
    if (shared_row0 >= 0)
#pragma unroll
      for (int i = 0; i < 8; ++i) acc[i] += sh[i];
    if (residual)
#pragma unroll
      for (int i = 0; i < 8; ++i) acc[i] += rs[i];
    uint4 o;
    o.x = pack_bf16x2(acc[0], acc[1]);
    o.y = pack_bf16x2(acc[2], acc[3]);
    o.z = pack_bf16x2(acc[4], acc[5]);
    o.w = pack_bf16x2(acc[6], acc[7]);
    *reinterpret_cast<uint4*>(out + (size_t)t * H + c) = o;
  }
}

}  // namespace sym

using namespace sym;

// Grid of the decode expert GEMMs: kPersistWGsPerCU workgroups per CU (kDownWGsPerCU for the
// bf16 down kernel), striding over the live tiles, or fewer when there are fewer tiles at most.
// Measured with the bf16 kernels at two resident per CU (below), batch 32 (4832 live tiles of
// 8224 possible): 20 to 32 per CU
// 223.3-223.8 us per step, 24 223.3-223.6, 16 224.5-225.2, 12 226.3-226.6, 8 228.2-228.5; the
// fp8 step at batch 128: 24 per CU 334.6-334.9 against 338.1-338.9 us at 16.
constexpr int kPersistWGsPerCU = 24;

// The bf16 decode expert GEMMs are launched with dynamic LDS (not read by the kernels) that
// bounds how many of them share a CU's 160 KB: gate/up at 64 KB, so at most 2 per CU (8 waves)
// instead of 3 by registers; fewer weight streams in flight at once stream faster (batch 32,
// with down's 4-wave workgroups also held to 2: 225.6 against 227.4-227.9 us per step). Down
// runs 2-wave workgroups held to 3 per CU (below). The fp8 kernels keep their own bound (4 and
// 5 per CU): capped at 3 per CU the fp8 step was no faster, at 2 it was 18 us slower.
constexpr size_t kDecodeGemmLds = 64 * 1024;
// moe_down_lds_kernel's 2-wave workgroups are held to 3 per CU (48 KB each; 6 waves per CU): at
// 2 per CU the step took 233.6-233.9 us, at 4 or 5 per CU 223.0-223.5, at 3 per CU 220.3-221.1,
// and 32 workgroups per CU in the grid (9664 live tiles at batch 32) 220.0-220.5 against
// 220.7-221.1 at 48, 220.8-221.0 at 28 and 222.0-223.3 at 16-24.
constexpr size_t kDownGemmLds = 48 * 1024;
constexpr int kDownWGsPerCU = 32;
// Above 32 rows more experts are live and their tiles outnumber those grids: gate/up at 32 and
// down at 56 per CU took the whole-model decode at batch 64 from 6.76 to 6.67-6.68 ms per step
// (gate/up at 32 alone 6.71; both at 40 / 64 6.68), while at batch 32 they cost 1.5 us.
constexpr int kPersistWGsPerCULarge = 32;
constexpr int kDownWGsPerCULarge = 56;
// The fp8 gate/up and LDS down kernels (batch 128: 7904 live tiles each): 40 workgroups per CU,
// one per tile, 331.5-332.1 us per fp8 step against 333.2-334.0 at 24 (48 and 64 the same as 40).
constexpr int kFp8WGsPerCU = 40;
static_assert(kGateUpLds < kDecodeGemmLds && kDownLds < kDownGemmLds, "the static LDS fits");

static int persistent_grid(int max_tiles, int per_cu = kPersistWGsPerCU) {
  const int n = per_cu * sym_host::cu_count();
  return max_tiles < n ? max_tiles : n;
}

static int check_gemm_args(const char* what, int T, int H, int I, int max_segments) {
  SYM_REQUIRE(T >= 0, SYM_ERR_INVALID, "%s: T=%d < 0", what, T);
  SYM_REQUIRE(H > 0 && H % 256 == 0, SYM_ERR_UNSUPPORTED,
              "%s: H=%d must be a positive multiple of 256", what, H);
  SYM_REQUIRE(I > 0 && I % 64 == 0, SYM_ERR_UNSUPPORTED,
              "%s: I=%d must be a positive multiple of 64", what, I);
  SYM_REQUIRE(max_segments >= 1 && max_segments <= 4096, SYM_ERR_INVALID,
              "%s: max_segments=%d out of range", what, max_segments);
  return SYM_OK;
}

extern "C" int sym_moe_gate_up(const void* x, int T, int H, int I, const int32_t* sorted_tokens,
                               const int32_t* seg_expert, const int32_t* seg_offset,
                               const int32_t* seg_count, const int32_t* n_segments,
                               int max_segments, const void* w_gate_up, void* h, void* stream) {
  int rc = check_gemm_args("moe_gate_up", T, H, I, max_segments);
  if (rc) return rc;
  if (T == 0) return SYM_OK;
  SYM_REQUIRE(x && sorted_tokens && seg_expert && seg_offset && seg_count && n_segments &&
                  w_gate_up && h,
              SYM_ERR_INVALID, "moe_gate_up: null pointer argument");
  (void)hipGetLastError();
  const int tiles = I / 16;
  const int wave_steps = H / 256;  // K-steps of 64 per wave (4 waves split H)
  const dim3 grid(persistent_grid(max_segments * tiles, T > 32 ? kPersistWGsPerCULarge
                                                               : kPersistWGsPerCU)),
      block(kGemmThreads);
#define SYM_LAUNCH_GATE_UP(UU)                                                                  \
  hipLaunchKernelGGL((moe_gate_up_kernel<UU>), grid, block, kDecodeGemmLds - kGateUpLds,         \
                     (hipStream_t)stream,                                                        \
                     (const uint16_t*)x, H, I, sorted_tokens, seg_expert, seg_offset, seg_count, \
                     n_segments, (const uint16_t*)w_gate_up, (uint16_t*)h, tiles)
  if (wave_steps % 4 == 0) SYM_LAUNCH_GATE_UP(4);
  else if (wave_steps % 2 == 0) SYM_LAUNCH_GATE_UP(2);
  else SYM_LAUNCH_GATE_UP(1);
#undef SYM_LAUNCH_GATE_UP
  return sym_host::check_launch("moe_gate_up_kernel");
}

extern "C" int sym_moe_down(const void* h, int T, int H, int I, const int32_t* seg_expert,
                            const int32_t* seg_offset, const int32_t* seg_count,
                            const int32_t* n_segments, int max_segments, const void* w_down,
                            float* y, void* stream) {
  int rc = check_gemm_args("moe_down", T, H, I, max_segments);
  if (rc) return rc;
  if (T == 0) return SYM_OK;
  SYM_REQUIRE(h && seg_expert && seg_offset && seg_count && n_segments && w_down && y,
              SYM_ERR_INVALID, "moe_down: null pointer argument");
  (void)hipGetLastError();
  const int steps = I / 64;  // K-steps of 64 per wave (one wave covers all of I)
  if (steps <= 8) {
    const int tiles = H / (16 * kDownWaves);
    const dim3 grid(persistent_grid(max_segments * tiles,
                                    T > 32 ? kDownWGsPerCULarge : kDownWGsPerCU)),
        block(64 * kDownWaves);
#define SYM_LAUNCH_DOWN_LDS(NS)                                                                 \
  case NS:                                                                                      \
    hipLaunchKernelGGL((moe_down_lds_kernel<NS>), grid, block, kDownGemmLds - kDownLds,        \
                       (hipStream_t)stream,                                                      \
                       (const uint16_t*)h, H, I, seg_expert, seg_offset, seg_count, n_segments,  \
                       (const uint16_t*)w_down, y, tiles);                                       \
    break;
    switch (steps) {
      SYM_LAUNCH_DOWN_LDS(1) SYM_LAUNCH_DOWN_LDS(2) SYM_LAUNCH_DOWN_LDS(3)
      SYM_LAUNCH_DOWN_LDS(4) SYM_LAUNCH_DOWN_LDS(5) SYM_LAUNCH_DOWN_LDS(6)
      SYM_LAUNCH_DOWN_LDS(7) SYM_LAUNCH_DOWN_LDS(8)
    }
#undef SYM_LAUNCH_DOWN_LDS
    return sym_host::check_launch("moe_down_lds_kernel");
  }
  const int tiles = (H + kColsPerWG - 1) / kColsPerWG;
  const dim3 grid(persistent_grid(max_segments * tiles)), block(kGemmThreads);
#define SYM_LAUNCH_DOWN(UU)                                                                     \
  hipLaunchKernelGGL((moe_down_kernel<UU>), grid, block, 0, (hipStream_t)stream,                 \
                     (const uint16_t*)h, H, I, seg_expert, seg_offset, seg_count, n_segments,    \
                     (const uint16_t*)w_down, y, tiles)
  if (steps % 4 == 0) SYM_LAUNCH_DOWN(4);
  else if (steps % 2 == 0) SYM_LAUNCH_DOWN(2);
  else SYM_LAUNCH_DOWN(1);
#undef SYM_LAUNCH_DOWN
  return sym_host::check_launch("moe_down_kernel");
}

extern "C" int sym_moe_grouped_swiglu(const void* x, int T, int H, int I,
                                      const int32_t* sorted_tokens, const int32_t* seg_expert,
                                      const int32_t* seg_offset, const int32_t* seg_count,
                                      const int32_t* n_segments, int max_segments,
                                      const void* w_gate_up, const void* w_down, void* h, float* y,
                                      void* stream) {
  int rc = sym_moe_gate_up(x, T, H, I, sorted_tokens, seg_expert, seg_offset, seg_count,
                           n_segments, max_segments, w_gate_up, h, stream);
  if (rc) return rc;
  return sym_moe_down(h, T, H, I, seg_expert, seg_offset, seg_count, n_segments, max_segments,
                      w_down, y, stream);
}

extern "C" int sym_moe_unpermute_combine(const void* y, int y_bf16, const int32_t* inv_perm,
                                         const float* topk_w, int T, int top_k, int H,
                                         int shared_row0, const float* residual, void* out,
                                         void* stream) {
  SYM_REQUIRE(T >= 0, SYM_ERR_INVALID, "moe_unpermute_combine: T=%d < 0", T);
  if (T == 0) return SYM_OK;
  SYM_REQUIRE(y && inv_perm && topk_w && out, SYM_ERR_INVALID,
              "moe_unpermute_combine: null pointer argument");
  SYM_REQUIRE(H > 0 && H % 8 == 0, SYM_ERR_UNSUPPORTED,
              "moe_unpermute_combine: H=%d must be a positive multiple of 8", H);
  SYM_REQUIRE(top_k >= 1 && top_k <= 64, SYM_ERR_INVALID, "moe_unpermute_combine: top_k=%d",
              top_k);
  (void)hipGetLastError();
  // a decode batch spreads each token's row over several 64-thread workgroups (more CUs
  // loading the assignments' rows at once); prefill sizes keep one 256-thread workgroup per
  // token
  const int threads = T >= 128 ? 256 : 64;
  const int chunks = (H + threads * 8 - 1) / (threads * 8);
  SYM_REQUIRE(chunks <= 65535, SYM_ERR_UNSUPPORTED, "moe_unpermute_combine: H=%d too large", H);
  const dim3 grid(T, chunks), block(threads);
  if (y_bf16)
    hipLaunchKernelGGL(moe_combine_kernel<uint16_t>, grid, block, 0, (hipStream_t)stream,
                       (const uint16_t*)y, inv_perm, topk_w, top_k, H, shared_row0, residual,
                       (uint16_t*)out);
  else
    hipLaunchKernelGGL(moe_combine_kernel<float>, grid, block, 0, (hipStream_t)stream,
                       (const float*)y, inv_perm, topk_w, top_k, H, shared_row0, residual,
                       (uint16_t*)out);
  return sym_host::check_launch("moe_combine_kernel");
}

static int check_fp8_gemm_args(const char* what, int T, int H, int I, int max_segments) {
  SYM_REQUIRE(T >= 0, SYM_ERR_INVALID, "%s: T=%d < 0", what, T);
  SYM_REQUIRE(H > 0 && H % 512 == 0, SYM_ERR_UNSUPPORTED,
              "%s: H=%d must be a positive multiple of 512", what, H);
  SYM_REQUIRE(I > 0 && I % 128 == 0, SYM_ERR_UNSUPPORTED,
              "%s: I=%d must be a positive multiple of 128", what, I);
  SYM_REQUIRE(max_segments >= 1 && max_segments <= 4096, SYM_ERR_INVALID,
              "%s: max_segments=%d out of range", what, max_segments);
  return SYM_OK;
}

extern "C" int sym_moe_gate_up_fp8(const void* x, int T, int H, int I,
                                   const int32_t* sorted_tokens, const int32_t* seg_expert,
                                   const int32_t* seg_offset, const int32_t* seg_count,
                                   const int32_t* n_segments, int max_segments,
                                   const void* w_gate_up, const float* s_gate_up, void* h,
                                   void* stream) {
  int rc = check_fp8_gemm_args("moe_gate_up_fp8", T, H, I, max_segments);
  if (rc) return rc;
  if (T == 0) return SYM_OK;
  SYM_REQUIRE(x && sorted_tokens && seg_expert && seg_offset && seg_count && n_segments &&
                  w_gate_up && s_gate_up && h,
              SYM_ERR_INVALID, "moe_gate_up_fp8: null pointer argument");
  (void)hipGetLastError();
  const int tiles = I / 16;
  const dim3 grid(persistent_grid(max_segments * tiles, kFp8WGsPerCU)), block(kGemmThreads);
#define SYM_LAUNCH_GATE_UP_FP8(UU)                                                              \
  hipLaunchKernelGGL((moe_gate_up_fp8_kernel<UU>), grid, block, 0, (hipStream_t)stream,          \
                     (const uint16_t*)x, H, I, sorted_tokens, seg_expert, seg_offset, seg_count, \
                     n_segments, (const uint8_t*)w_gate_up, s_gate_up, (uint16_t*)h, tiles)
  // a wave's K-range is H / 512 steps of 128 (H % 512 == 0): two per batch when it is even
  if ((H / 512) % 2 == 0) SYM_LAUNCH_GATE_UP_FP8(2);
  else SYM_LAUNCH_GATE_UP_FP8(1);
#undef SYM_LAUNCH_GATE_UP_FP8
  return sym_host::check_launch("moe_gate_up_fp8_kernel");
}

extern "C" int sym_moe_down_fp8(const void* h, int T, int H, int I, const int32_t* seg_expert,
                                const int32_t* seg_offset, const int32_t* seg_count,
                                const int32_t* n_segments, int max_segments, const void* w_down,
                                const float* s_down, float* y, void* stream) {
  int rc = check_fp8_gemm_args("moe_down_fp8", T, H, I, max_segments);
  if (rc) return rc;
  if (T == 0) return SYM_OK;
  SYM_REQUIRE(h && seg_expert && seg_offset && seg_count && n_segments && w_down && s_down && y,
              SYM_ERR_INVALID, "moe_down_fp8: null pointer argument");
  (void)hipGetLastError();
  if (I <= 512) {
    const int tiles = H / kColsPerWG8Lds;
    const dim3 grid(persistent_grid(max_segments * tiles, kFp8WGsPerCU)), block(kGemmThreads);
#define SYM_LAUNCH_DOWN_FP8_LDS(NS)                                                             \
  case NS:                                                                                      \
    hipLaunchKernelGGL((moe_down_fp8_lds_kernel<NS>), grid, block, 0, (hipStream_t)stream,       \
                       (const uint16_t*)h, H, I, seg_expert, seg_offset, seg_count, n_segments,  \
                       (const uint8_t*)w_down, s_down, y, tiles);                                \
    break;
    switch (I / 128) {
      SYM_LAUNCH_DOWN_FP8_LDS(1) SYM_LAUNCH_DOWN_FP8_LDS(2) SYM_LAUNCH_DOWN_FP8_LDS(3)
      SYM_LAUNCH_DOWN_FP8_LDS(4)
    }
#undef SYM_LAUNCH_DOWN_FP8_LDS
    return sym_host::check_launch("moe_down_fp8_lds_kernel");
  }
  const int tiles = (H + kColsPerWG8 - 1) / kColsPerWG8;
  const dim3 grid(persistent_grid(max_segments * tiles)), block(kGemmThreads);
#define SYM_LAUNCH_DOWN_FP8(UU)                                                                 \
  hipLaunchKernelGGL((moe_down_fp8_kernel<UU>), grid, block, 0, (hipStream_t)stream,             \
                     (const uint16_t*)h, H, I, seg_expert, seg_offset, seg_count, n_segments,    \
                     (const uint8_t*)w_down, s_down, y, tiles)
  SYM_LAUNCH_DOWN_FP8(1);
#undef SYM_LAUNCH_DOWN_FP8
  return sym_host::check_launch("moe_down_fp8_kernel");
}
