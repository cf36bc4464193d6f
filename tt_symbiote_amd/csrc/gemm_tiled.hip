// Tiled bf16 GEMMs for prefill-size problems (MFMA-bound): dense projections and the grouped
// expert GEMMs over ragged, expert-sorted rows.
//
// Reference: the projections of TTNNBailingMoEAttention (ttnn_attention.py:2001-2011) at
// sequence length > 1, and the expert sparse_matmuls of TTNNExperts.forward
// (ttnn_moe.py:1250-1289) with the shared expert (ttnn_moe.py:656-675), for prefill batches.
//
// Design (gfx950): a workgroup of 8 waves computes a 128 x 256 output tile; wave w owns the
// 64 x 64 block (rows 64*(w/4), columns 64*(w%4)) as 4 x 4 v_mfma_f32_16x16x32_bf16 tiles. The
// K loop moves 32 columns per step through a 3-stage LDS ring (24 KB per stage, 72 KB, so two
// workgroups share a CU and one's barrier waits are covered by the other's MFMAs): the operand
// tiles go from global memory straight into LDS (global_load_lds_dwordx4, no register staging),
// two steps ahead of the MFMAs, with one barrier per step; a step's fragment reads are all
// issued before its MFMAs. A wave-wide LDS-DMA instruction writes 1 KB = 16 rows of 32 bf16
// contiguously (lane l -> row l/4, 16-byte slot l%4), so each lane fetches the global chunk
// (l%4) ^ swz(row) with swz(r) = (r/2) % 4: chunk c of row r sits in slot c ^ swz(r), and the 16
// rows of an MFMA fragment read (one chunk each) fall in distinct banks. (A 64-wide step with
// 144 KB of LDS, one workgroup per CU, measured 10% slower on the dense projections.)
//   DENSE:   out[M, N] = A[M, K] . W[N, K]^T (+ bias) (+ residual fp32), bf16 or fp32 out.
//   GATE_UP: rows of a segment gather x[sorted_tokens[row]]; the B tile holds 128 gate rows and
//            the matching 128 up rows of the expert, so each wave's block pairs 32 gate with 32
//            up columns and the epilogue writes h = silu(gate) * up (bf16).
//   DOWN:    rows of a segment are h rows (contiguous); y = h . W_down^T (fp32 or bf16).
// Rows past a tile's valid rows and columns past N repeat the last row / column in the loads
// (always in bounds) and are not stored.
// Grouped modes: the workgroup's row tile is found from the device-side segment list (each
// segment owns ceil(count / 128) consecutive tiles of the grid's y range); workgroups past the
// last tile exit.
#include "common.h"

namespace sym {

constexpr int kTK = 32;  // 72 KB of LDS: two workgroups per CU (64: 144 KB, one; 10% slower)
constexpr int kTM = 128, kTN = 256;
constexpr int kWavesN = 4;  // waves along N (2 along M, 64 rows each)
constexpr int kTileWaves = 2 * kWavesN;
constexpr int kTileThreads = 64 * kTileWaves;
constexpr int kWN = kTN / kWavesN;  // output columns per wave (B rows of its fragments)
constexpr int kNJ = kWN / 16;       // 16-column MFMA tiles per wave
constexpr int kAStage = kTM * kTK;  // bf16 elements of one A stage (16 KB at kTK = 64)
constexpr int kBStage = kTN * kTK;  // bf16 elements of one B stage (32 KB)
constexpr int kStage = kAStage + kBStage;
constexpr int kDmaPerStep = (kAStage + kBStage) * 2 / 1024 / kTileWaves;  // per wave
constexpr int kChunksPerRow = kTK / 8;          // 16-byte chunks per LDS row
constexpr int kRowsPerDma = 64 / kChunksPerRow;  // rows one wave-wide LDS-DMA instruction fills
static_assert(kTK == 32 || kTK == 64, "tile K");

// LDS slot of chunk c in row r: c ^ swz(r), chosen so that the 16 rows of a fragment read (one
// chunk each) fall in distinct banks: 8 chunks per 128-byte row -> r % 8; 4 chunks per 64-byte
// row (two rows per 128 bytes) -> (r / 2) % 4.
__device__ __forceinline__ int tile_swz(int r) {
  return kChunksPerRow == 8 ? (r & 7) : ((r >> 1) & 3);
}
constexpr int kMaxGemmSegments = 4096;  // grid bound on segments (y range)

enum TileMode { kDense = 0, kGateUp = 1, kDown = 2 };

struct TileArgs {
  const uint16_t* a;        // DENSE/DOWN: rows [., K]; GATE_UP: x [T, K]
  const uint16_t* w;        // DENSE: [N, K]; GATE_UP: [S, 2I, K]; DOWN: [S, N, K]
  const uint16_t* bias;     // DENSE, optional [N]
  const float* residual;    // DENSE, optional [M, N] fp32
  const int32_t* sorted_tokens;
  const int32_t* seg_expert;
  const int32_t* seg_offset;
  const int32_t* seg_count;
  const int32_t* n_segments;
  int M, N, K;              // GATE_UP: N = I (h columns); DOWN: N = H
  uint16_t* out_bf16;
  float* out_f32;
  long long w_zstride;      // DENSE: grid z selects weight plane w + z * w_zstride ...
  long long out_zstride;    // ... and output plane out + z * out_zstride (elements)
};

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// 16 bytes per lane from global memory into LDS at base + 16 * lane (base wave-uniform, in M0).
// Written as asm so that the compiler does not add its own (conservative) waits for these LDS
// writes: the kernel waits for them explicitly (SYM_TILE_SYNC) before the barrier that
// publishes a stage.
// (M0 is written here only; no other instruction of these kernels reads it.)
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
__device__ __forceinline__ void dma16(const uint16_t* g, const uint16_t* lds_base) {
  const uint32_t lds = (uint32_t)(uintptr_t)lds_base;
  asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dwordx4 %1, off" ::"s"(lds), "v"(g)
               : "memory", "m0");
}
#pragma clang diagnostic pop

// Wait until at most N of this wave's vector-memory loads are outstanding (the LDS-DMA of the
// later steps), then the workgroup barrier. The asm is a compiler memory barrier, so no LDS
// access moves across it; a plain __syncthreads would also wait for every DMA in flight.
#define SYM_TILE_SYNC(N) \
  asm volatile("s_waitcnt vmcnt(" #N ")\n\ts_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory")

template <int MODE>
__global__ __launch_bounds__(kTileThreads) __attribute__((amdgpu_waves_per_eu(kTileWaves / 4 * 2)))
void gemm_tile_kernel(TileArgs p) {
  // stage s = [A (16 KB) | B (32 KB)] at smem + s * kStage: one base address per stage keeps every
  // fragment read of the stage within the 64 KB immediate offset of an LDS instruction
  __shared__ __align__(1024) uint16_t smem[3 * kStage];

  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
  const int wm = wave / kWavesN, wn = wave % kWavesN;
  const int r16 = lane & 15, kq = lane >> 4;
  const int K = p.K;

  // ---- locate the tile ----
  int row0, rows, e = 0;  // first output row, valid rows in the tile, expert
  const int ct = blockIdx.x, gy = blockIdx.y;
  if constexpr (MODE == kDense) {
    row0 = gy * kTM;
    rows = min(kTM, p.M - row0);
    p.w += blockIdx.z * p.w_zstride;
    if (p.out_f32) p.out_f32 += blockIdx.z * p.out_zstride;
    else p.out_bf16 += blockIdx.z * p.out_zstride;
  } else {
    // Every wave scans the segment list 64 segments at a time (prefix sum by lane shuffles)
    // and stops at the one holding tile g: no LDS and no barrier, and all waves agree.
    const int nseg = p.n_segments[0];
    const int g = gy;
    int seg = -1, start = 0, run = 0;
    for (int s0 = 0; s0 < nseg; s0 += 64) {
      const int s = s0 + lane;
      const int nt = s < nseg ? (p.seg_count[s] + kTM - 1) / kTM : 0;
      int x = nt;
#pragma unroll
      for (int off = 1; off < 64; off <<= 1) {
        const int y = __shfl_up(x, off);
        if (lane >= off) x += y;
      }
      const int st = run + x - nt;
      const unsigned long long hit = __ballot(nt > 0 && st <= g && g < st + nt);
      if (hit) {
        const int l = __ffsll((long long)hit) - 1;
        seg = s0 + l;
        start = __shfl(st, l);
        break;
      }
      run += __shfl(x, 63);
    }
    if (seg < 0) return;  // past the last tile (the grid is sized for the worst case)
    const int rt = g - start;
    e = p.seg_expert[seg];
    row0 = p.seg_offset[seg] + rt * kTM;
    rows = min(kTM, p.seg_count[seg] - rt * kTM);
  }

  // ---- LDS-DMA sources: this wave fills A rows 16w .. 16w+15 and B rows 32w .. 32w+31 of
  // every stage; lane l takes row + l / kChunksPerRow, slot l % kChunksPerRow, i.e. global chunk
  // slot ^ swz(row)
  constexpr int kARows = kTM / kTileWaves, kBRows = kTN / kTileWaves;  // rows filled per wave
  constexpr int kADma = kARows / kRowsPerDma, kBDma = kBRows / kRowsPerDma;
  const int lr = lane / kChunksPerRow;
  const int a_row_l = wave * kARows + lr;   // + kRowsPerDma * i
  const int b_row_l = wave * kBRows + lr;
  const int chunk = ((lane % kChunksPerRow) ^ tile_swz(lr)) * 8;  // swz(row) == swz(lr)
  const uint16_t* a_src[kADma];
  const uint16_t* b_src[kBDma];
#pragma unroll
  for (int i = 0; i < kADma; ++i) {
    const int r = min(a_row_l + kRowsPerDma * i, rows - 1);
    size_t arow;
    if constexpr (MODE == kGateUp) arow = (size_t)p.sorted_tokens[row0 + r];
    else arow = (size_t)(row0 + r);
    a_src[i] = p.a + arow * K + chunk;
  }
#pragma unroll
  for (int i = 0; i < kBDma; ++i) {
    const int br = b_row_l + kRowsPerDma * i;  // B tile row 0..255
    size_t brow;
    if constexpr (MODE == kGateUp) {
      // 128 gate rows then the matching 128 up rows of expert e
      const int col = min(ct * 128 + (br & 127), p.N - 1);
      brow = (size_t)e * 2 * p.N + (br < 128 ? col : p.N + col);
    } else if constexpr (MODE == kDown) {
      brow = (size_t)e * p.N + min(ct * kTN + br, p.N - 1);
    } else {
      brow = (size_t)min(ct * kTN + br, p.N - 1);
    }
    b_src[i] = p.w + brow * K + chunk;
  }
  const int a_dst = wave * kARows * kTK;  // element offset of this wave's first A row in a stage
  const int b_dst = wave * kBRows * kTK;

  auto issue = [&](int kt, uint16_t* stage) {
    const int k = kt * kTK;
#pragma unroll
    for (int i = 0; i < kADma; ++i) dma16(a_src[i] + k, stage + a_dst + i * 512);
#pragma unroll
    for (int i = 0; i < kBDma; ++i) dma16(b_src[i] + k, stage + kAStage + b_dst + i * 512);
  };

  // fragment rows of this wave: A rows wm*64 + 16i + r16; B rows per column tile j
  // GATE_UP: the first kNJ/2 tiles are gate columns wn*kWN/2 .. +kWN/2, the rest the matching
  // up columns (B rows 128 + ...)
  int b_frag[kNJ];
#pragma unroll
  for (int j = 0; j < kNJ; ++j) {
    if constexpr (MODE == kGateUp)
      b_frag[j] = (j < kNJ / 2 ? 0 : 128) + wn * (kWN / 2) + (j % (kNJ / 2)) * 16 + r16;
    else
      b_frag[j] = wn * kWN + j * 16 + r16;
  }
  const int sw = tile_swz(r16);  // every fragment row r has swz(r) == swz(r16)

  floatx4 acc[4][kNJ];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < kNJ; ++j) acc[i][j] = floatx4{0.f, 0.f, 0.f, 0.f};

  // all fragment reads of the step are issued before its MFMAs
  auto compute = [&](const uint16_t* stage) {
    const uint16_t* sA = stage;
    const uint16_t* sB = stage + kAStage;
    u32x4 fa[2][4], fb[2][kNJ];
#pragma unroll
    for (int kh = 0; kh < kTK / 32; ++kh) {
      const int slot = ((kh * 4 + kq) ^ sw) * 8;
#pragma unroll
      for (int i = 0; i < 4; ++i)
        fa[kh][i] = *reinterpret_cast<const u32x4*>(&sA[(wm * 64 + i * 16 + r16) * kTK + slot]);
#pragma unroll
      for (int j = 0; j < kNJ; ++j)
        fb[kh][j] = *reinterpret_cast<const u32x4*>(&sB[b_frag[j] * kTK + slot]);
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int kh = 0; kh < kTK / 32; ++kh)
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < kNJ; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
              __builtin_bit_cast(bf16x8, fa[kh][i]), __builtin_bit_cast(bf16x8, fb[kh][j]),
              acc[i][j], 0, 0, 0);
  };

  // Step k: wait for its stage (the DMA of step k + 1 may still be in flight), barrier (every
  // wave is also done with step k - 1's stage), issue step k + 2 into that stage, MFMAs. Step k
  // uses stage k % 3.
  static_assert(kDmaPerStep == 3 || kDmaPerStep == 6 || kDmaPerStep == 12, "SYM_TILE_SYNC count");
  const int nk = K / kTK;
  issue(0, smem);
  if (nk > 1) issue(1, smem + kStage);
  int cur = 0;  // stage of step kt (element offset)
  for (int kt = 0; kt < nk; ++kt) {
    if (kt + 1 >= nk) SYM_TILE_SYNC(0);
    else if constexpr (kDmaPerStep == 12) SYM_TILE_SYNC(12);
    else if constexpr (kDmaPerStep == 6) SYM_TILE_SYNC(6);
    else SYM_TILE_SYNC(3);
    const int nxt = cur == 0 ? 2 * kStage : cur - kStage;  // stage of step kt + 2
    if (kt + 2 < nk) issue(kt + 2, smem + nxt);
    compute(smem + cur);
    cur = cur == 2 * kStage ? 0 : cur + kStage;
  }

  // ---- epilogue: lane holds rows 4*(l/16)+q, column l%16 of each 16 x 16 tile ----
#pragma unroll
  for (int i = 0; i < 4; ++i) {
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int r = wm * 64 + i * 16 + kq * 4 + q;
      if (r >= rows) continue;
      const size_t orow = (size_t)(row0 + r);
      if constexpr (MODE == kGateUp) {
#pragma unroll
        for (int j = 0; j < kNJ / 2; ++j) {
          const int col = ct * 128 + wn * (kWN / 2) + j * 16 + r16;
          if (col >= p.N) continue;
          const float g = acc[i][j][q], u = acc[i][j + kNJ / 2][q];
          p.out_bf16[orow * p.N + col] = f32_to_bf16(g / (1.0f + expf(-g)) * u);
        }
      } else {
#pragma unroll
        for (int j = 0; j < kNJ; ++j) {
          const int col = ct * kTN + wn * kWN + j * 16 + r16;
          if (col >= p.N) continue;
          float v = acc[i][j][q];
          if constexpr (MODE == kDense) {
            if (p.bias) v += bf16_to_f32(p.bias[col]);
            if (p.residual) v += p.residual[orow * p.N + col];
          }
          if (p.out_f32) p.out_f32[orow * p.N + col] = v;
          else p.out_bf16[orow * p.N + col] = f32_to_bf16(v);
        }
      }
    }
  }
}

}  // namespace sym

using namespace sym;

extern "C" int sym_gemm_bf16(const void* a, const void* w, const void* bias, const float* residual,
                             int M, int N, int K, void* out, int out_fp32, void* stream) {
  SYM_REQUIRE(M >= 0, SYM_ERR_INVALID, "gemm_bf16: M=%d < 0", M);
  if (M == 0) return SYM_OK;
  SYM_REQUIRE(a && w && out, SYM_ERR_INVALID, "gemm_bf16: null pointer argument");
  SYM_REQUIRE(N > 0 && N % 16 == 0, SYM_ERR_UNSUPPORTED,
              "gemm_bf16: N=%d must be a positive multiple of 16", N);
  SYM_REQUIRE(K > 0 && K % kTK == 0, SYM_ERR_UNSUPPORTED,
              "gemm_bf16: K=%d must be a positive multiple of %d", K, kTK);
  SYM_REQUIRE((M + kTM - 1) / kTM <= 65535, SYM_ERR_UNSUPPORTED, "gemm_bf16: M=%d too large", M);
  TileArgs p{};
  p.a = (const uint16_t*)a;
  p.w = (const uint16_t*)w;
  p.bias = (const uint16_t*)bias;
  p.residual = residual;
  p.M = M;
  p.N = N;
  p.K = K;
  p.out_bf16 = out_fp32 ? nullptr : (uint16_t*)out;
  p.out_f32 = out_fp32 ? (float*)out : nullptr;
  (void)hipGetLastError();
  hipLaunchKernelGGL((gemm_tile_kernel<kDense>), dim3((N + kTN - 1) / kTN, (M + kTM - 1) / kTM),
                     dim3(kTileThreads), 0, (hipStream_t)stream, p);
  return sym_host::check_launch("gemm_tile_kernel");
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
  SYM_REQUIRE(H > 0 && H % kTK == 0, SYM_ERR_UNSUPPORTED,
              "moe_router_logits_split: H=%d must be a positive multiple of %d", H, kTK);
  SYM_REQUIRE((T + kTM - 1) / kTM <= 65535, SYM_ERR_UNSUPPORTED,
              "moe_router_logits_split: T=%d too large", T);
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
  hipLaunchKernelGGL((gemm_tile_kernel<kDense>), dim3((E + kTN - 1) / kTN, (T + kTM - 1) / kTM, 3),
                     dim3(kTileThreads), 0, (hipStream_t)stream, p);
  return sym_host::check_launch("gemm_tile_kernel");
}

static int check_grouped(const char* what, int T, int H, int I, int rows, int max_segments) {
  SYM_REQUIRE(T >= 0 && rows >= 0, SYM_ERR_INVALID, "%s: T=%d rows=%d", what, T, rows);
  SYM_REQUIRE(H > 0 && H % kTK == 0, SYM_ERR_UNSUPPORTED, "%s: H=%d must be a multiple of %d",
              what, H, kTK);
  SYM_REQUIRE(I > 0 && I % kTK == 0, SYM_ERR_UNSUPPORTED, "%s: I=%d must be a multiple of %d",
              what, I, kTK);
  SYM_REQUIRE(max_segments >= 1 && max_segments <= kMaxGemmSegments, SYM_ERR_INVALID,
              "%s: max_segments=%d out of range", what, max_segments);
  SYM_REQUIRE((long long)rows / kTM + max_segments <= 65535, SYM_ERR_UNSUPPORTED,
              "%s: %d rows too many", what, rows);
  return SYM_OK;
}

extern "C" int sym_moe_gate_up_tiled(const void* x, int T, int H, int I, int rows,
                                     const int32_t* sorted_tokens, const int32_t* seg_expert,
                                     const int32_t* seg_offset, const int32_t* seg_count,
                                     const int32_t* n_segments, int max_segments,
                                     const void* w_gate_up, void* h, void* stream) {
  int rc = check_grouped("moe_gate_up_tiled", T, H, I, rows, max_segments);
  if (rc || rows == 0 || T == 0) return rc;
  SYM_REQUIRE(x && sorted_tokens && seg_expert && seg_offset && seg_count && n_segments &&
                  w_gate_up && h,
              SYM_ERR_INVALID, "moe_gate_up_tiled: null pointer argument");
  TileArgs p{};
  p.a = (const uint16_t*)x;
  p.w = (const uint16_t*)w_gate_up;
  p.sorted_tokens = sorted_tokens;
  p.seg_expert = seg_expert;
  p.seg_offset = seg_offset;
  p.seg_count = seg_count;
  p.n_segments = n_segments;
  p.M = rows;
  p.N = I;
  p.K = H;
  p.out_bf16 = (uint16_t*)h;
  (void)hipGetLastError();
  hipLaunchKernelGGL((gemm_tile_kernel<kGateUp>),
                     dim3((I + 127) / 128, rows / kTM + max_segments), dim3(kTileThreads), 0,
                     (hipStream_t)stream, p);
  return sym_host::check_launch("gemm_tile_kernel");
}

extern "C" int sym_moe_down_tiled(const void* h, int T, int H, int I, int rows,
                                  const int32_t* seg_expert, const int32_t* seg_offset,
                                  const int32_t* seg_count, const int32_t* n_segments,
                                  int max_segments, const void* w_down, void* y, int y_bf16,
                                  void* stream) {
  int rc = check_grouped("moe_down_tiled", T, H, I, rows, max_segments);
  if (rc || rows == 0 || T == 0) return rc;
  SYM_REQUIRE(h && seg_expert && seg_offset && seg_count && n_segments && w_down && y,
              SYM_ERR_INVALID, "moe_down_tiled: null pointer argument");
  TileArgs p{};
  p.a = (const uint16_t*)h;
  p.w = (const uint16_t*)w_down;
  p.seg_expert = seg_expert;
  p.seg_offset = seg_offset;
  p.seg_count = seg_count;
  p.n_segments = n_segments;
  p.M = rows;
  p.N = H;
  p.K = I;
  if (y_bf16) p.out_bf16 = (uint16_t*)y;
  else p.out_f32 = (float*)y;
  (void)hipGetLastError();
  hipLaunchKernelGGL((gemm_tile_kernel<kDown>),
                     dim3((H + kTN - 1) / kTN, rows / kTM + max_segments), dim3(kTileThreads), 0,
                     (hipStream_t)stream, p);
  return sym_host::check_launch("gemm_tile_kernel");
}
