// Prefill: expert-sorted grouped dequant-GEMM on bf16 MFMA (gfx950).
//
// Used when a call routes at least 64 (token, slot) rows, the point where
// the packed module sorts its rows by expert (src/runnel/mlx.py:59-63).
//
//   prefill_hist_kernel,    stable counting sort of the (token, slot) rows
//   prefill_place_kernel    by expert id (mlx-lm _gather_sort order) over
//                           slices of 2048 rows, one per workgroup: bucket
//                           counts per slice, then every workgroup places
//                           its rows; the shared expert's rows appended as
//                           bucket E, out-of-range ids as bucket E + 1; row
//                           and m-tile offsets per bucket and one
//                           descriptor per m-tile.
//   prefill_gemm_kernel     MODE 0 (gate/up): one (m-tile, n-tile of [up;
//                           gate] pairs) per workgroup; the x rows of the
//                           tile staged in LDS (128-row tiles: by LDS-DMA,
//                           three stages ahead), every wave streams its own
//                           up and gate weight rows straight from HBM into
//                           registers, dequantises them to bf16 (fl32(q*s +
//                           b) rounded to nearest even) and feeds
//                           v_mfma_f32_16x16x32_bf16; SwiGLU epilogue, bf16
//                           activations in sorted row order.
//                           MODE 1 (down): the same over the activations
//                           (contiguous in sorted order) and the down bank;
//                           bf16 rows written to their (token, slot) place.
//   prefill_combine_kernel  per token: sum of score * row over the slots and
//                           the gated shared row, residual, bf16.
//
// Tiles are 32 rows (short prefill: memory bound, few rows per expert) or
// 128 rows (long prefill: matrix-core bound).  32-row tiles: a workgroup is
// 8 waves, 4 for the gate/up tiles, each wave owning 32 weight columns;
// 128-row tiles: 4 waves of 64 columns, two workgroups per CU (at least two
// waves per SIMD either way: a single wave per SIMD issues vector
// instructions too slowly to keep the dequantisation beside the MFMAs).
//
// MFMA operand layout (16x16x32 bf16, checked on the device): lane l holds
// A row l % 16 and B column l % 16, k = 8 (l / 16) + [0, 8); D column l % 16,
// rows 4 (l / 16) + [0, 4).  The k index of each lane is remapped so that a
// lane's operands come from one 16-byte load: within a chunk of KC values of
// one row, lane group g = l / 16 owns k = g KC / 4 + [0, KC / 4), and MFMA j
// of the chunk takes k = g KC / 4 + 8 j + [0, 8) for both A and B.
#include <type_traits>
#include <utility>

#include "common.h"
#include "kernels.h"

namespace rmoe {

namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));

constexpr int kSortThreads = 1024;
constexpr int kSortWaves = kSortThreads / 64;
constexpr int kSortRowsPerSlice = 2048;  // rows per sorting workgroup
// up to this many rows one workgroup sorts them all, without the
// histogram pass (a launch of ~4.6 us)
constexpr int kSortOneSliceRows = 8192;
constexpr int kPad = 8;                         // bf16 of padding per LDS row

// K advances in chunks of KC values.  Each lane group g = l / 16 owns KC / 4
// consecutive values of a weight row per chunk, so a chunk reads 128
// contiguous bytes of every row (a whole cache line): 8-bit rows in chunks
// of 128 values, 4-bit rows in chunks of 256 where the A tile still fits
// (32-row tiles over K = H, a multiple of 256), else 128.
template <int BITS, int BM, int MODE>
struct Chunk {
  // 8 waves, except the short prefill's gate/up tiles: 4 waves (64 pairs),
  // four workgroups per CU, so the last partial round of tiles is half as
  // long (the shared expert's tiles make the count just over a round)
  static constexpr int THREADS = BM == 32 && MODE == 0 ? 256 : 512;
  static constexpr int QPW = 2;                        // 16-column blocks per wave
  static constexpr int MIN_WAVES = BM == 32 ? 4 : 2;   // waves per SIMD (registers)
  static constexpr int KC = BITS == 8 ? 128 : ((BM == 32 && MODE == 0) ? 256 : 128);
  static constexpr int NJ = KC / 32;                   // MFMAs per chunk
  static constexpr int WORDS = KC * BITS / 32;         // u32 per row per chunk
  static constexpr int LANE_WORDS = WORDS / 4;         // u32 per lane per row
  static constexpr int LPC = LANE_WORDS / 4;           // 16-byte loads per lane per row
  static constexpr int ROW = KC + kPad;                // LDS row (bf16)
  // A stages in LDS: down (K = I, short) keeps up to four chunks, the whole
  // K of I = 512, resident; gate/up double-buffers
  static constexpr int STAGES = MODE == 1 ? 4 : 2;
  static constexpr int PIECES = BM * KC / 8;           // 16-byte A pieces
  static constexpr int PPT = PIECES / THREADS;         // pieces per thread
  static_assert(PIECES % THREADS == 0, "A tile must split evenly");
};

__device__ __forceinline__ uint32_t pack_bf16x2(float a, float b) {
  const f32x2_t f = {a, b};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(f, bf16x2_t));
}

__device__ __forceinline__ uint32_t word_of(const uint4 v, int c) {
  return c == 0 ? v.x : c == 1 ? v.y : c == 2 ? v.z : v.w;
}
// Word i & 3 of v without indexing the vector (a run-time index would put
// it in scratch memory).
__device__ __forceinline__ uint32_t word4(const u32x4& v, int i) {
  i &= 3;
  return i == 0 ? v.x : i == 1 ? v.y : i == 2 ? v.z : v.w;
}

// The bf16 MFMA fragment j (8 consecutive k) of a lane's weight slice (LPC
// 16-byte loads): bf16(fl32(q s + b)).
// 4 bits: the codes, split into bytes, go through the fp8 (OCP e4m3)
// conversion: a byte 0..15 is e4m3 q 2^-9 (codes 0-7 subnormal, 8-15 with
// exponent 1), so scaled by 2^9 it is q exactly, two codes per instruction
// instead of one byte conversion each (checked for every code and byte
// position on the device; dense 65536 x 1024 x 2048 4-bit GEMM 283 -> 272
// us).
template <int BITS, int LPC>
__device__ __forceinline__ bf16x8_t dequant_frag(const uint4 (&w)[LPC], int j, float s,
                                                 float b) {
  u32x4 d;
  if constexpr (BITS == 8) {
    const uint32_t w0 = word_of(w[j >> 1], 2 * (j & 1));
    const uint32_t w1 = word_of(w[j >> 1], 2 * (j & 1) + 1);
    d.x = pack_bf16x2(fmaf((float)(w0 & 0xFFu), s, b), fmaf((float)((w0 >> 8) & 0xFFu), s, b));
    d.y = pack_bf16x2(fmaf((float)((w0 >> 16) & 0xFFu), s, b), fmaf((float)(w0 >> 24), s, b));
    d.z = pack_bf16x2(fmaf((float)(w1 & 0xFFu), s, b), fmaf((float)((w1 >> 8) & 0xFFu), s, b));
    d.w = pack_bf16x2(fmaf((float)((w1 >> 16) & 0xFFu), s, b), fmaf((float)(w1 >> 24), s, b));
  } else {
    const uint32_t wj = word_of(w[j >> 2], j & 3);
    const uint32_t lo = wj & 0x0F0F0F0Fu;         // codes 0, 2, 4, 6
    const uint32_t hi = (wj >> 4) & 0x0F0F0F0Fu;  // codes 1, 3, 5, 7
    const f32x2_t l0 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp8(lo, 512.0f, false);
    const f32x2_t l1 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp8(lo, 512.0f, true);
    const f32x2_t h0 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp8(hi, 512.0f, false);
    const f32x2_t h1 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp8(hi, 512.0f, true);
    d.x = pack_bf16x2(fmaf(l0.x, s, b), fmaf(h0.x, s, b));
    d.y = pack_bf16x2(fmaf(l0.y, s, b), fmaf(h0.y, s, b));
    d.z = pack_bf16x2(fmaf(l1.x, s, b), fmaf(h1.x, s, b));
    d.w = pack_bf16x2(fmaf(l1.y, s, b), fmaf(h1.y, s, b));
  }
  return __builtin_bit_cast(bf16x8_t, d);
}

__device__ __forceinline__ f32x4_t mfma(const bf16x8_t a, const bf16x8_t b, const f32x4_t c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

// Work item of this workgroup: (n-tile, bucket, rows).  Returns false when
// the workgroup has nothing to do.
struct Tile {
  int n, bucket, row0, nrows;
};

// Items are (m-tile, n-tile) with n innermost, cut into 8 contiguous runs,
// one per XCD (workgroup i runs on XCD i % 8): the n-tiles of one m-tile
// share its A rows in that XCD's L2, and the m-tiles of one expert share
// its weight columns there.  For 128-row tiles the sort lists the full
// m-tiles first and the partial ones (each bucket's last) after them, and
// each XCD takes its run of full items before its run of partial ones: the
// cheap partial tiles fill the last round instead of a full tile starting
// late (8192 tokens: down 255.9 -> 246.6 us).  The partial m-tiles are
// dealt to the XCDs in turn, largest first, so each XCD ends on its
// smallest ones.
__device__ __forceinline__ bool decode_tile(const PrefillArgs& p, int nt, Tile& t) {
  const int xcd = blockIdx.x & 7;
  const int slot = blockIdx.x >> 3;
  if (p.dense) {
    const int MT = (p.T + p.bm - 1) / p.bm;
    const int total = nt * MT;
    const int L = (total + 7) >> 3;
    if (slot >= L) return false;
    const int item = xcd * L + slot;
    if (item >= total) return false;
    const int m = item / nt;
    t.n = item - m * nt;
    // rows m bm .. of the one bank, in order
    t.bucket = 0;
    t.row0 = m * p.bm;
    t.nrows = min(p.bm, p.T - t.row0);
    return true;
  }
  const int mf = p.tile_offs[p.E + 1];  // full m-tiles
  const int mp = p.tile_offs[p.E + 2] - mf;
  const int nf = nt * mf;
  const int lf = (nf + 7) >> 3;
  int m;
  if (slot < lf) {
    const int item = xcd * lf + slot;
    if (item >= nf) return false;
    m = item / nt;
    t.n = item - m * nt;
  } else {
    // partial m-tiles (largest first) dealt to the XCDs in turn, the
    // n-tiles of one m-tile together
    const int s2 = slot - lf;
    const int j = s2 / nt;
    if (xcd + 8 * j >= mp) return false;
    m = mf + xcd + 8 * j;
    t.n = s2 - j * nt;
  }
  const int4 d = reinterpret_cast<const int4*>(p.tile_desc)[m];
  t.bucket = d.x;
  t.row0 = d.y;
  t.nrows = d.z;
  return true;
}

}  // namespace

// ------------------------------------------------------------------- sort
// Rows r = t K + j are cut into contiguous slices, one per workgroup, and
// each slice into contiguous runs, one per wave: a row's place in its
// bucket is (rows of the bucket in earlier slices) + (in earlier runs of
// its slice) + (earlier in its run), so the order within a bucket is the
// row order (stable).

// This workgroup's slice [*r0, *r1) of the n rows.
__device__ __forceinline__ void sort_slice(int n, int nw, int w, int& r0, int& r1) {
  const int per = ((n + nw - 1) / nw + 63) & ~63;
  r0 = min(n, w * per);
  r1 = min(n, r0 + per);
}

__device__ __forceinline__ int bucket_of(const PrefillArgs& p, int r) {
  const int e = p.idx[r];
  return (unsigned)e < (unsigned)p.E ? e : p.E + 1;
}

// Pass 1: rows per bucket of each slice -> hist[slice][bucket].
__global__ __launch_bounds__(kSortThreads) void prefill_hist_kernel(const PrefillArgs p) {
  const int NB = p.E + 2;
  __shared__ int s_hist[kPrefillMaxExperts + 2];
  const int tid = threadIdx.x;
  for (int b = tid; b < NB; b += kSortThreads) s_hist[b] = 0;
  __syncthreads();
  int r0, r1;
  sort_slice(p.T * p.K, gridDim.x, blockIdx.x, r0, r1);
  // two rows per thread per step, both loads issued before either is used
  for (int r = r0 + tid; r < r1; r += 2 * kSortThreads) {
    const int ra = r, rb = r + kSortThreads;
    const int ea = bucket_of(p, ra), eb = bucket_of(p, min(rb, r1 - 1));
    issue_fence();
    atomicAdd(&s_hist[ea], 1);
    if (rb < r1) atomicAdd(&s_hist[eb], 1);
  }
  __syncthreads();
  for (int b = tid; b < NB; b += kSortThreads) p.hist[blockIdx.x * NB + b] = s_hist[b];
}

// Pass 2: every workgroup scans the bucket totals itself (workgroup 0 also
// publishes the offsets and the m-tile descriptors), then places the rows
// of its slice.
__global__ __launch_bounds__(kSortThreads) void prefill_place_kernel(const PrefillArgs p) {
  const int NB = p.E + 2;  // routed buckets, shared, out-of-range
  const int NW = gridDim.x;
  const int w = blockIdx.x;
  __shared__ int s_hist[kSortWaves * (kPrefillMaxExperts + 2)];
  __shared__ int s_wsum[3][kSortWaves];
  __shared__ int s_shared_off;
  __shared__ int s_full;
  __shared__ int s_cls[8];
  const int tid = threadIdx.x;
  const int wave = tid >> 6;
  const int lane = tid & 63;
  for (int i = tid; i < kSortWaves * NB; i += kSortThreads) s_hist[i] = 0;

  // this workgroup's slice, one run per wave
  const int n = p.T * p.K;
  int r0, r1;
  sort_slice(n, NW, w, r0, r1);
  const int per = ((r1 - r0 + kSortWaves - 1) / kSortWaves + 63) & ~63;
  const int q0 = min(r1, r0 + wave * per);
  const int q1 = min(r1, q0 + per);

  // Per bucket: total rows, rows in earlier slices, full m-tiles and the
  // partial one.  The slices' counts are loaded 16 at a time (a loop of
  // single loads waited for each).
  int rows_b = 0, before_b = 0, full_b = 0, part_b = 0;
  if (tid < NB) {
    if (tid == p.E) {
      rows_b = p.has_shared ? p.T : 0;
    } else if (NW > 1) {
      for (int v0 = 0; v0 < NW; v0 += 16) {
        int c[16];
#pragma unroll
        for (int u = 0; u < 16; ++u) c[u] = p.hist[min(v0 + u, NW - 1) * NB + tid];
#pragma unroll
        for (int u = 0; u < 16; ++u) {
          const int v = v0 + u;
          rows_b += v < NW ? c[u] : 0;
          before_b += v < w ? c[u] : 0;
        }
      }
    }
  }

  // per-wave counts of this wave's run (two chunks of 64 rows per step);
  // the buckets of the first kKeep steps stay in registers for the ranking
  // below (no second round trip for them)
  constexpr int kKeep = 4;
  int kept[2 * kKeep];
  int* my = s_hist + wave * NB;
  __syncthreads();  // the zeroed counts
#pragma unroll
  for (int k = 0; k < kKeep; ++k) {
    const int c0 = q0 + 128 * k;
    kept[2 * k] = kept[2 * k + 1] = 0;
    if (c0 < q1) {
      const int ra = c0 + lane, rb = c0 + 64 + lane;
      const int ea = bucket_of(p, min(ra, q1 - 1)), eb = bucket_of(p, min(rb, q1 - 1));
      issue_fence();
      kept[2 * k] = ea;
      kept[2 * k + 1] = eb;
      if (ra < q1) atomicAdd(&my[ea], 1);
      if (rb < q1) atomicAdd(&my[eb], 1);
    }
  }
  for (int c0 = q0 + 128 * kKeep; c0 < q1; c0 += 128) {
    const int ra = c0 + lane, rb = c0 + 64 + lane;
    const int ea = bucket_of(p, min(ra, q1 - 1)), eb = bucket_of(p, min(rb, q1 - 1));
    issue_fence();
    if (ra < q1) atomicAdd(&my[ea], 1);
    if (rb < q1) atomicAdd(&my[eb], 1);
  }
  __syncthreads();  // every wave's counts
  if (tid < NB) {
    // one slice (no histogram pass): the totals are this workgroup's counts
    if (NW == 1 && tid != p.E)
      for (int v = 0; v < kSortWaves; ++v) rows_b += s_hist[v * NB + tid];
    // 32-row tiles (short prefill, weight-stream bound) keep bucket order:
    // every m-tile counts as full (512 tokens: 254 against 248 us with the
    // partial tiles listed last)
    const bool split = p.bm == kPrefillBM;
    full_b = split ? rows_b / p.bm : (rows_b + p.bm - 1) / p.bm;
    part_b = split && rows_b - full_b * p.bm > 0 ? 1 : 0;
  }
  // inclusive scans of rows_b, full_b and part_b over the buckets: within
  // each wave, then the earlier waves' totals added
  int sr = rows_b, sf = full_b, sp = part_b;
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    const int a = __shfl_up(sr, d, 64);
    const int b = __shfl_up(sf, d, 64);
    const int c = __shfl_up(sp, d, 64);
    if (lane >= d) {
      sr += a;
      sf += b;
      sp += c;
    }
  }
  if (lane == 63) {
    s_wsum[0][wave] = sr;
    s_wsum[1][wave] = sf;
    s_wsum[2][wave] = sp;
  }

  __syncthreads();  // the wave totals
  for (int v = 0; v < wave; ++v) {
    sr += s_wsum[0][v];
    sf += s_wsum[1][v];
    sp += s_wsum[2][v];
  }
  if (tid == NB - 1) s_full = sf;
  __syncthreads();

  if (tid < NB) {
    const int row_off = sr - rows_b;
    if (w == 0) {
      // the full m-tiles in bucket order, then the partial ones
      p.offs[tid] = row_off;
      if (tid == NB - 1) {
        p.offs[NB] = sr;
        p.tile_offs[NB - 1] = sf;  // full m-tiles
        p.tile_offs[NB] = sf + sp;
      }
      const int f0 = sf - full_b;
      for (int i = 0; i < full_b; ++i)
        *reinterpret_cast<int4*>(p.tile_desc + 4 * (f0 + i)) =
            make_int4(tid, row_off + i * p.bm, min(p.bm, rows_b - i * p.bm), 0);
    }
    // per-wave bases of this bucket in this slice
    int base = row_off + before_b;
    if (tid != p.E) {
      for (int v = 0; v < kSortWaves; ++v) {
        const int c = s_hist[v * NB + tid];
        s_hist[v * NB + tid] = base;
        base += c;
      }
    } else {
      s_shared_off = row_off;
    }
  }
  __syncthreads();
  if (w == 0 && p.bm == kPrefillBM) {
    // the partial m-tiles after the full ones, largest first (counting sort
    // by 16-row blocks; the order within a class does not matter)
    if (tid < 8) s_cls[tid] = 0;
    __syncthreads();
    const int rem = rows_b - full_b * p.bm;
    const int cls = 8 - ((rem + 15) >> 4);  // 0: eight blocks
    if (part_b) atomicAdd(&s_cls[cls], 1);
    __syncthreads();
    if (tid == 0) {
      int a = 0;
      for (int c = 0; c < 8; ++c) {
        const int k = s_cls[c];
        s_cls[c] = a;
        a += k;
      }
    }
    __syncthreads();
    if (part_b) {
      const int pos = atomicAdd(&s_cls[cls], 1);
      *reinterpret_cast<int4*>(p.tile_desc + 4 * (s_full + pos)) =
          make_int4(tid, sr - rows_b + full_b * p.bm, rem, 0);
    }
  }
  if (p.has_shared)
    for (int t = w * kSortThreads + tid; t < p.T; t += NW * kSortThreads)
      p.rows[s_shared_off + t] = n + t;

  // Stable ranking: each wave walks its run in order, 64 at a time; the
  // lanes holding one bucket find each other with one ballot per id bit.
  auto rank_chunk = [&](int r, int e, bool v) {
    uint64_t mask = __ballot(v);
#pragma unroll
    for (int b = 0; b < 10; ++b) {
      const bool bit = (e >> b) & 1;
      const uint64_t bal = __ballot(v && bit);
      mask &= bit ? bal : ~bal;
    }
    if (v) {
      const uint64_t below = mask & ((1ull << lane) - 1ull);
      const int pos = my[e] + __popcll(below);
      p.rows[pos] = r;
    }
    // every lane has read its base before the leaders advance them
    __builtin_amdgcn_wave_barrier();
    if (v && (mask >> lane) == 1ull) my[e] += __popcll(mask);
    __builtin_amdgcn_wave_barrier();
  };
#pragma unroll
  for (int k = 0; k < kKeep; ++k) {
    const int c0 = q0 + 128 * k;
    if (c0 < q1) {
      const int ra = c0 + lane, rb = c0 + 64 + lane;
      rank_chunk(ra, ra < q1 ? kept[2 * k] : 0, ra < q1);
      if (c0 + 64 < q1) rank_chunk(rb, rb < q1 ? kept[2 * k + 1] : 0, rb < q1);
    }
  }
  for (int c0 = q0 + 128 * kKeep; c0 < q1; c0 += 128) {
    const int ra = c0 + lane, rb = c0 + 64 + lane;
    const int ea = bucket_of(p, min(ra, q1 - 1)), eb = bucket_of(p, min(rb, q1 - 1));
    issue_fence();
    rank_chunk(ra, ra < q1 ? ea : 0, ra < q1);
    if (c0 + 64 < q1) rank_chunk(rb, rb < q1 ? eb : 0, rb < q1);
  }
}

// ------------------------------------------------------------- epilogue
// The tile's bf16 outputs go through LDS (the A buffers, free once every wave
// has finished its last chunk) so that each row leaves in 16-byte pieces:
// act rows (SwiGLU) in sorted order, or y rows at their (token, slot) place.
// Wave w holds tile columns w 16 QPW + [0, 16 QPW): for gate/up the first
// half of its blocks are up rows and the second half the matching gate rows,
// so a wave's 8 QPW activation columns are local to it.
// Rows are staged in LDS parts of RPP rows each (so[r / RPP]).
template <int MODE, int MB, int QPW, int TN, int THREADS, int RPP>
__device__ __forceinline__ void store_tile(const PrefillArgs& p, const Tile& tile,
                                           const int* s_row, uint16_t* const* so,
                                           const f32x4_t (&acc)[MB][QPW], int mba) {
  constexpr int OS = TN + 8;  // LDS row stride (bf16)
  const int tid = threadIdx.x;
  const int wave = tid >> 6;
  const int col_l = tid & 15;
  const int kg = (tid & 63) >> 4;
  __syncthreads();
#pragma unroll
  for (int mb = 0; mb < MB; ++mb) {
    if (mb >= mba) continue;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int r = mb * 16 + kg * 4 + i;
      if constexpr (MODE == 0) {
#pragma unroll
        for (int h = 0; h < QPW / 2; ++h) {
          const int c = wave * (8 * QPW) + h * 16 + col_l;
          const float up = round_bf16(acc[mb][h][i]);
          const float gate = round_bf16(acc[mb][QPW / 2 + h][i]);
          so[r / RPP][(r % RPP) * OS + c] = (uint16_t)f32_to_bf16(silu(gate) * up);
        }
      } else {
#pragma unroll
        for (int qq = 0; qq < QPW; ++qq) {
          const int c = wave * (16 * QPW) + qq * 16 + col_l;
          so[r / RPP][(r % RPP) * OS + c] = (uint16_t)f32_to_bf16(acc[mb][qq][i]);
        }
      }
    }
  }
  __syncthreads();
  constexpr int PR = TN / 8;  // 16-byte pieces per row
  for (int pi = tid; pi < tile.nrows * PR; pi += THREADS) {
    const int r = pi / PR;
    const int c8 = pi - r * PR;
    const uint4 v = *reinterpret_cast<const uint4*>(so[r / RPP] + (r % RPP) * OS + c8 * 8);
    uint16_t* dst = MODE == 0 ? p.act + (size_t)(tile.row0 + r) * p.I
                              : p.y + (size_t)s_row[r] * p.H;
    *reinterpret_cast<uint4*>(dst + tile.n * TN + c8 * 8) = v;
  }
}

// ------------------------------------------------------------ grouped GEMM
// MODE 0: gate/up.  A = x rows of the tile's tokens (K = H); the wave's four
//         B column blocks are up rows c, c + 16 and gate rows I + c, I + c +
//         16 of 32 pairs c; SwiGLU epilogue -> act[sorted row].
// MODE 1: down.  A = act rows (contiguous in sorted order, K = I); B column
//         blocks are 4 x 16 consecutive output columns; -> y[source row].
// Rows of a partial tile are zero in LDS; only the 16-row blocks that hold
// rows are multiplied (two specialisations: all blocks, or the first half).
template <int BITS, int BM, int MODE>
struct Gemm {
  using C = Chunk<BITS, BM, MODE>;
  static constexpr int MB = BM / 16;
  // columns per workgroup: gate/up pairs (two rows each) or down columns
  static constexpr int TN = (C::THREADS / 64) * 16 * C::QPW / (MODE == 0 ? 2 : 1);

  const PrefillArgs& p;
  const Tile& tile;
  uint16_t (*s_a)[BM * C::ROW];  // [C::STAGES]
  const int* s_row;
  int tid, wave, lane, col_l, kg, K;
  QW q;
  static constexpr int QPW = C::QPW;
  static constexpr int THREADS = C::THREADS;
  static constexpr int MIN_WAVES = C::MIN_WAVES;
  static constexpr int LDS = C::STAGES * BM * C::ROW;  // bf16
  size_t brow[QPW];
  const uint32_t* wptr[QPW];
  // Scales and biases come in blocks of 8 groups (16 bytes of a row) through
  // bounds-checked buffer resources: lane l loads the block of the wave's
  // column (l / 16) % QPW, l % 16 and ds_bpermute hands every lane the
  // values of its column (one load per array and CPB chunks instead of a
  // 2-byte load per column block and chunk, each touching 16 rows).
  static constexpr int CPB = 8 * 64 / C::KC;  // chunks per block
  __amdgpu_buffer_rsrc_t rs, rb;
  uint32_t soff;

  __device__ Gemm(const PrefillArgs& p_, const Tile& t_, uint16_t* lds, const int* srow)
      : p(p_), tile(t_), s_a(reinterpret_cast<uint16_t (*)[BM * C::ROW]>(lds)), s_row(srow) {
    tid = threadIdx.x;
    wave = tid >> 6;
    lane = tid & 63;
    col_l = lane & 15;
    kg = lane >> 4;
    const bool shared = tile.bucket == p.E;
    const size_t e = shared ? 0 : (size_t)tile.bucket;
    K = MODE == 0 ? p.H : p.I;
    const int WPR = K * BITS / 32;
#pragma unroll
    for (int qq = 0; qq < QPW; ++qq) {
      if constexpr (MODE == 0) {
        // blocks 0 .. QPW/2-1: up rows of this wave's pairs, then gate rows
        q = shared ? p.sgu : p.gu;
        const int c = tile.n * TN + wave * (8 * QPW) + (qq % (QPW / 2)) * 16 + col_l;
        brow[qq] = e * 2 * p.I + (size_t)(c + (qq / (QPW / 2)) * p.I);
      } else {
        q = shared ? p.sdn : p.dn;
        const int c = tile.n * TN + wave * (16 * QPW) + qq * 16 + col_l;
        brow[qq] = e * p.H + (size_t)c;
      }
      wptr[qq] = q.w + brow[qq] * WPR + kg * C::LANE_WORDS;
    }
    const size_t G = (size_t)K / 64;
    const size_t rows = (MODE == 0 ? 2 * (size_t)p.I : (size_t)p.H) * (shared ? 1 : (size_t)p.E);
    rs = __builtin_amdgcn_make_buffer_rsrc((void*)q.s, (short)0, (int)(rows * G * 2), 0x00020000);
    rb = __builtin_amdgcn_make_buffer_rsrc((void*)q.b, (short)0, (int)(rows * G * 2), 0x00020000);
    // lanes 32-63 hold the same blocks one word (two groups) on, for chunks
    // whose lane groups need two different words (KC = 256)
    size_t br = brow[0];  // (selected, not indexed: an index would put the object in memory)
#pragma unroll
    for (int qq = 1; qq < QPW; ++qq)
      if (((lane >> 4) % QPW) == qq) br = brow[qq];
    soff = (uint32_t)(br * G * 2) + (C::KC > 128 && lane >= 32 ? 4 : 0);
  }

  // This thread's A pieces: row base pointers, fixed for the whole tile.
  // Rows past the tile's end read a row that exists (x row of token 0, or
  // the tile's last row) and are stored as zeros, so every load is
  // unconditional and the compiler can count the loads still in flight.
  __device__ __forceinline__ void a_rows(const uint16_t* (&src)[C::PPT],
                                         bool (&live)[C::PPT]) const {
#pragma unroll
    for (int j = 0; j < C::PPT; ++j) {
      const int pi = tid + THREADS * j;
      const int r = pi / (C::KC / 8);
      const int c8 = pi - r * (C::KC / 8);
      live[j] = r < tile.nrows;
      if constexpr (MODE == 0)
        src[j] = p.x + (size_t)s_row[r] * p.H + c8 * 8;  // s_row is 0 past the end
      else
        src[j] = p.act + (size_t)(tile.row0 + min(r, tile.nrows - 1)) * p.I + c8 * 8;
    }
  }

  __device__ __forceinline__ void load_a(int ch, const uint16_t* const (&src)[C::PPT],
                                         uint4 (&ar)[C::PPT]) const {
#pragma unroll
    for (int j = 0; j < C::PPT; ++j) ar[j] = load16(src[j] + ch * C::KC);
  }
  // Only the live rows (a memory-bound short tile does not fetch its padding).
  __device__ __forceinline__ void load_a_live(int ch, const uint16_t* const (&src)[C::PPT],
                                              const bool (&live)[C::PPT],
                                              uint4 (&ar)[C::PPT]) const {
#pragma unroll
    for (int j = 0; j < C::PPT; ++j) {
      ar[j] = make_uint4(0, 0, 0, 0);
      if (live[j]) ar[j] = load16(src[j] + ch * C::KC);
    }
  }
  __device__ __forceinline__ void store_a(int buf, const uint4 (&ar)[C::PPT],
                                          const bool (&live)[C::PPT]) const {
#pragma unroll
    for (int j = 0; j < C::PPT; ++j) {
      const int pi = tid + THREADS * j;
      const int r = pi / (C::KC / 8);
      const int c8 = pi - r * (C::KC / 8);
      // rows past the tile's end hold a copy of a live row (or zeros, for
      // the short tiles that load live rows only): they only reach output
      // rows the epilogue does not store, so no select is needed
      *reinterpret_cast<uint4*>(&s_a[buf][r * C::ROW + c8 * 8]) = ar[j];
    }
  }
  __device__ __forceinline__ void load_b(int ch, uint4 (&w)[QPW][C::LPC]) const {
#pragma unroll
    for (int qq = 0; qq < QPW; ++qq)
#pragma unroll
      for (int l = 0; l < C::LPC; ++l) w[qq][l] = load16_stream(wptr[qq] + ch * C::WORDS + 4 * l);
  }
  // Block k (groups 8 k .. 8 k + 7) of the lane's block row; groups past the
  // row's end are never used (and past the array read as zeros).
  __device__ __forceinline__ void load_blk(int k, u32x4& bs, u32x4& bb) const {
    bs = __builtin_amdgcn_raw_buffer_load_b128(rs, soff, k * 16, 0);
    bb = __builtin_amdgcn_raw_buffer_load_b128(rb, soff, k * 16, 0);
  }
  // Scale and bias of chunk cip of a block (a constant once unrolled) for
  // this lane's column and group: the lane's group is the chunk's first plus
  // kg KC / 256 (KC / 4 values per lane group, 64 per group).
  __device__ __forceinline__ void scales(int cip, const u32x4& bs, const u32x4& bb,
                                         float (&sc)[QPW], float (&bi)[QPW]) const {
    const int gi = cip * (C::KC / 64) + ((kg * C::KC) >> 8);
    const int sh = (gi & 1) * 16;
#pragma unroll
    for (int qq = 0; qq < QPW; ++qq) {
      const int from = 4 * (qq * 16 + col_l);
      uint32_t vs, vb;
      if constexpr (C::KC <= 128) {
        // both groups of the chunk in word cip
        const int w = cip * (C::KC / 128);
        vs = (uint32_t)__builtin_amdgcn_ds_bpermute(from, (int)word4(bs, w));
        vb = (uint32_t)__builtin_amdgcn_ds_bpermute(from, (int)word4(bb, w));
      } else {
        // four groups in words 2 cip, 2 cip + 1: lane groups 2, 3 read word
        // 2 cip of the shifted copy, which is word 2 cip + 1
        const int w = 2 * cip;
        const int from2 = from + (kg >> 1) * 128;
        vs = (uint32_t)__builtin_amdgcn_ds_bpermute(from2, (int)word4(bs, w));
        vb = (uint32_t)__builtin_amdgcn_ds_bpermute(from2, (int)word4(bb, w));
      }
      sc[qq] = bf16_to_f32((vs >> sh) & 0xFFFFu);
      bi[qq] = bf16_to_f32((vb >> sh) & 0xFFFFu);
    }
  }

  // One chunk of KC: NJ MFMA steps over the first MBA row blocks.  The LDS
  // reads and the dequantisation of step j + 1 are interleaved with the
  // MFMAs of step j, so the matrix core, the vector ALU and the LDS of the
  // SIMD work at the same time.
  template <int MBA>
  __device__ __forceinline__ void chunk(int buf, const uint4 (&w)[QPW][C::LPC],
                                        const float (&s)[QPW], const float (&b)[QPW],
                                        f32x4_t (&acc)[MB][QPW]) const {
    const uint16_t* sa = &s_a[buf][col_l * C::ROW + kg * (C::KC / 4)];
    auto read_a = [&](int j, bf16x8_t (&a)[MBA]) {
#pragma unroll
      for (int mb = 0; mb < MBA; ++mb)
        a[mb] = __builtin_bit_cast(
            bf16x8_t, *reinterpret_cast<const u32x4*>(sa + mb * 16 * C::ROW + 8 * j));
    };
    bf16x8_t a[MBA], bf[QPW];
    read_a(0, a);
#pragma unroll
    for (int qq = 0; qq < QPW; ++qq) bf[qq] = dequant_frag<BITS, C::LPC>(w[qq], 0, s[qq], b[qq]);
#pragma unroll
    for (int j = 0; j < C::NJ; ++j) {
      bf16x8_t na[MBA], nbf[QPW];
      if (j + 1 < C::NJ) {
        read_a(j + 1, na);
#pragma unroll
        for (int qq = 0; qq < QPW; ++qq)
          nbf[qq] = dequant_frag<BITS, C::LPC>(w[qq], j + 1, s[qq], b[qq]);
      }
#pragma unroll
      for (int mb = 0; mb < MBA; ++mb)
#pragma unroll
        for (int qq = 0; qq < QPW; ++qq) acc[mb][qq] = mfma(a[mb], bf[qq], acc[mb][qq]);
      if (j + 1 < C::NJ) {
        // per MFMA: one MFMA, a share of the next step's LDS reads and of
        // its dequantisation
        constexpr int kValuPer = (BITS == 8 ? 20 : 28) / MBA + 1;
#pragma unroll
        for (int i = 0; i < QPW * MBA; ++i) {
          __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
          if (i % QPW == 0) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
          __builtin_amdgcn_sched_group_barrier(0x002, kValuPer, 0);
        }
#pragma unroll
        for (int mb = 0; mb < MBA; ++mb) a[mb] = na[mb];
#pragma unroll
        for (int qq = 0; qq < QPW; ++qq) bf[qq] = nbf[qq];
      }
    }
  }

  // 32-row tiles (registers for four waves per SIMD): everything one chunk
  // ahead.
  template <int MBA>
  __device__ void run1(f32x4_t (&acc)[MB][QPW]) const {
    const int nch = K / C::KC;
    const uint16_t* asrc[C::PPT];
    bool live[C::PPT];
    a_rows(asrc, live);
    uint4 ar[C::PPT];
    uint4 bw[QPW][C::LPC];
    u32x4 bs, bb;
    float sc[QPW], bi[QPW];
    load_blk(0, bs, bb);
    load_b(0, bw);
    load_a_live(0, asrc, live, ar);
    store_a(0, ar, live);
    __syncthreads();
    for (int ch0 = 0; ch0 < nch; ch0 += CPB) {
#pragma unroll
      for (int i = 0; i < CPB; ++i) {
        const int ch = ch0 + i;
        if (ch < nch) {
          const int nx = min(ch + 1, nch - 1);
          uint4 nw[QPW][C::LPC];
          load_b(nx, nw);
          load_a_live(nx, asrc, live, ar);
          scales(i, bs, bb, sc, bi);
          // the next block into the same registers, in flight during the
          // block's last chunk (the chunk's closing barrier waits for it)
          if (i == CPB - 1) load_blk(ch0 / CPB + 1, bs, bb);
          chunk<MBA>(ch & 1, bw, sc, bi, acc);
          store_a((ch & 1) ^ 1, ar, live);
          __syncthreads();
#pragma unroll
          for (int qq = 0; qq < QPW; ++qq)
#pragma unroll
            for (int l = 0; l < C::LPC; ++l) bw[qq][l] = nw[qq][l];
        }
      }
    }
  }

  // Down with K <= STAGES chunks: every A chunk is loaded and stored once up
  // front (one barrier for the whole tile); weights stream two chunks ahead;
  // the scales and biases of at most 8 groups are one block.
  template <int MBA>
  __device__ void run_full(f32x4_t (&acc)[MB][QPW]) const {
    static_assert(C::STAGES <= CPB, "one scale / bias block covers the tile's K");
    const int nch = K / C::KC;
    const uint16_t* asrc[C::PPT];
    bool live[C::PPT];
    a_rows(asrc, live);
    uint4 bw[2][QPW][C::LPC];
    u32x4 bs, bb;
    float sc[QPW], bi[QPW];
    uint4 ar[C::STAGES][C::PPT];
#pragma unroll
    for (int c = 0; c < C::STAGES; ++c)
      if (c < nch) load_a_live(min(c, nch - 1), asrc, live, ar[c]);
    load_blk(0, bs, bb);
    load_b(0, bw[0]);
    load_b(min(1, nch - 1), bw[1]);
#pragma unroll
    for (int c = 0; c < C::STAGES; ++c)
      if (c < nch) store_a(c, ar[c], live);
    __syncthreads();
#pragma unroll
    for (int c = 0; c < C::STAGES; ++c) {
      if (c >= nch) break;
      const int S = c & 1;
      scales(c, bs, bb, sc, bi);
      chunk<MBA>(c, bw[S], sc, bi, acc);
      load_b(min(c + 2, nch - 1), bw[S]);
    }
  }

  template <int MBA>
  __device__ void run(f32x4_t (&acc)[MB][QPW]) const {
    static_assert(BM == 32, "128-row tiles run on the Wide engine");
    if constexpr (MODE == 1) {
      if (K <= C::STAGES * C::KC) {
        run_full<MBA>(acc);
        return;
      }
    }
    run1<MBA>(acc);
  }

  __device__ void epilogue(const f32x4_t (&acc)[MB][QPW], int mba) const {
    static_assert(BM * (TN + 8) <= C::STAGES * BM * C::ROW, "output tile fits in the A buffers");
    uint16_t* so[1] = {&s_a[0][0]};
    store_tile<MODE, MB, QPW, TN, THREADS, BM>(p, tile, s_row, so, acc, mba);
  }
};

// ------------------------------------------------------- 128-row tiles
// Four waves per workgroup, two workgroups per CU.  Each wave owns 64 weight
// columns (four 16-column blocks) of the 128-row tile, so every A fragment
// read from LDS feeds four MFMAs: half the LDS reads per MFMA of 32-column
// waves, which at the full matrix-core rate needed all of the LDS bandwidth.
//
// A reaches LDS without passing through registers: global_load_lds_dwordx4
// writes 16 bytes per lane at (wave-uniform base + 16 lane), and each lane
// fetches the piece that belongs at its position.  Four A stages of 64 k
// values (16 KB each) are loaded three stages ahead; each stage ends with a
// wait for this wave's copy of the next stage and a bare barrier, after which
// that stage has landed for every wave (a fenced __syncthreads would wait
// for every load in flight, the weights and the later stages included).  The
// wait is counted: every stage issues the same loads in the same order, the
// stages past the end reloading the last one into a buffer nobody reads, so
// after the copy of stage c + 1 exactly 2 ND + NBL loads have been issued at
// the end of stage c (fewer only in the first stage, where waiting for the
// extra ones costs nothing: they are the weights in use).  Sched barriers
// keep the compiler from reordering the load groups.
//
// Weights (B) stream into registers one chunk ahead (KB values: 128 at 4
// bits, 64 at 8; 16 bytes of each of the wave's 4 columns per lane).
//
// LDS stage layout: row r holds 8 slots of 16 bytes; slot sl of row r sits at
// position 8 r + (sl ^ f(r)), f(r) = (r & 7) ^ ((r >> 3) & 1).  An operand
// read takes one slot (two, for the two lane groups of a half wave) of rows
// r0 .. r0 + 15: any 8, 16 or 32 of its lanes then fall on distinct 16-byte
// bank groups, whether the LDS has 64 or 128 banks (the plain XOR with r / 2
// left 32-lane passes two-way conflicted).  Slot sl = 2 kg + j
// holds the 8 k values that lane group kg feeds to k-step j of the stage:
// k = (KB / 4) kg + 8 (2 h + j) + [0, 8) of the weight chunk, h = the
// stage's index within its chunk, the k of the lane's B fragment.
template <int BITS, int MODE>
struct Wide {
  static constexpr int BM = 128, MB = BM / 16, QPW = 4, WAVES = 4, THREADS = 64 * WAVES;
  static constexpr int MIN_WAVES = 2;
  static constexpr int TN = WAVES * 16 * QPW / (MODE == 0 ? 2 : 1);
  static constexpr int KB = BITS == 4 ? 128 : 64;  // weight values per chunk
  static constexpr int SB = KB / 64;               // A stages per weight chunk
  static constexpr int STAGE = BM * 64;            // bf16 per A stage
  static constexpr int NBUF = 4;
  // each buffer also holds a quarter of the output tile (32 rows) in the epilogue
  static constexpr int BUF = STAGE > (BM / NBUF) * (TN + 8) ? STAGE : (BM / NBUF) * (TN + 8);
  static constexpr int NBL = QPW;  // load instructions per weight chunk
  // Scales and biases come in blocks of 8 groups (16 bytes of a row), one
  // block per PS stages: each lane loads the block of one of the wave's 64
  // columns (lane l: column block l / 16, column l % 16) and ds_bpermute
  // hands every lane the values of its column.  One block load per array
  // and period replaces a 2-byte load per column block and chunk, each of
  // which touched 16 rows: the memory pipeline, not the bytes, was the cost.
  static constexpr int PS = 8 * 64 / KB * SB;  // stages per block (8 groups)
  static constexpr int NSB = 2;                // block load instructions
  // A fragments read ahead of their MFMAs (dense 65536 x 1024 x 2048 4-bit
  // GEMM: each pair read just before its MFMAs 276 us, 2 ahead 255-260, 3
  // ahead 254-261, 4 ahead 261-326)
  static constexpr int PF = 2;

  struct Bw {
    u32x4 w[QPW];
  };

  const PrefillArgs& p;
  const Tile& tile;
  uint16_t *l0, *l1, *l2, *l3;  // four distinct LDS arrays
  const int* s_row;
  int tid, wave, lane, kg, nst, nbc;
  // Buffer resources based at the tile's expert (offsets stay 32-bit) and
  // this lane's byte offsets in them, per column block.
  __amdgpu_buffer_rsrc_t rw, rs, rb, ra;
  uint32_t woff[QPW];
  uint32_t soff;  // this lane's block row: column block lane / 16, column lane % 16

  __device__ Wide(const PrefillArgs& p_, const Tile& t_, uint16_t* l0_, uint16_t* l1_,
                  uint16_t* l2_, uint16_t* l3_, const int* srow)
      : p(p_), tile(t_), l0(l0_), l1(l1_), l2(l2_), l3(l3_), s_row(srow) {
    tid = threadIdx.x;
    wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    lane = tid & 63;
    kg = lane >> 4;
    const int col_l = lane & 15;
    const bool shared = tile.bucket == p.E;
    const size_t e = shared ? 0 : (size_t)tile.bucket;
    const int K = MODE == 0 ? p.H : p.I;
    const int N = MODE == 0 ? 2 * p.I : p.H;  // weight rows per expert
    nst = K / 64;
    nbc = K / KB;
    const QW q = MODE == 0 ? (shared ? p.sgu : p.gu) : (shared ? p.sdn : p.dn);
    const size_t WPR = (size_t)K * BITS / 32;  // u32 per weight row
    const size_t G = (size_t)K / 64;           // groups per weight row
    rw = __builtin_amdgcn_make_buffer_rsrc((void*)(q.w + e * N * WPR), (short)0,
                                           (int)(N * WPR * 4), 0x00020000);
    rs = __builtin_amdgcn_make_buffer_rsrc((void*)(q.s + e * N * G), (short)0, (int)(N * G * 2),
                                           0x00020000);
    rb = __builtin_amdgcn_make_buffer_rsrc((void*)(q.b + e * N * G), (short)0, (int)(N * G * 2),
                                           0x00020000);
    if constexpr (MODE == 0)
      ra = __builtin_amdgcn_make_buffer_rsrc((void*)p.x, (short)0, (int)((size_t)p.T * p.H * 2),
                                             0x00020000);
    else
      ra = __builtin_amdgcn_make_buffer_rsrc((void*)(p.act + (size_t)tile.row0 * p.I), (short)0,
                                             tile.nrows * p.I * 2, 0x00020000);
#pragma unroll
    for (int qq = 0; qq < QPW; ++qq) {
      uint32_t row;  // weight row within the expert
      if constexpr (MODE == 0) {
        // blocks 0, 1: up rows of the wave's 32 pairs; 2, 3: their gate rows
        row = tile.n * TN + wave * 32 + (qq & 1) * 16 + col_l + (qq >> 1) * p.I;
      } else {
        row = tile.n * TN + wave * 64 + qq * 16 + col_l;
      }
      woff[qq] = (row * (uint32_t)WPR + kg * 4) * 4;
    }
    {
      const int qq = lane >> 4;
      uint32_t row;
      if constexpr (MODE == 0)
        row = tile.n * TN + wave * 32 + (qq & 1) * 16 + col_l + (qq >> 1) * p.I;
      else
        row = tile.n * TN + wave * 64 + qq * 16 + col_l;
      soff = row * (uint32_t)G * 2;
    }
  }

  // Weight chunk b of the wave's columns (16 bytes per lane and column).
  __device__ __forceinline__ void load_b(int b, Bw& r) const {
    const int wb = b * 64;  // bytes into each row's words
#pragma unroll
    for (int qq = 0; qq < QPW; ++qq)
      r.w[qq] = __builtin_amdgcn_raw_buffer_load_b128(rw, woff[qq], wb, 0);
  }
  // Scale and bias block k (groups 8 k .. 8 k + 7) of the lane's block row;
  // groups past the row's end are never used.
  __device__ __forceinline__ void load_blk(int k, u32x4& bs, u32x4& bb) const {
    bs = __builtin_amdgcn_raw_buffer_load_b128(rs, soff, k * 16, 0);
    bb = __builtin_amdgcn_raw_buffer_load_b128(rb, soff, k * 16, 0);
  }
  // The scale and bias (as floats) of chunk CIP of a block, for this lane's
  // column and group: word (group / 2) from the lane that holds its column.
  template <int CIP>
  __device__ __forceinline__ void scales(const u32x4& bs, const u32x4& bb, float (&sc)[QPW],
                                         float (&bi)[QPW]) const {
    constexpr int G0 = CIP * KB / 64;  // first group of the chunk within the block
    const int gi = BITS == 4 ? G0 + (kg >> 1) : G0;
    const int sh = (gi & 1) * 16;
#pragma unroll
    for (int qq = 0; qq < QPW; ++qq) {
      const int from = 4 * (qq * 16 + (lane & 15));
      const uint32_t vs = (uint32_t)__builtin_amdgcn_ds_bpermute(from, (int)bs[G0 >> 1]);
      const uint32_t vb = (uint32_t)__builtin_amdgcn_ds_bpermute(from, (int)bb[G0 >> 1]);
      sc[qq] = bf16_to_f32((vs >> sh) & 0xFFFFu);
      bi[qq] = bf16_to_f32((vb >> sh) & 0xFFFFu);
    }
  }

  // DMA instruction i of a stage covers tile rows 32 i + 8 wave + [0, 8);
  // lane l writes slot position l & 7 of row 32 i + 8 wave + l / 8.  Byte
  // offsets of the lane's pieces in the A resource.
  __device__ __forceinline__ void a_src(uint32_t (&src)[MB / 2]) const {
    const int rl = 8 * wave + (lane >> 3);  // row within each 32-row group
    const int sl = (lane & 7) ^ ((rl & 7) ^ ((rl >> 3) & 1));
    const int koff = BITS == 4 ? (4 * (sl >> 1) + (sl & 1)) * 8 : sl * 8;
#pragma unroll
    for (int i = 0; i < MB / 2; ++i) {
      const int r = 32 * i + rl;
      if constexpr (MODE == 0)
        src[i] = ((uint32_t)s_row[r] * p.H + koff) * 2;  // s_row is token 0 past the end
      else
        src[i] = ((uint32_t)min(r, tile.nrows - 1) * p.I + koff) * 2;
    }
  }

  // First k value of stage c in a row (the pieces of a stage start there).
  __device__ __forceinline__ static int stage_col(int c) {
    return BITS == 4 ? (c >> 1) * 128 + (c & 1) * 16 : c * 64;
  }

  template <int ND>
  __device__ __forceinline__ void dma(uint16_t* buf, int c, const uint32_t (&src)[MB / 2]) const {
    const int col = stage_col(c) * 2;
#pragma unroll
    for (int i = 0; i < ND; ++i)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(
          ra, (__attribute__((address_space(3))) void*)(buf + (i * 256 + wave * 64) * 8), 16,
          src[i], col, 0, 0);
  }

  static constexpr int vmcnt(int n) { return (n & 15) | ((n >> 4) << 14) | (7 << 4) | (15 << 8); }

  // Loads after the copy of A stage c + 1 by the end of stage c (POS = c %
  // PS), counting only stages c - 1 and c: two A stages, the weights of the
  // stages that start a chunk, the block loads of a period's first stage.
  // In the first stages more have been issued: waiting for the extra ones
  // costs nothing (they are in use).
  template <int POS>
  static constexpr int after_next(int nd) {
    int n = 2 * nd;
    for (int d = POS - 1; d <= POS; ++d) {
      if ((d + PS) % SB == 0) n += NBL;
      if ((d + PS) % PS == 0) n += NSB;
    }
    return n;
  }

  template <int POS, int MBA>
  __device__ __forceinline__ void stage(uint16_t* b0, uint16_t* b1, uint16_t* b2, uint16_t* b3,
                                        int c, const uint32_t (&src)[MB / 2],
                                        const int (&rd)[2], Bw& cur, Bw& nxt, u32x4& bs,
                                        u32x4& bb, u32x4& nbs, u32x4& nbb, float (&sc)[QPW],
                                        float (&bi)[QPW], f32x4_t (&acc)[MB][QPW]) const {
    constexpr int ND = MBA / 2;
    constexpr int BUF = POS % NBUF;
    constexpr int H = POS % SB;
    uint16_t* const bufs[NBUF] = {b0, b1, b2, b3};
    __builtin_amdgcn_sched_barrier(0);
    dma<ND>(bufs[(BUF + 3) % NBUF], min(c + 3, nst - 1), src);
    __builtin_amdgcn_sched_barrier(0);
    if constexpr (H == 0) {
      load_b(min(c / SB + 1, nbc - 1), nxt);
      __builtin_amdgcn_sched_barrier(0);
    }
    if constexpr (POS == 0) {
      load_blk(c / PS + 1, nbs, nbb);
      __builtin_amdgcn_sched_barrier(0);
    }
    if constexpr (H == 0) scales<POS / SB>(bs, bb, sc, bi);
    const uint16_t* cb = bufs[BUF];
    // The first PF A fragments of a step are read before its
    // dequantisation, then each MFMA group reads the fragment PF ahead, so
    // no MFMA waits for a read just issued.
    constexpr int NPF = MBA < PF ? MBA : PF;
    auto read_a = [&](int j, int mb) {
      return __builtin_bit_cast(bf16x8_t,
                                *reinterpret_cast<const u32x4*>(cb + mb * 1024 + rd[j]));
    };
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      bf16x8_t a[MBA], bf[QPW];
#pragma unroll
      for (int mb = 0; mb < NPF; ++mb) a[mb] = read_a(j, mb);
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int qq = 0; qq < QPW; ++qq)
        bf[qq] = dequant_frag<BITS, 1>(
            *reinterpret_cast<const uint4(*)[1]>(&cur.w[qq]), 2 * H + j, sc[qq], bi[qq]);
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int mb = 0; mb < MBA; ++mb) {
        if (mb + NPF < MBA) a[mb + NPF] = read_a(j, mb + NPF);
#pragma unroll
        for (int qq = 0; qq < QPW; ++qq) acc[mb][qq] = mfma(a[mb], bf[qq], acc[mb][qq]);
      }
#pragma unroll
      for (int mb = 0; mb < MBA; ++mb) {
        if (mb + NPF < MBA) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
        __builtin_amdgcn_sched_group_barrier(0x008, QPW, 0);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
    if constexpr (H == SB - 1) cur = nxt;
    if constexpr (POS == PS - 1) {
      bs = nbs;
      bb = nbb;
    }
    __builtin_amdgcn_sched_barrier(0);
    __builtin_amdgcn_s_waitcnt(vmcnt(after_next<POS>(ND)));
    __builtin_amdgcn_s_barrier();
  }

  template <int MBA, int... P>
  __device__ __forceinline__ void period(std::integer_sequence<int, P...>, uint16_t* b0,
                                         uint16_t* b1, uint16_t* b2, uint16_t* b3, int c,
                                         const uint32_t (&src)[MB / 2], const int (&rd)[2],
                                         Bw& cur, Bw& nxt, u32x4& bs, u32x4& bb, u32x4& nbs,
                                         u32x4& nbb, float (&sc)[QPW], float (&bi)[QPW],
                                         f32x4_t (&acc)[MB][QPW]) const {
    (stage<P, MBA>(b0, b1, b2, b3, c + P, src, rd, cur, nxt, bs, bb, nbs, nbb, sc, bi, acc), ...);
  }
  template <int MBA, int... P>
  __device__ __forceinline__ void tail(std::integer_sequence<int, P...>, uint16_t* b0,
                                       uint16_t* b1, uint16_t* b2, uint16_t* b3, int c,
                                       const uint32_t (&src)[MB / 2], const int (&rd)[2],
                                       Bw& cur, Bw& nxt, u32x4& bs, u32x4& bb, u32x4& nbs,
                                       u32x4& nbb, float (&sc)[QPW], float (&bi)[QPW],
                                       f32x4_t (&acc)[MB][QPW]) const {
    ((c + P < nst ? stage<P, MBA>(b0, b1, b2, b3, c + P, src, rd, cur, nxt, bs, bb, nbs, nbb,
                                  sc, bi, acc)
                  : void()),
     ...);
  }

  template <int MBA>
  __device__ __forceinline__ void pipeline(uint16_t* __restrict__ b0, uint16_t* __restrict__ b1,
                                           uint16_t* __restrict__ b2, uint16_t* __restrict__ b3,
                                           f32x4_t (&acc)[MB][QPW]) const {
    constexpr int ND = MBA / 2;
    uint32_t src[MB / 2];
    a_src(src);
    int rd[2];
#pragma unroll
    for (int j = 0; j < 2; ++j)
      rd[j] = ((lane & 15) * 8 + ((2 * kg + j) ^ ((lane & 7) ^ ((lane >> 3) & 1)))) * 8;
    Bw cur, nxt;
    u32x4 bs, bb, nbs, nbb;
    float sc[QPW], bi[QPW];
    __builtin_amdgcn_sched_barrier(0);
    load_blk(0, bs, bb);
    __builtin_amdgcn_sched_barrier(0);
    dma<ND>(b0, 0, src);
    __builtin_amdgcn_sched_barrier(0);
    dma<ND>(b1, min(1, nst - 1), src);
    __builtin_amdgcn_sched_barrier(0);
    load_b(0, cur);
    __builtin_amdgcn_sched_barrier(0);
    dma<ND>(b2, min(2, nst - 1), src);
    __builtin_amdgcn_sched_barrier(0);
    __builtin_amdgcn_s_waitcnt(vmcnt(2 * ND + NBL));
    __builtin_amdgcn_s_barrier();
    int c = 0;
    for (; c + PS <= nst; c += PS)
      period<MBA>(std::make_integer_sequence<int, PS>{}, b0, b1, b2, b3, c, src, rd, cur, nxt,
                  bs, bb, nbs, nbb, sc, bi, acc);
    if (c < nst)  // K not a multiple of PS * 64: the last stages, each guarded
      tail<MBA>(std::make_integer_sequence<int, PS - 1>{}, b0, b1, b2, b3, c, src, rd, cur, nxt,
                bs, bb, nbs, nbb, sc, bi, acc);
  }

  template <int MBA>
  __device__ void run(f32x4_t (&acc)[MB][QPW]) const {
    pipeline<MBA>(l0, l1, l2, l3, acc);
  }

  __device__ void epilogue(const f32x4_t (&acc)[MB][QPW], int mba) const {
    uint16_t* so[NBUF] = {l0, l1, l2, l3};
    store_tile<MODE, MB, QPW, TN, THREADS, BM / NBUF>(p, tile, s_row, so, acc, mba);
  }
};

// The engine of a tile size: 128-row tiles on Wide, 32-row tiles on Gemm.
template <int BITS, int BM, int MODE>
struct EngineOf {
  using type = Gemm<BITS, BM, MODE>;
};
template <int BITS, int MODE>
struct EngineOf<BITS, 128, MODE> {
  using type = Wide<BITS, MODE>;
};
template <int BITS, int BM, int MODE>
using Engine = typename EngineOf<BITS, BM, MODE>::type;

template <int BITS, int BM, int MODE>
__global__ __launch_bounds__((Engine<BITS, BM, MODE>::THREADS))
__attribute__((amdgpu_waves_per_eu(Engine<BITS, BM, MODE>::MIN_WAVES))) void prefill_gemm_kernel(
    const PrefillArgs p, const int nt) {
  using G = Engine<BITS, BM, MODE>;
  __shared__ int s_row[BM];
  Tile tile;
  if (!decode_tile(p, nt, tile)) return;
  const int tid = threadIdx.x;
  const int TK = p.T * p.K;
  if (tid < BM) {
    int v = 0;
    if (tid < tile.nrows) {
      if (MODE == 1 && p.dense) {
        v = tile.row0 + tid;  // a dense product writes row m of y
      } else {
        const int src = p.rows[tile.row0 + tid];
        // gate/up: the token of the row; down: where its output goes
        v = MODE == 0 ? (src < TK ? src / p.K : src - TK) : src;
      }
    }
    s_row[tid] = v;
  }
  __syncthreads();
  if (tile.bucket == p.E + 1) {
    // out-of-range expert ids: zero rows, nothing loaded
    for (int i = tid; i < tile.nrows * G::TN; i += G::THREADS) {
      const int r = i / G::TN;
      const int c = tile.n * G::TN + (i - r * G::TN);
      if constexpr (MODE == 0)
        p.act[(size_t)(tile.row0 + r) * p.I + c] = 0;
      else
        p.y[(size_t)s_row[r] * p.H + c] = 0;
    }
    return;
  }
  // Wide: four distinct arrays, so that the compiler can tell the DMA into
  // one stage from the reads of another (a single array makes it wait for
  // every DMA in flight before each read)
  constexpr bool kWide = BM == 128;
  __shared__ __attribute__((aligned(16))) uint16_t s_l0[kWide ? Wide<BITS, MODE>::BUF : 1];
  __shared__ __attribute__((aligned(16))) uint16_t s_l1[kWide ? Wide<BITS, MODE>::BUF : 1];
  __shared__ __attribute__((aligned(16))) uint16_t s_l2[kWide ? Wide<BITS, MODE>::BUF : 1];
  __shared__ __attribute__((aligned(16))) uint16_t s_l3[kWide ? Wide<BITS, MODE>::BUF : 1];
  __shared__ __attribute__((aligned(16))) uint16_t s_lds[kWide ? 1 : Gemm<BITS, BM, MODE>::LDS];
  const G g = [&] {
    if constexpr (kWide)
      return G(p, tile, s_l0, s_l1, s_l2, s_l3, s_row);
    else
      return G(p, tile, s_lds, s_row);
  }();
  f32x4_t acc[G::MB][G::QPW];
#pragma unroll
  for (int mb = 0; mb < G::MB; ++mb)
#pragma unroll
    for (int qq = 0; qq < G::QPW; ++qq) acc[mb][qq] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  const int mba = (tile.nrows + 15) >> 4;
  if (mba > G::MB / 2) {
    g.template run<G::MB>(acc);
    g.epilogue(acc, G::MB);
  } else if constexpr (G::MB >= 4) {
    if (mba > G::MB / 4) {
      g.template run<G::MB / 2>(acc);
      g.epilogue(acc, G::MB / 2);
    } else {
      g.template run<G::MB / 4>(acc);
      g.epilogue(acc, G::MB / 4);
    }
  } else {
    g.template run<G::MB / 2>(acc);
    g.epilogue(acc, G::MB / 2);
  }
}

// ---------------------------------------------------------------- combine
// out[t] = bf16(sum_j score_j y[t K + j] + sg_t y[T K + t]) (+ residual):
// the slots in order, then the shared expert, as the decode kernels sum.
// From this many tokens the combine requests all of a token's rows at once
// (8192 tokens: 67.1 -> 56.7 us per call, 5.9 TB/s); below it one row per
// round trip was faster (512 tokens: 5.9 against 6.5 us).
constexpr int kCombineBatchTokens = 2048;

__global__ __launch_bounds__(256) void prefill_combine_kernel(const PrefillArgs p) {
  const int t = blockIdx.x;
  const int H = p.H;
  const int K = p.K;
  const int units = K + p.has_shared;
  const float* sc = p.scores + (size_t)t * p.score_stride;
  auto row_of = [&](int u) { return u < K ? (size_t)t * K + u : (size_t)p.T * K + t; };
  auto add_row = [](float (&acc)[8], const uint4 v, float w) {
    const uint32_t vv[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      acc[2 * i] += w * bf16_lo(vv[i]);
      acc[2 * i + 1] += w * bf16_hi(vv[i]);
    }
  };
  for (int h0 = threadIdx.x * 8; h0 < H; h0 += 256 * 8) {
    float acc[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) acc[i] = 0.0f;
    uint4 r = make_uint4(0u, 0u, 0u, 0u);
    if (units <= kMaxFusedUnits && p.T >= kCombineBatchTokens) {
      // every unit's row (and the residual) requested at once, then summed
      // in slot order: one load in flight per unit instead of one per
      // round trip
      uint4 v[kMaxFusedUnits];
#pragma unroll
      for (int u = 0; u < kMaxFusedUnits; ++u)
        if (u < units) v[u] = load16_stream(p.y + row_of(u) * H + h0);
      if (p.residual) r = load16(p.residual + (size_t)t * H + h0);
#pragma unroll
      for (int u = 0; u < kMaxFusedUnits; ++u)
        if (u < units) add_row(acc, v[u], sc[u]);
    } else {
      for (int u = 0; u < units; ++u) add_row(acc, load16(p.y + row_of(u) * H + h0), sc[u]);
      if (p.residual) r = load16(p.residual + (size_t)t * H + h0);
    }
    uint32_t o[4];
    const uint32_t rr[4] = {r.x, r.y, r.z, r.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      float a = round_bf16(acc[2 * i]);
      float b = round_bf16(acc[2 * i + 1]);
      if (p.residual) {
        a = bf16_lo(rr[i]) + a;
        b = bf16_hi(rr[i]) + b;
      }
      o[i] = f32_to_bf16(a) | (f32_to_bf16(b) << 16);
    }
    *reinterpret_cast<uint4*>(p.out + (size_t)t * H + h0) = make_uint4(o[0], o[1], o[2], o[3]);
  }
}

// --------------------------------------------------------------- launchers
int prefill_tile_rows(int T, int K, int E) {
  // few rows per expert (a short prefill chunk): 32-row tiles keep the
  // wasted MFMA rows low; otherwise 128-row tiles share each dequantised
  // weight fragment across more rows
  return (long)T * K <= 48L * E ? 32 : kPrefillBM;
}

int prefill_sort_slices(int T, int K) {
  const long n = (long)T * K;
  if (n <= kSortOneSliceRows) return 1;
  const long nw = (n + kSortRowsPerSlice - 1) / kSortRowsPerSlice;
  return (int)(nw < 1 ? 1 : nw > kPrefillMaxSlices ? kPrefillMaxSlices : nw);
}

int prefill_max_mtiles(int T, int K, int E, int bm) {
  return (T * K + T + bm - 1) / bm + E + 2;
}

template <int BITS, int BM>
void launch_gemms(const PrefillArgs& a, int mt, hipStream_t s) {
  const int nt_gu = a.I / Engine<BITS, BM, 0>::TN;
  const int nt_dn = a.H / Engine<BITS, BM, 1>::TN;
  // the full items are split over the XCDs in runs, the partial m-tiles
  // dealt in turn: up to 1 + nt more slots per XCD than an even split
  const int g_gu = 8 * ((nt_gu * mt + 7) / 8 + 1 + nt_gu);
  const int g_dn = 8 * ((nt_dn * mt + 7) / 8 + 1 + nt_dn);
  hipLaunchKernelGGL((prefill_gemm_kernel<BITS, BM, 0>), dim3(g_gu),
                     dim3(Engine<BITS, BM, 0>::THREADS), 0, s, a, nt_gu);
  hipLaunchKernelGGL((prefill_gemm_kernel<BITS, BM, 1>), dim3(g_dn),
                     dim3(Engine<BITS, BM, 1>::THREADS), 0, s, a, nt_dn);
}

bool dense_qmm_eligible(int M, int N, int K) {
  return M >= kDenseQmmMinRows && K >= 128 && K % 128 == 0 && N >= 256 && N % 256 == 0;
}

// The down GEMM's plain epilogue over a dense A: A = x rows in order (as the
// activations), the bank's expert 0 as the weights, y rows in place.
hipError_t launch_dense_qmm(const uint16_t* x, int M, const QW& w, int N, int K, int bits,
                            uint16_t* y, hipStream_t s) {
  PrefillArgs a{};
  a.T = M;
  a.K = 1;
  a.E = 1;
  a.H = N;       // output columns
  a.I = K;       // reduction
  a.dense = 1;
  a.act = const_cast<uint16_t*>(x);
  a.dn = w;
  a.y = y;
  // short products: 32-row tiles give more workgroups
  a.bm = M <= 256 ? 32 : kPrefillBM;
  if (a.bm == kPrefillBM && ((uint64_t)M * K * 2 > 0xFFFFFFFFull ||
                             (uint64_t)N * K * bits / 8 > 0xFFFFFFFFull))
    return hipErrorInvalidValue;
  const int mt = (M + a.bm - 1) / a.bm;
  auto go = [&](auto bits_c, auto bm_c) {
    constexpr int B = decltype(bits_c)::value;
    constexpr int BMc = decltype(bm_c)::value;
    const int nt = N / Engine<B, BMc, 1>::TN;
    const int g = 8 * ((nt * mt + 7) / 8);
    hipLaunchKernelGGL((prefill_gemm_kernel<B, BMc, 1>), dim3(g),
                       dim3(Engine<B, BMc, 1>::THREADS), 0, s, a, nt);
  };
  using I8 = std::integral_constant<int, 8>;
  using I4 = std::integral_constant<int, 4>;
  using B32 = std::integral_constant<int, 32>;
  using B128 = std::integral_constant<int, kPrefillBM>;
  if (bits == 8) {
    if (a.bm == 32) go(I8{}, B32{});
    else go(I8{}, B128{});
  } else {
    if (a.bm == 32) go(I4{}, B32{});
    else go(I4{}, B128{});
  }
  return hipGetLastError();
}

// The 128-row tiles address x, the activations and one expert's weights
// through buffer resources with 32-bit byte offsets.
bool buffer_offsets_fit(const PrefillArgs& a, int bits) {
  const uint64_t lim = 0xFFFFFFFFull;
  const uint64_t x = (uint64_t)a.T * a.H * 2;
  const uint64_t act = ((uint64_t)a.T * a.K + a.T) * a.I * 2;
  const uint64_t w = (uint64_t)2 * a.I * a.H * bits / 8;  // one expert's gate/up or down
  return x <= lim && act <= lim && w <= lim;
}

hipError_t launch_prefill(const PrefillArgs& args, int bits, bool combine, hipStream_t s) {
  PrefillArgs a = args;
  a.bm = prefill_tile_rows(a.T, a.K, a.E);
  if (a.bm == kPrefillBM && !buffer_offsets_fit(a, bits)) return hipErrorInvalidValue;
  const int nw = prefill_sort_slices(a.T, a.K);
  // one slice: the place kernel counts its rows itself
  if (nw > 1) hipLaunchKernelGGL(prefill_hist_kernel, dim3(nw), dim3(kSortThreads), 0, s, a);
  hipLaunchKernelGGL(prefill_place_kernel, dim3(nw), dim3(kSortThreads), 0, s, a);
  const int mt = prefill_max_mtiles(a.T, a.K, a.E, a.bm);
  if (bits == 8) {
    if (a.bm == 32) launch_gemms<8, 32>(a, mt, s);
    else launch_gemms<8, kPrefillBM>(a, mt, s);
  } else {
    if (a.bm == 32) launch_gemms<4, 32>(a, mt, s);
    else launch_gemms<4, kPrefillBM>(a, mt, s);
  }
  if (combine) hipLaunchKernelGGL(prefill_combine_kernel, dim3(a.T), dim3(256), 0, s, a);
  return hipGetLastError();
}

}  // namespace rmoe
