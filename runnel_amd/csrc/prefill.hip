// Prefill: expert-sorted grouped dequant-GEMM on bf16 MFMA (gfx950).
//
// Used when a call routes at least 64 (token, slot) rows, the point where
// the packed module sorts its rows by expert (src/runnel/mlx.py:59-63).
//
//   prefill_sort_kernel     one workgroup: stable counting sort of the
//                           (token, slot) rows by expert id (mlx-lm
//                           _gather_sort order), the shared expert's rows
//                           appended as bucket E, out-of-range ids as
//                           bucket E + 1; row and m-tile offsets per bucket.
//   prefill_gate_up_kernel  one (bucket, m-tile of 128 rows, n-tile of 128
//                           [up; gate] pairs) per workgroup: the x rows of
//                           the tile staged in LDS, every wave streams its
//                           own 32 up and 32 gate weight rows straight from
//                           HBM into registers, dequantises them to bf16
//                           (fl32(q*s + b) rounded to nearest even) and
//                           feeds v_mfma_f32_16x16x32_bf16; SwiGLU epilogue,
//                           bf16 activations in sorted row order.
//   prefill_down_kernel     the same over the activations (already in
//                           sorted order, contiguous) and the down bank, 256
//                           output columns per workgroup; bf16 rows written
//                           to their (token, slot) place.
//   prefill_combine_kernel  per token: sum of score * row over the slots and
//                           the gated shared row, residual, bf16.
//
// Work items are ordered (n-tile, bucket, m-tile) and cut into eight equal
// contiguous runs, one per XCD (workgroup i runs on XCD i % 8): the m-tiles
// of one (bucket, n-tile) run back to back on one XCD, so their common
// weight tile is read from HBM once and then hit in that XCD's L2.
//
// MFMA operand layout (16x16x32 bf16, checked on the device): lane l holds
// A row l % 16 and B column l % 16, k = 8 (l / 16) + [0, 8); D column l % 16,
// rows 4 (l / 16) + [0, 4).  The k index of each lane is remapped so that a
// lane's operands come from one 16-byte load: within a chunk of KC values of
// one row, lane group g = l / 16 owns k = g KC / 4 + [0, KC / 4), and MFMA j
// of the chunk takes k = g KC / 4 + 8 j + [0, 8) for both A and B.
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
constexpr int kGemmThreads = 256;               // 4 waves
constexpr int kBM = kPrefillBM;                 // rows per m-tile
constexpr int kMB = kBM / 16;                   // MFMA row blocks per tile
constexpr int kCB = kPrefillTileN / 64;         // 16-column blocks per wave
constexpr int kDownTileN = 2 * kPrefillTileN;   // down columns per workgroup
constexpr int kPad = 8;                         // bf16 of padding per LDS row

template <int BITS>
struct Chunk {
  static constexpr int KC = BITS == 8 ? 64 : 128;      // k values per chunk
  static constexpr int NJ = KC / 32;                   // MFMAs per chunk
  static constexpr int WORDS = KC * BITS / 32;         // u32 per row per chunk
  static constexpr int ROW = KC + kPad;                // LDS row (bf16)
  static constexpr int PIECES = kBM * KC / 8;          // 16-byte A pieces
  static constexpr int PPT = PIECES / kGemmThreads;    // pieces per thread
};

__device__ __forceinline__ uint32_t pack_bf16x2(float a, float b) {
  const f32x2_t f = {a, b};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(f, bf16x2_t));
}

// The bf16 MFMA fragment j (8 consecutive k) of a lane's 16-byte weight load.
template <int BITS>
__device__ __forceinline__ bf16x8_t dequant_frag(const uint4 w, int j, float s, float b) {
  u32x4 d;
  if constexpr (BITS == 8) {
    const uint32_t w0 = j == 0 ? w.x : w.z;
    const uint32_t w1 = j == 0 ? w.y : w.w;
    d.x = pack_bf16x2(fmaf((float)(w0 & 0xFFu), s, b), fmaf((float)((w0 >> 8) & 0xFFu), s, b));
    d.y = pack_bf16x2(fmaf((float)((w0 >> 16) & 0xFFu), s, b), fmaf((float)(w0 >> 24), s, b));
    d.z = pack_bf16x2(fmaf((float)(w1 & 0xFFu), s, b), fmaf((float)((w1 >> 8) & 0xFFu), s, b));
    d.w = pack_bf16x2(fmaf((float)((w1 >> 16) & 0xFFu), s, b), fmaf((float)(w1 >> 24), s, b));
  } else {
    const uint32_t wj = j == 0 ? w.x : j == 1 ? w.y : j == 2 ? w.z : w.w;
    const uint32_t lo = wj & 0x0F0F0F0Fu;         // codes 0, 2, 4, 6
    const uint32_t hi = (wj >> 4) & 0x0F0F0F0Fu;  // codes 1, 3, 5, 7
    d.x = pack_bf16x2(fmaf((float)(lo & 0xFFu), s, b), fmaf((float)(hi & 0xFFu), s, b));
    d.y = pack_bf16x2(fmaf((float)((lo >> 8) & 0xFFu), s, b),
                      fmaf((float)((hi >> 8) & 0xFFu), s, b));
    d.z = pack_bf16x2(fmaf((float)((lo >> 16) & 0xFFu), s, b),
                      fmaf((float)((hi >> 16) & 0xFFu), s, b));
    d.w = pack_bf16x2(fmaf((float)(lo >> 24), s, b), fmaf((float)(hi >> 24), s, b));
  }
  return __builtin_bit_cast(bf16x8_t, d);
}

__device__ __forceinline__ f32x4_t mfma(const bf16x8_t a, const bf16x8_t b, const f32x4_t c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

// Work item of this workgroup: (n-tile, bucket, m-tile).  Returns false when
// the workgroup has nothing to do.
struct Tile {
  int n, bucket, row0, nrows;
};

__device__ __forceinline__ bool decode_tile(const PrefillArgs& p, int nt, Tile& t) {
  const int NB = p.E + 2;
  const int MT = p.tile_offs[NB];
  const int total = nt * MT;
  const int L = (total + 7) >> 3;
  const int xcd = blockIdx.x & 7;
  const int slot = blockIdx.x >> 3;
  if (slot >= L) return false;
  const int item = xcd * L + slot;
  if (item >= total) return false;
  t.n = item / MT;
  const int rem = item - t.n * MT;
  int lo = 0, hi = NB - 1;  // last bucket whose first tile is <= rem
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if (p.tile_offs[mid] <= rem) lo = mid;
    else hi = mid - 1;
  }
  t.bucket = lo;
  t.row0 = p.offs[lo] + (rem - p.tile_offs[lo]) * kBM;
  t.nrows = min(kBM, p.offs[lo + 1] - t.row0);
  return true;
}

}  // namespace

// ------------------------------------------------------------------- sort
__global__ __launch_bounds__(kSortThreads) void prefill_sort_kernel(const PrefillArgs p) {
  const int NB = p.E + 2;  // routed buckets, shared, out-of-range
  __shared__ int s_hist[kSortWaves * (kPrefillMaxExperts + 2)];
  __shared__ int s_scan[2][kSortThreads];
  __shared__ int s_shared_off;
  const int tid = threadIdx.x;
  const int wave = tid >> 6;
  const int lane = tid & 63;
  for (int i = tid; i < kSortWaves * NB; i += kSortThreads) s_hist[i] = 0;
  __syncthreads();

  const int n = p.T * p.K;
  const int per = ((n + kSortWaves - 1) / kSortWaves + 63) & ~63;
  const int r0 = min(n, wave * per);
  const int r1 = min(n, r0 + per);
  int* my = s_hist + wave * NB;
  for (int r = r0 + lane; r < r1; r += 64) {
    int e = p.idx[r];
    e = (unsigned)e < (unsigned)p.E ? e : p.E + 1;
    atomicAdd(&my[e], 1);
  }
  __syncthreads();

  // Per bucket: total rows and m-tiles; exclusive scans over buckets.
  int rows_b = 0, tiles_b = 0;
  if (tid < NB) {
    if (tid == p.E) {
      rows_b = p.has_shared ? p.T : 0;
    } else {
      for (int w = 0; w < kSortWaves; ++w) rows_b += s_hist[w * NB + tid];
    }
    tiles_b = (rows_b + kBM - 1) / kBM;
  }
  s_scan[0][tid] = rows_b;
  s_scan[1][tid] = tiles_b;
  __syncthreads();
  for (int d = 1; d < kSortThreads; d <<= 1) {
    const int a = tid >= d ? s_scan[0][tid - d] : 0;
    const int b = tid >= d ? s_scan[1][tid - d] : 0;
    __syncthreads();
    s_scan[0][tid] += a;
    s_scan[1][tid] += b;
    __syncthreads();
  }
  if (tid < NB) {
    const int row_off = s_scan[0][tid] - rows_b;
    p.offs[tid] = row_off;
    p.tile_offs[tid] = s_scan[1][tid] - tiles_b;
    if (tid == NB - 1) {
      p.offs[NB] = s_scan[0][tid];
      p.tile_offs[NB] = s_scan[1][tid];
    }
    // per-wave bases of this bucket (stable: wave order = row order)
    int base = row_off;
    if (tid != p.E) {
      for (int w = 0; w < kSortWaves; ++w) {
        const int c = s_hist[w * NB + tid];
        s_hist[w * NB + tid] = base;
        base += c;
      }
    } else {
      s_shared_off = row_off;
    }
  }
  __syncthreads();
  if (p.has_shared)
    for (int t = tid; t < p.T; t += kSortThreads) p.rows[s_shared_off + t] = n + t;

  // Stable ranking: each wave walks its rows in order, 64 at a time; the
  // lanes holding one bucket find each other with one ballot per id bit.
  for (int c0 = r0; c0 < r1; c0 += 64) {
    const int r = c0 + lane;
    const bool v = r < r1;
    int e = 0;
    if (v) {
      e = p.idx[r];
      e = (unsigned)e < (unsigned)p.E ? e : p.E + 1;
    }
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
  }
}

// ----------------------------------------------------------- gate/up GEMM
template <int BITS>
__global__ __launch_bounds__(kGemmThreads) void prefill_gate_up_kernel(const PrefillArgs p,
                                                                        const int nt) {
  using C = Chunk<BITS>;
  __shared__ __attribute__((aligned(16))) uint16_t s_a[2][kBM * C::ROW];
  __shared__ int s_tok[kBM];
  Tile tile;
  if (!decode_tile(p, nt, tile)) return;
  const int tid = threadIdx.x;
  const int wave = tid >> 6;
  const int lane = tid & 63;
  const int I = p.I;
  const int H = p.H;
  const int TK = p.T * p.K;
  const int col_l = lane & 15;
  const int kg = lane >> 4;

  if (tile.bucket == p.E + 1) {
    // out-of-range expert ids: zero activations, nothing loaded
    for (int i = tid; i < tile.nrows * kPrefillTileN; i += kGemmThreads) {
      const int r = i / kPrefillTileN;
      const int c = tile.n * kPrefillTileN + (i - r * kPrefillTileN);
      p.act[(size_t)(tile.row0 + r) * I + c] = 0;
    }
    return;
  }
  if (tid < kBM) {
    int t = 0;
    if (tid < tile.nrows) {
      const int src = p.rows[tile.row0 + tid];
      t = src < TK ? src / p.K : src - TK;
    }
    s_tok[tid] = t;
  }
  const bool shared = tile.bucket == p.E;
  const QW q = shared ? p.sgu : p.gu;
  const size_t e = shared ? 0 : (size_t)tile.bucket;
  const int WPR = H * BITS / 32;
  const int G = H / 64;
  // this lane's up rows (c) and gate rows (I + c), one per column block
  const uint32_t* wrow[kCB][2];
  size_t prow[kCB][2];
#pragma unroll
  for (int cb = 0; cb < kCB; ++cb) {
    const int c = tile.n * kPrefillTileN + wave * (16 * kCB) + cb * 16 + col_l;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      prow[cb][h] = e * 2 * I + (size_t)(c + h * I);
      wrow[cb][h] = q.w + prow[cb][h] * WPR + kg * 4;
    }
  }
  __syncthreads();  // s_tok

  const int nch = H / C::KC;
  const int mb_active = (tile.nrows + 15) >> 4;
  // A staging: piece i of the tile is row i / (KC / 8), 16-byte column i % (KC / 8)
  uint4 ar[C::PPT];
  auto load_a = [&](int ch) {
#pragma unroll
    for (int j = 0; j < C::PPT; ++j) {
      const int pi = tid + kGemmThreads * j;
      const int r = pi / (C::KC / 8);
      const int c8 = pi - r * (C::KC / 8);
      ar[j] = make_uint4(0, 0, 0, 0);
      if (r < tile.nrows)
        ar[j] = load16(p.x + (size_t)s_tok[r] * H + ch * C::KC + c8 * 8);
    }
  };
  auto store_a = [&](int buf) {
#pragma unroll
    for (int j = 0; j < C::PPT; ++j) {
      const int pi = tid + kGemmThreads * j;
      const int r = pi / (C::KC / 8);
      const int c8 = pi - r * (C::KC / 8);
      *reinterpret_cast<uint4*>(&s_a[buf][r * C::ROW + c8 * 8]) = ar[j];
    }
  };
  uint4 bw[kCB][2];
  float bs[kCB][2], bb[kCB][2];
  auto load_b = [&](int ch, uint4 (&w)[kCB][2], float (&s)[kCB][2], float (&b)[kCB][2]) {
    const int g = BITS == 8 ? ch : 2 * ch + (kg >> 1);
#pragma unroll
    for (int cb = 0; cb < kCB; ++cb)
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        s[cb][h] = bf16_to_f32(q.s[prow[cb][h] * G + g]);
        b[cb][h] = bf16_to_f32(q.b[prow[cb][h] * G + g]);
      }
#pragma unroll
    for (int cb = 0; cb < kCB; ++cb)
#pragma unroll
      for (int h = 0; h < 2; ++h) w[cb][h] = load16_stream(wrow[cb][h] + ch * C::WORDS);
  };

  f32x4_t acc[kMB][kCB][2];
#pragma unroll
  for (int mb = 0; mb < kMB; ++mb)
#pragma unroll
    for (int cb = 0; cb < kCB; ++cb)
#pragma unroll
      for (int h = 0; h < 2; ++h) acc[mb][cb][h] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  load_b(0, bw, bs, bb);
  load_a(0);
  store_a(0);
  __syncthreads();
  for (int ch = 0; ch < nch; ++ch) {
    const int buf = ch & 1;
    uint4 nw[kCB][2];
    float ns[kCB][2], nb[kCB][2];
    const bool more = ch + 1 < nch;
    if (more) {
      load_b(ch + 1, nw, ns, nb);
      load_a(ch + 1);
    }
    const uint16_t* sa = &s_a[buf][col_l * C::ROW + kg * (C::KC / 4)];
#pragma unroll
    for (int j = 0; j < C::NJ; ++j) {
      bf16x8_t bf[kCB][2];
#pragma unroll
      for (int cb = 0; cb < kCB; ++cb)
#pragma unroll
        for (int h = 0; h < 2; ++h)
          bf[cb][h] = dequant_frag<BITS>(bw[cb][h], j, bs[cb][h], bb[cb][h]);
#pragma unroll
      for (int mb = 0; mb < kMB; ++mb) {
        if (mb < mb_active) {
          const bf16x8_t a = __builtin_bit_cast(
              bf16x8_t, *reinterpret_cast<const u32x4*>(sa + mb * 16 * C::ROW + 8 * j));
#pragma unroll
          for (int cb = 0; cb < kCB; ++cb)
#pragma unroll
            for (int h = 0; h < 2; ++h) acc[mb][cb][h] = mfma(a, bf[cb][h], acc[mb][cb][h]);
        }
      }
    }
    if (more) store_a(buf ^ 1);
    __syncthreads();
    if (more) {
#pragma unroll
      for (int cb = 0; cb < kCB; ++cb)
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          bw[cb][h] = nw[cb][h];
          bs[cb][h] = ns[cb][h];
          bb[cb][h] = nb[cb][h];
        }
    }
  }

  // SwiGLU epilogue: up and gate of one pair sit in the same lane/register
#pragma unroll
  for (int mb = 0; mb < kMB; ++mb) {
    if (mb >= mb_active) continue;
#pragma unroll
    for (int cb = 0; cb < kCB; ++cb) {
      const int c = tile.n * kPrefillTileN + wave * (16 * kCB) + cb * 16 + col_l;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int r = mb * 16 + kg * 4 + i;
        if (r < tile.nrows) {
          const float up = round_bf16(acc[mb][cb][0][i]);
          const float gate = round_bf16(acc[mb][cb][1][i]);
          p.act[(size_t)(tile.row0 + r) * I + c] = (uint16_t)f32_to_bf16(silu(gate) * up);
        }
      }
    }
  }
}

// -------------------------------------------------------------- down GEMM
template <int BITS>
__global__ __launch_bounds__(kGemmThreads) void prefill_down_kernel(const PrefillArgs p,
                                                                     const int nt) {
  using C = Chunk<BITS>;
  __shared__ __attribute__((aligned(16))) uint16_t s_a[2][kBM * C::ROW];
  __shared__ int s_dst[kBM];
  Tile tile;
  if (!decode_tile(p, nt, tile)) return;
  const int tid = threadIdx.x;
  const int wave = tid >> 6;
  const int lane = tid & 63;
  const int I = p.I;
  const int H = p.H;
  const int col_l = lane & 15;
  const int kg = lane >> 4;
  if (tid < kBM) s_dst[tid] = tid < tile.nrows ? p.rows[tile.row0 + tid] : 0;
  __syncthreads();

  if (tile.bucket == p.E + 1) {
    for (int i = tid; i < tile.nrows * kDownTileN; i += kGemmThreads) {
      const int r = i / kDownTileN;
      const int c = tile.n * kDownTileN + (i - r * kDownTileN);
      p.y[(size_t)s_dst[r] * H + c] = 0;
    }
    return;
  }
  const bool shared = tile.bucket == p.E;
  const QW q = shared ? p.sdn : p.dn;
  const size_t e = shared ? 0 : (size_t)tile.bucket;
  const int WPR = I * BITS / 32;
  const int G = I / 64;
  const uint32_t* wrow[kCB][2];
  size_t prow[kCB][2];
  // the down tile's 256 output columns: wave w owns 64, as 2 x kCB
  // 16-column MFMA tiles
#pragma unroll
  for (int cb = 0; cb < kCB; ++cb)
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int c = tile.n * kDownTileN + wave * 64 + h * 16 * kCB + cb * 16 + col_l;
      prow[cb][h] = e * H + (size_t)c;
      wrow[cb][h] = q.w + prow[cb][h] * WPR + kg * 4;
    }

  const int nch = I / C::KC;
  const int mb_active = (tile.nrows + 15) >> 4;
  uint4 ar[C::PPT];
  auto load_a = [&](int ch) {
#pragma unroll
    for (int j = 0; j < C::PPT; ++j) {
      const int pi = tid + kGemmThreads * j;
      const int r = pi / (C::KC / 8);
      const int c8 = pi - r * (C::KC / 8);
      ar[j] = make_uint4(0, 0, 0, 0);
      if (r < tile.nrows)
        ar[j] = load16(p.act + (size_t)(tile.row0 + r) * I + ch * C::KC + c8 * 8);
    }
  };
  auto store_a = [&](int buf) {
#pragma unroll
    for (int j = 0; j < C::PPT; ++j) {
      const int pi = tid + kGemmThreads * j;
      const int r = pi / (C::KC / 8);
      const int c8 = pi - r * (C::KC / 8);
      *reinterpret_cast<uint4*>(&s_a[buf][r * C::ROW + c8 * 8]) = ar[j];
    }
  };
  uint4 bw[kCB][2];
  float bs[kCB][2], bb[kCB][2];
  auto load_b = [&](int ch, uint4 (&w)[kCB][2], float (&s)[kCB][2], float (&b)[kCB][2]) {
    const int g = BITS == 8 ? ch : 2 * ch + (kg >> 1);
#pragma unroll
    for (int cb = 0; cb < kCB; ++cb)
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        s[cb][h] = bf16_to_f32(q.s[prow[cb][h] * G + g]);
        b[cb][h] = bf16_to_f32(q.b[prow[cb][h] * G + g]);
      }
#pragma unroll
    for (int cb = 0; cb < kCB; ++cb)
#pragma unroll
      for (int h = 0; h < 2; ++h) w[cb][h] = load16_stream(wrow[cb][h] + ch * C::WORDS);
  };

  f32x4_t acc[kMB][kCB][2];
#pragma unroll
  for (int mb = 0; mb < kMB; ++mb)
#pragma unroll
    for (int cb = 0; cb < kCB; ++cb)
#pragma unroll
      for (int h = 0; h < 2; ++h) acc[mb][cb][h] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  load_b(0, bw, bs, bb);
  load_a(0);
  store_a(0);
  __syncthreads();
  for (int ch = 0; ch < nch; ++ch) {
    const int buf = ch & 1;
    uint4 nw[kCB][2];
    float ns[kCB][2], nb[kCB][2];
    const bool more = ch + 1 < nch;
    if (more) {
      load_b(ch + 1, nw, ns, nb);
      load_a(ch + 1);
    }
    const uint16_t* sa = &s_a[buf][col_l * C::ROW + kg * (C::KC / 4)];
#pragma unroll
    for (int j = 0; j < C::NJ; ++j) {
      bf16x8_t bf[kCB][2];
#pragma unroll
      for (int cb = 0; cb < kCB; ++cb)
#pragma unroll
        for (int h = 0; h < 2; ++h)
          bf[cb][h] = dequant_frag<BITS>(bw[cb][h], j, bs[cb][h], bb[cb][h]);
#pragma unroll
      for (int mb = 0; mb < kMB; ++mb) {
        if (mb < mb_active) {
          const bf16x8_t a = __builtin_bit_cast(
              bf16x8_t, *reinterpret_cast<const u32x4*>(sa + mb * 16 * C::ROW + 8 * j));
#pragma unroll
          for (int cb = 0; cb < kCB; ++cb)
#pragma unroll
            for (int h = 0; h < 2; ++h) acc[mb][cb][h] = mfma(a, bf[cb][h], acc[mb][cb][h]);
        }
      }
    }
    if (more) store_a(buf ^ 1);
    __syncthreads();
    if (more) {
#pragma unroll
      for (int cb = 0; cb < kCB; ++cb)
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          bw[cb][h] = nw[cb][h];
          bs[cb][h] = ns[cb][h];
          bb[cb][h] = nb[cb][h];
        }
    }
  }

#pragma unroll
  for (int mb = 0; mb < kMB; ++mb) {
    if (mb >= mb_active) continue;
#pragma unroll
    for (int cb = 0; cb < kCB; ++cb)
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const int c = tile.n * kDownTileN + wave * 64 + h * 16 * kCB + cb * 16 + col_l;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int r = mb * 16 + kg * 4 + i;
          if (r < tile.nrows)
            p.y[(size_t)s_dst[r] * H + c] = (uint16_t)f32_to_bf16(acc[mb][cb][h][i]);
        }
      }
  }
}

// ---------------------------------------------------------------- combine
// out[t] = bf16(sum_j score_j y[t K + j] + sg_t y[T K + t]) (+ residual):
// the slots in order, then the shared expert, as the decode kernels sum.
__global__ __launch_bounds__(256) void prefill_combine_kernel(const PrefillArgs p) {
  const int t = blockIdx.x;
  const int H = p.H;
  const int K = p.K;
  const int units = K + p.has_shared;
  const float* sc = p.scores + (size_t)t * (K + 1);
  for (int h0 = threadIdx.x * 8; h0 < H; h0 += 256 * 8) {
    float acc[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) acc[i] = 0.0f;
    for (int u = 0; u < units; ++u) {
      const size_t row = u < K ? (size_t)t * K + u : (size_t)p.T * K + t;
      const uint4 v = load16(p.y + row * H + h0);
      const float w = sc[u];
      const uint32_t vv[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        acc[2 * i] += w * bf16_lo(vv[i]);
        acc[2 * i + 1] += w * bf16_hi(vv[i]);
      }
    }
    uint32_t o[4];
    uint32_t rr[4] = {0, 0, 0, 0};
    if (p.residual) {
      const uint4 r = load16(p.residual + (size_t)t * H + h0);
      rr[0] = r.x;
      rr[1] = r.y;
      rr[2] = r.z;
      rr[3] = r.w;
    }
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
int prefill_max_mtiles(int T, int K, int E) {
  return (T * K + T + kBM - 1) / kBM + E + 2;
}

hipError_t launch_prefill(const PrefillArgs& a, int bits, bool combine, hipStream_t s) {
  hipLaunchKernelGGL(prefill_sort_kernel, dim3(1), dim3(kSortThreads), 0, s, a);
  const int mt = prefill_max_mtiles(a.T, a.K, a.E);
  const int nt_gu = a.I / kPrefillTileN;
  const int nt_dn = a.H / kDownTileN;
  const int g_gu = 8 * ((nt_gu * mt + 7) / 8);
  const int g_dn = 8 * ((nt_dn * mt + 7) / 8);
  if (bits == 8) {
    hipLaunchKernelGGL(prefill_gate_up_kernel<8>, dim3(g_gu), dim3(kGemmThreads), 0, s, a, nt_gu);
    hipLaunchKernelGGL(prefill_down_kernel<8>, dim3(g_dn), dim3(kGemmThreads), 0, s, a, nt_dn);
  } else {
    hipLaunchKernelGGL(prefill_gate_up_kernel<4>, dim3(g_gu), dim3(kGemmThreads), 0, s, a, nt_gu);
    hipLaunchKernelGGL(prefill_down_kernel<4>, dim3(g_dn), dim3(kGemmThreads), 0, s, a, nt_dn);
  }
  if (combine) hipLaunchKernelGGL(prefill_combine_kernel, dim3(a.T), dim3(256), 0, s, a);
  return hipGetLastError();
}

}  // namespace rmoe
