// qgemm.hip -- grouped int8-MFMA GEMM for prefill (see qgemm.h for the
// numerics).  gfx950: v_mfma_i32_32x32x32_i8, wave64.
//
// Workgroup: 8 waves in a 4 x 2 arrangement over a 128 (token rows) x 256
// (weight rows) tile; each wave owns 32 x 128 = 1 x 4 MFMA blocks per limb
// (three limbs: 192 int32 accumulators, two waves per SIMD).  Pipeline: q8
// has three LDS stages of 64-wide k slices copied straight into LDS by
// global_load_lds, two in flight while one is multiplied; q4 has two stages,
// 64-wide slices unpacked in registers on the way.  One barrier per slice.
// MFMA operand layout (measured on gfx950): lane l supplies row (l % 32) and
// the 16-byte k chunk (l / 32) of a 32-wide k step, for A rows and for B
// columns alike; result register r of lane l is
// C[(r / 4) * 8 + (l / 32) * 4 + r % 4][l % 32].
#include "qgemm.h"

#include <cstdlib>
#include <type_traits>

namespace mlh {

typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef int i32x16 __attribute__((ext_vector_type(16)));

constexpr int kLimbs = 3;
constexpr float kQuantMax = 4194304.0f;  // 2^22: |65536 * hi + 256 * mid + lo| bound

bool qgemm_shape_ok(int fmt, int k) {
    return (fmt == kQ8 || fmt == kQ4) && k > 0 && k % kQgBK == 0;
}

// ---------------------------------------------------------------------------
// activation quantisation: one wave per row
// ---------------------------------------------------------------------------

// v * inv rounded to an integer q, |q| <= 2^22, as q = 65536 h + 256 m + l
// with m, l in [-128, 127] and h in [-64, 64]
__device__ __forceinline__ void quant_limbs(float v, float inv, int &h, int &m, int &l) {
    float q = rintf(v * inv);
    q = fminf(fmaxf(q, -kQuantMax), kQuantMax);
    const int qi = (int)q;
    const int t = (qi + 128) >> 8;  // floor: l lands in [-128, 127]
    l = qi - t * 256;
    h = (t + 128) >> 8;
    m = t - h * 256;
}

__device__ __forceinline__ unsigned pack_bytes(int a, int b, int c, int d) {
    return (unsigned)(a & 0xFF) | ((unsigned)(b & 0xFF) << 8) | ((unsigned)(c & 0xFF) << 16) |
           ((unsigned)(d & 0xFF) << 24);
}

// Rows of up to kQuantRegChunks * 256 values stay in registers (one read of
// the row); wider rows (the 11264-wide dense down input) are read per pass.
constexpr int kQuantRegChunks = 16;

// One set of rows to quantise: x (row stride x_stride, optionally
// RMSNorm'ed with norm_w) -> limbs hi, mid, lo at q, q + plane, q + 2 plane
// (row stride width) and scales.
struct QuantSeg {
    const float *x = nullptr;
    long x_stride = 0;
    int rows = 0, width = 0;
    const float *norm_w = nullptr;
    float eps = 0.0f;
    int8_t *q = nullptr;
    long plane = 0;
    float *scale = nullptr;
};

// Row `row` of a segment by one wave.
template <bool REG>
__device__ __forceinline__ void quantize_row(const QuantSeg &s, int row) {
    const float *x = s.x, *norm_w = s.norm_w;
    const int width = s.width;
    const float eps = s.eps;
    int8_t *hi = s.q, *mid = s.q + s.plane, *lo = s.q + 2 * s.plane;
    float *scale = s.scale;
    const int lane = threadIdx.x & (kWave - 1);
    const float *xr = x + (long)row * s.x_stride;
    const int nchunks = (width / 4 + kWave - 1) / kWave;  // float4 chunks per lane (upper)
    f32x4 v[REG ? kQuantRegChunks : 1];
    if constexpr (REG) {
#pragma unroll
        for (int c = 0; c < kQuantRegChunks; ++c) {
            const int i = (c * kWave + lane) * 4;
            v[c] = (c < nchunks && i < width) ? load_f4(xr + i) : f32x4{0.f, 0.f, 0.f, 0.f};
        }
    }
    auto value = [&](int c) -> f32x4 {
        if constexpr (REG) return v[c];
        const int i = (c * kWave + lane) * 4;
        return i < width ? load_f4(xr + i) : f32x4{0.f, 0.f, 0.f, 0.f};
    };
    const int nc = REG ? kQuantRegChunks : nchunks;
    float inv_rms = 1.0f;
    if (norm_w) {
        float ss = 0.0f;
        for (int c = 0; c < nc; ++c) {
            const f32x4 t = value(c);
            ss += t.x * t.x + t.y * t.y + t.z * t.z + t.w * t.w;
        }
        ss = dpp_wave_sum(ss);
        inv_rms = 1.0f / sqrtf(ss / (float)width + eps);
    }
    auto normed = [&](int c) -> f32x4 {
        f32x4 t = value(c);
        const int i = (c * kWave + lane) * 4;
        if (norm_w && i < width) {
            const f32x4 n = load_f4(norm_w + i);
            t.x = t.x * inv_rms * n.x;
            t.y = t.y * inv_rms * n.y;
            t.z = t.z * inv_rms * n.z;
            t.w = t.w * inv_rms * n.w;
        }
        return t;
    };
    float amax = 0.0f;
    for (int c = 0; c < nc; ++c) {
        const f32x4 t = normed(c);
        amax = fmaxf(amax, fmaxf(fmaxf(fabsf(t.x), fabsf(t.y)), fmaxf(fabsf(t.z), fabsf(t.w))));
    }
    amax = dpp_wave_max(amax);
    const float inv = amax > 0.0f ? kQuantMax / amax : 0.0f;
    if (lane == 0) scale[row] = amax / kQuantMax;
    int8_t *hr = hi + (long)row * width;
    int8_t *mr = mid + (long)row * width;
    int8_t *lr = lo + (long)row * width;
    for (int c = 0; c < nc; ++c) {
        const int i = (c * kWave + lane) * 4;
        if (i >= width) continue;
        const f32x4 t = normed(c);
        int h0, h1, h2, h3, m0, m1, m2, m3, l0, l1, l2, l3;
        quant_limbs(t.x, inv, h0, m0, l0);
        quant_limbs(t.y, inv, h1, m1, l1);
        quant_limbs(t.z, inv, h2, m2, l2);
        quant_limbs(t.w, inv, h3, m3, l3);
        *reinterpret_cast<unsigned *>(hr + i) = pack_bytes(h0, h1, h2, h3);
        *reinterpret_cast<unsigned *>(mr + i) = pack_bytes(m0, m1, m2, m3);
        *reinterpret_cast<unsigned *>(lr + i) = pack_bytes(l0, l1, l2, l3);
    }
}

// Workgroups [0, blocks_a) take 4 rows of segment a each, the rest 4 rows of
// segment b (two segments in one launch).
template <bool REG>
__global__ __launch_bounds__(256) void quantize_act_kernel(QuantSeg a, QuantSeg b, int blocks_a) {
    const bool in_b = (int)blockIdx.x >= blocks_a;
    const QuantSeg s = in_b ? b : a;
    const int row = ((int)blockIdx.x - (in_b ? blocks_a : 0)) * 4 + (int)(threadIdx.x >> 6);
    if (row >= s.rows) return;
    quantize_row<REG>(s, row);
}

static bool quant_seg_ok(const QuantSeg &s) {
    return s.rows == 0 || (s.x && s.q && s.plane >= (long)s.rows * s.width && s.scale &&
                           s.rows > 0 && s.width > 0 &&
                           s.width % 4 == 0 && s.x_stride % 4 == 0);
}

static int quantize_segments(const QuantSeg &a, const QuantSeg &b, hipStream_t stream) {
    if (a.rows <= 0 || !quant_seg_ok(a) || !quant_seg_ok(b)) return kErrArgs;
    const int blocks_a = (a.rows + 3) / 4, blocks_b = (b.rows + 3) / 4;
    const bool reg = a.width <= kQuantRegChunks * kWave * 4 &&
                     (b.rows == 0 || b.width <= kQuantRegChunks * kWave * 4);
    if (reg)
        hipLaunchKernelGGL(quantize_act_kernel<true>, dim3(blocks_a + blocks_b), dim3(256), 0,
                           stream, a, b, blocks_a);
    else
        hipLaunchKernelGGL(quantize_act_kernel<false>, dim3(blocks_a + blocks_b), dim3(256), 0,
                           stream, a, b, blocks_a);
    return hipGetLastError() == hipSuccess ? kOk : kErrLaunch;
}

int quantize_activations(const float *x, long x_stride, int rows, int width, const float *norm_w,
                         float eps, int8_t *q, long plane, float *scale, hipStream_t stream) {
    if (!x || !q || !scale || rows <= 0 || width <= 0) return kErrArgs;
    QuantSeg a;
    a.x = x;
    a.x_stride = x_stride;
    a.rows = rows;
    a.width = width;
    a.norm_w = norm_w;
    a.eps = eps;
    a.q = q;
    a.plane = plane;
    a.scale = scale;
    return quantize_segments(a, QuantSeg{}, stream);
}

// ---------------------------------------------------------------------------
// GEMM
// ---------------------------------------------------------------------------

// 16 packed nibbles (stored q + 8, column 2j low) -> 8 int8 values q.
__device__ __forceinline__ void unpack_q4_word(unsigned w, unsigned &out0, unsigned &out1) {
    const unsigned lo = w & 0x0F0F0F0Fu;         // even columns
    const unsigned hi = (w >> 4) & 0x0F0F0F0Fu;  // odd columns
    // bytes [lo0, hi0, lo1, hi1] and [lo2, hi2, lo3, hi3]
    const unsigned a = __builtin_amdgcn_perm(hi, lo, 0x05010400u);
    const unsigned b = __builtin_amdgcn_perm(hi, lo, 0x07030602u);
    // stored u in [0, 15] -> u - 8 as int8: (u + 0x78) ^ 0x80, no carry between bytes
    out0 = (a + 0x78787878u) ^ 0x80808080u;
    out1 = (b + 0x78787878u) ^ 0x80808080u;
}

__device__ __forceinline__ int find_task(const int *tile_start, int n, int tile) {
    // last t in [0, n) with tile_start[t] <= tile (tile_start non-decreasing,
    // tile_start[0] = 0): every lane of the wave tests entries lane, lane +
    // 64, ... and the ballots count them -- one round of loads for the first
    // 128 tasks instead of a chain of dependent ones
    const int lane = threadIdx.x & 63;
    const int i0 = lane, i1 = lane + 64;
    const int v0 = tile_start[i0 < n ? i0 : 0];
    const int v1 = tile_start[i1 < n ? i1 : 0];
    int count = __popcll(__ballot(i0 < n && v0 <= tile)) + __popcll(__ballot(i1 < n && v1 <= tile));
    for (int c0 = 128; c0 < n; c0 += 64) {
        const int i = c0 + lane;
        const int v = tile_start[i < n ? i : 0];
        count += __popcll(__ballot(i < n && v <= tile));
    }
    return count - 1;
}

template <bool DUAL, int BM>
__host__ __device__ __forceinline__ int tiles_of(int rows, int n_out) {
    constexpr int outw = DUAL ? kQgBW / 2 : kQgBW;
    return ((rows + BM - 1) / BM) * ((n_out + outw - 1) / outw);
}

// Tile blockIdx.x of a launch -> its task record and the first token row m0
// and output n0 of its BM x 256 tile; false for workgroups past the tiles.
// Tiles run in XCD-contiguous order (workgroup i goes to XCD i % 8): each XCD
// takes a contiguous range of tiles, and within a task groups of kQgGroup row
// tiles share one column tile, so neighbouring workgroups of an XCD reuse
// weight tiles from its L2.
template <bool DUAL, int BM>
__device__ __forceinline__ bool map_tile(const QGemmLaunch &L, GemmTask &tk, int &m0, int &n0) {
    int local;
    {
        int begin = 0, end;
        int n_tasks = 1;
        if (L.tasks) {
            const int nr = *L.n_routed;
            n_tasks = nr + L.n_shared;
            end = L.range == 1 ? L.tile_start[nr] : L.tile_start[nr + L.n_shared];
            if (L.range == 2) begin = L.tile_start[nr];
        } else {
            end = tiles_of<DUAL, BM>(L.single.rows, L.single.n_out);
        }
        const int total = end - begin;
        const int per = (total + 7) >> 3;
        const int slot = blockIdx.x >> 3;
        if (slot >= per) return false;
        const int tile = begin + (blockIdx.x & 7) * per + slot;
        if (tile >= end) return false;
        if (L.tasks) {
            const int t = find_task(L.tile_start, n_tasks, tile);
            tk = L.tasks[t];
            local = tile - L.tile_start[t];
        } else {
            tk = L.single;
            local = tile;
        }
    }
    constexpr int outw = DUAL ? kQgBW / 2 : kQgBW;
    const int n_tiles = (tk.n_out + outw - 1) / outw;
    const int m_tiles = (tk.rows + BM - 1) / BM;
    const int per_group = kQgGroup * n_tiles;
    const int grp = local / per_group;
    const int gsize = min(kQgGroup, m_tiles - grp * kQgGroup);
    const int rem = local - grp * per_group;
    m0 = (grp * kQgGroup + rem % gsize) * BM;
    n0 = (rem / gsize) * outw;
    return true;
}

// LDS tiles hold one k slice per stage as rows of RB bytes (RB / 16 chunks of
// 16 bytes): q8 slices are 128 wide and go straight from global memory into
// LDS (global_load_lds_dwordx4, full 128-byte lines per row); q4 slices are
// 64 wide and are unpacked in registers on the way.  Chunk c of row r lives
// at chunk c ^ g(r):
//   RB = 64:  g(r) = ((r >> 1) ^ (r >> 3)) & 3
//   RB = 128: g(r) = (r ^ (r >> 3)) & 7
// so that the MFMA fragment reads (32 consecutive rows, one chunk) and the
// tile writes hit distinct banks whether the LDS serves 8 or 16 lanes of a
// 128-bit access per cycle.
// Stage width: q8 32-row tiles (weight-stream bound) copy 128-k slices, so a
// DMA instruction covers 8 rows x 128 contiguous bytes (on MI355X runs of
// 128 bytes stream ~6 TB/s, runs of 64 bytes ~4.2 TB/s); the 128-row tile
// (MFMA bound) keeps 64-k slices to fit more stages.
template <int FMT, int BM> struct QgCfg {
    static constexpr int kRB = (FMT == kQ8 && BM == 32) ? 128 : 64;
};

template <int RB>
__device__ __forceinline__ int lds_off(int row, int chunk) {
    if constexpr (RB == 64) return row * 64 + ((chunk ^ (((row >> 1) ^ (row >> 3)) & 3)) << 4);
    else return row * 128 + ((chunk ^ ((row ^ (row >> 3)) & 7)) << 4);
}

// Tile shape of a BM-row tile (BM = 128 or kQgBMSmall = 32).  BM = 128: 8
// waves (two per SIMD) in a 4 (token rows) x 2 (weight rows) grid, each wave
// 32 x 128 = 1 x 4 blocks of 32 x 32 per limb (192 int32 accumulators);
// BM = 32: 4 waves side by side, each 32 x 64 = 1 x 2 blocks.  A stage holds
// the three limb tiles of A and the weight tile.  q8 DMA: blocks of 1 KB
// (1024 / kRB rows), wave w taking A blocks w, w + kWaves, ... (waves may
// issue one more than others when the count does not divide), B blocks
// likewise.
template <int FMT, int BM> struct QgShape {
    static constexpr int kRB = QgCfg<FMT, BM>::kRB;
    static constexpr int kRowsDma = 1024 / kRB;    // rows per DMA block
    static constexpr int kWaves = BM == 128 ? 8 : 4;
    static constexpr int kThreads = kWaves * kWave;
    static constexpr int kWM = BM / 32;            // waves along the token rows
    static constexpr int kWN = kWaves / kWM;       // waves along the weight rows
    static constexpr int kMI = 1;
    static constexpr int kNF = kQgBW / 32 / kWN;   // 32-row weight blocks per wave
    static constexpr int kStages = FMT == kQ8 ? 3 : 2;
    static constexpr int kLdsA = kLimbs * BM * kRB;
    static constexpr int kStage = (kLimbs * BM + kQgBW) * kRB;
    static constexpr int kLds = kStages * kStage + BM * 8;  // + scales and row map
    static constexpr int kRowBlocks = BM / kRowsDma;
    static constexpr int kABlocks = kLimbs * kRowBlocks;
    static constexpr int kBBlocks = kQgBW / kRowsDma;
    static constexpr int kBPer = kBBlocks / kWaves;
    static constexpr int kAMax = (kABlocks + kWaves - 1) / kWaves, kAMin = kABlocks / kWaves;
    static constexpr int kDmaMax = kAMax + kBPer, kDmaMin = kAMin + kBPer;
    // register path (q4): 16-byte A chunks and packed B chunks per thread and slice
    static constexpr int kNA = (kLimbs * BM * 4 + kThreads - 1) / kThreads;
    static constexpr int kNB = kQgBW * 2 / kThreads;
    static_assert(kWaves % kRowBlocks == 0 || kRowBlocks % kWaves == 0, "A row block per wave");
    static_assert(kBBlocks % kWaves == 0 && (kQgBW * 2) % kThreads == 0, "B split");
};
static_assert(QgShape<kQ8, kQgBM>::kLds <= 160 * 1024, "q8 128-row tile exceeds the LDS");
static_assert(QgShape<kQ8, kQgBMSmall>::kLds <= 160 * 1024, "q8 32-row tile exceeds the LDS");
static_assert(2 * QgShape<kQ4, kQgBMSmall>::kLds <= 160 * 1024, "two q4 32-row tiles per CU");

// s_waitcnt on the vector-memory counter only (gfx9 encoding: vmcnt in bits
// 3:0 and 15:14, expcnt 6:4 and lgkmcnt 11:8 left at their no-wait maxima).
template <int N> __device__ __forceinline__ void wait_vmcnt() {
    __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

// Workgroup over a BM x 256 tile (QgShape).  The 32-row tile serves
// batches whose experts hold few rows each: the MFMA work per weight byte is
// a quarter, so the tile is bound by the weight stream instead of by padding.
template <int FMT, bool DUAL, int BM>
__global__ __launch_bounds__((QgShape<FMT, BM>::kThreads),
                             (BM == 128 || QgShape<FMT, BM>::kRB == 128) ? 1 : 2) void qgemm_kernel(
    QGemmLaunch L) {
    extern __shared__ __attribute__((aligned(16))) int8_t qg_lds[];
    using Sh = QgShape<FMT, BM>;
    constexpr int kRB = Sh::kRB;
    constexpr int kStages = Sh::kStages;
    constexpr int kStage = Sh::kStage;
    constexpr int kLdsA = Sh::kLdsA;
    constexpr int kMI = Sh::kMI, kNF = Sh::kNF;
    constexpr bool kDma = FMT == kQ8;
    float *lds_scale = reinterpret_cast<float *>(qg_lds + kStages * kStage);
    int *lds_arow = reinterpret_cast<int *>(qg_lds + kStages * kStage + BM * 4);
    GemmTask tk;
    int m0, n0;
    if (!map_tile<DUAL, BM>(L, tk, m0, n0)) return;

    constexpr int kThreads = Sh::kThreads;
    const int tid = threadIdx.x;
    const int lane = tid & (kWave - 1);
    const int wave = tid >> 6;
    // 128-row tiles: the two waves that share a SIMD (waves w and w + 4)
    // take 32-row blocks from different halves of the tile (wm and wm + 2)
    // and the same weight rows, so that in a tile of at most 64 token rows
    // every SIMD still has one wave with products to run.
    const int wm = Sh::kWM == 4 ? (wave & 1) | ((wave >> 2) << 1) : wave % Sh::kWM;
    const int wn = Sh::kWM == 4 ? (wave >> 1) & 1 : wave / Sh::kWM;
    static_assert(Sh::kWM == 1 || (Sh::kWM == 4 && Sh::kWN == 2), "wave grid");
    // a wave whose 32 rows all lie past the task's end skips its products
    // (wave-uniform; it still issues its share of the copies and barriers)
    // (32-row tiles have one wave row: always live, no branch)
    const bool live =
        Sh::kWM == 1 || __builtin_amdgcn_readfirstlane(m0 + wm * (Sh::kMI * 32)) < tk.rows;

    if (tid < BM) {
        const int m = m0 + tid;
        int arow = -1;
        float sc = 0.0f;
        if (m < tk.rows) {
            arow = tk.a_rows ? tk.a_rows[m] : m;
            sc = tk.a_scale[arow];
        }
        lds_arow[tid] = arow;
        lds_scale[tid] = sc;
    }
    __syncthreads();

    // ---- per-thread global sources (fixed over k).  Rows past the task's end
    // read row m0 (A) or weight row 0 (B): their outputs are never stored.
    const int w_ld = tk.w_ld ? tk.w_ld : tk.k;
    const long w_row_bytes = FMT == kQ8 ? w_ld : w_ld / 2;
    const uint8_t *const w_gate = tk.w;
    const uint8_t *const w_up = tk.w2;
    // output / weight row held by LDS B row j: SwiGLU tiles give each wave
    // its kNF / 2 gate blocks and then the matching up blocks (kNF = 4:
    // blocks f = 0, 1 gate, 2, 3 up of a 128-row wave half; kNF = 2: block 0
    // gate, 1 up of a 64-row wave quarter)
    auto b_out = [&](int j, bool &up) -> int {
        if (!DUAL) {
            up = false;
            return n0 + j;
        }
        constexpr int kHalf = kNF / 2;
        const int f = (j >> 5) % kNF;
        up = f >= kHalf;
        return n0 + (j / (kNF * 32)) * (kHalf * 32) + (f % kHalf) * 32 + (j & 31);
    };
    auto b_row_src = [&](int j) -> const uint8_t * {
        bool up;
        const int out = b_out(j, up);
        return (up ? w_up : w_gate) + (long)(out < tk.n_out ? out : 0) * w_row_bytes;
    };
    // limb planes at a fixed distance: the limb of an address is arithmetic,
    // not a choice between pointers (which would put them in scratch memory)
    const int8_t *const a_base = tk.a;
    const long a_plane = tk.a_plane;
    auto limb_base = [a_base, a_plane](int limb) -> const int8_t * {
        return a_base + limb * a_plane;
    };
    auto a_row_src = [&](int limb, int r) -> const int8_t * {
        const int arow = lds_arow[r] >= 0 ? lds_arow[r] : lds_arow[0];
        return limb_base(limb) + (long)arow * tk.a_stride;
    };

    // DMA path (q8), blocks of R = 1024 / kRB rows = 1 KB: A block b holds
    // limb b / kRowBlocks, rows (b % kRowBlocks) * R + l / (kRB / 16); wave w
    // issues A blocks w, w + kWaves, ..., all in row block w % kRowBlocks,
    // and B blocks (rows (w + kWaves q) * R + l / (kRB / 16)); lane l fills
    // LDS row (block row 0 + l / (kRB / 16)), physical chunk l % (kRB / 16),
    // so it loads the logical chunk (l % (kRB / 16)) ^ g(row).  The limbs
    // share a lane's A rows.
    constexpr int kCh = kRB / 16;
    const int lr = lane / kCh, lc = lane % kCh;
    auto swz = [](int r) { return kRB == 64 ? (((r >> 1) ^ (r >> 3)) & 3) : ((r ^ (r >> 3)) & 7); };
    unsigned a_off = 0u;  // byte offset of this lane's A row
    // register path (q4, 64-byte rows): kNA A chunks and kNB packed B chunks
    constexpr int kNA = Sh::kNA, kNB = Sh::kNB;
    const int8_t *a_src[kNA];
    int a_dst[kNA];
    const uint8_t *b_src[kNB];
    int b_dst[kNB];
    u32x4 ra[kNA], rb[kNB];
    if constexpr (kDma) {
        const int r = (wave % Sh::kRowBlocks) * Sh::kRowsDma + lr;
        const int arow = lds_arow[r] >= 0 ? lds_arow[r] : lds_arow[0];
        a_off = (unsigned)(arow * tk.a_stride);
    } else {
#pragma unroll
        for (int q = 0; q < kNA; ++q) {
            const int c = min(tid + kThreads * q, kLimbs * BM * 4 - 1);
            const int limb = c / (4 * BM), r = (c >> 2) & (BM - 1), kc = c & 3;
            a_src[q] = a_row_src(limb, r) + kc * 16;
            a_dst[q] = limb * (BM * kRB) + lds_off<kRB>(r, kc);
        }
#pragma unroll
        for (int q = 0; q < kNB; ++q) {
            const int c = tid + kThreads * q;
            const int j = c >> 1, part = c & 1;  // 32 packed columns per part
            b_src[q] = b_row_src(j) + part * 16;
            b_dst[q] = (j << 1) | part;
        }
    }

    // one k slice of 64 into LDS stage buf (kDmaMin or kDmaMax DMA
    // instructions per wave)
    auto issue_dma = [&](int k0, int buf) {
        __attribute__((address_space(3))) int8_t *stage =
            (__attribute__((address_space(3))) int8_t *)(qg_lds + buf * kStage);
        constexpr int kRowBlocks = Sh::kRowBlocks;
#pragma unroll
        for (int h = 0; h < Sh::kAMax; ++h) {
            const int b = wave + Sh::kWaves * h;  // A block
            if (h >= Sh::kAMin && b >= Sh::kABlocks) break;  // wave-uniform
            const int limb = b / kRowBlocks, rb = b % kRowBlocks;
            const int r = rb * Sh::kRowsDma + lr;  // A row of this lane
            const int ca = lc ^ swz(r);
            // uniform base + 32-bit lane offset: one VGPR per address
            const unsigned aoff = a_off + (unsigned)(k0 + ca * 16);
            __builtin_amdgcn_global_load_lds(
                (const __attribute__((address_space(1))) void *)(limb_base(limb) + aoff),
                stage + b * 1024, 16, 0, 0);
        }
#pragma unroll
        for (int q = 0; q < Sh::kBPer; ++q) {
            const int bb = wave + Sh::kWaves * q;
            const int j = bb * Sh::kRowsDma + lr;  // B row of this lane
            bool up;
            const int out = b_out(j, up);
            const uint8_t *bbase = up ? w_up : w_gate;
            const int cb = lc ^ swz(j);
            const unsigned boff =
                (unsigned)((out < tk.n_out ? out : 0) * w_row_bytes) + (unsigned)(k0 + cb * 16);
            __builtin_amdgcn_global_load_lds(
                (const __attribute__((address_space(1))) void *)(bbase + boff),
                stage + kLdsA + bb * 1024, 16, 0, 0);
        }
    };
    auto fetch = [&](int k0) {
#pragma unroll
        for (int q = 0; q < kNA; ++q) ra[q] = load_global16(a_src[q] + k0);
#pragma unroll
        for (int q = 0; q < kNB; ++q) rb[q] = load_global16(b_src[q] + k0 / 2);
    };
    auto stash = [&](int buf) {
        int8_t *a = qg_lds + buf * kStage;
#pragma unroll
        for (int q = 0; q < kNA; ++q) *reinterpret_cast<u32x4 *>(a + a_dst[q]) = ra[q];
        int8_t *b = a + kLdsA;
#pragma unroll
        for (int q = 0; q < kNB; ++q) {
            const int j = b_dst[q] >> 1, part = b_dst[q] & 1;
            unsigned v[8];
            unpack_q4_word(rb[q].x, v[0], v[1]);
            unpack_q4_word(rb[q].y, v[2], v[3]);
            unpack_q4_word(rb[q].z, v[4], v[5]);
            unpack_q4_word(rb[q].w, v[6], v[7]);
            *reinterpret_cast<u32x4 *>(b + lds_off<kRB>(j, 2 * part)) =
                u32x4{v[0], v[1], v[2], v[3]};
            *reinterpret_cast<u32x4 *>(b + lds_off<kRB>(j, 2 * part + 1)) =
                u32x4{v[4], v[5], v[6], v[7]};
        }
    };

    i32x16 acc[kLimbs][kMI][kNF];  // [limb][row block][weight-row block]
#pragma unroll
    for (int a = 0; a < kLimbs; ++a)
#pragma unroll
        for (int i = 0; i < kMI; ++i)
#pragma unroll
            for (int f = 0; f < kNF; ++f)
#pragma unroll
                for (int r = 0; r < 16; ++r) acc[a][i][f][r] = 0;

    const int frow = lane & 31;
    const int half = lane >> 5;
    // two 32-wide k steps: all fragments are read before the first MFMA so
    // the LDS latency overlaps the MFMAs
    auto compute_pair = [&](int buf, int ksub0) {
        const int8_t *a0 = qg_lds + buf * kStage;
        const int8_t *bb = a0 + kLdsA;
        i32x4 fa[2][kLimbs][kMI], fb[2][kNF];
#pragma unroll
        for (int s2 = 0; s2 < 2; ++s2) {
            const int chunk = (ksub0 + s2) * 2 + half;
#pragma unroll
            for (int i = 0; i < kMI; ++i) {
                const int row = wm * (kMI * 32) + i * 32 + frow;
#pragma unroll
                for (int a = 0; a < kLimbs; ++a)
                    fa[s2][a][i] = *reinterpret_cast<const i32x4 *>(a0 + a * (BM * kRB) +
                                                                    lds_off<kRB>(row, chunk));
            }
#pragma unroll
            for (int f = 0; f < kNF; ++f) {
                const int row = wn * (kNF * 32) + f * 32 + frow;
                fb[s2][f] = *reinterpret_cast<const i32x4 *>(bb + lds_off<kRB>(row, chunk));
            }
        }
#pragma unroll
        for (int s2 = 0; s2 < 2; ++s2)
#pragma unroll
            for (int i = 0; i < kMI; ++i)
#pragma unroll
                for (int f = 0; f < kNF; ++f)
#pragma unroll
                    for (int a = 0; a < kLimbs; ++a)
                        acc[a][i][f] = __builtin_amdgcn_mfma_i32_32x32x32_i8(
                            fa[s2][a][i], fb[s2][f], acc[a][i][f], 0, 0, 0);
    };

    if constexpr (kDma) {
        // kStages stages: slices ks + 1 .. ks + kStages - 1 stream into LDS
        // while slice ks is multiplied.  A wave's DMA completes in order, its
        // kDmaMax or kDmaMin instructions per slice, so slice ks has landed
        // when at most that many for the later slice in flight remain; the
        // barrier after the wait makes every wave's part visible and frees
        // the stage of slice ks - 1 for slice ks + kStages - 1.
        static_assert(kStages == 3, "waits below assume one later slice in flight");
        const bool more = Sh::kDmaMax == Sh::kDmaMin ||
                          __builtin_amdgcn_readfirstlane(wave) + Sh::kWaves * Sh::kAMin <
                              Sh::kABlocks;
        const int nk = tk.k / kRB;  // k % kRB == 0 (qgemm_shape_ok, and the tile pickers for kRB = 128)
        for (int st = 0; st < kStages - 1 && st < nk; ++st) issue_dma(st * kRB, st);
        for (int ks = 0; ks < nk; ++ks) {
            if (ks + 1 < nk) {
                if (more) wait_vmcnt<Sh::kDmaMax>();
                else wait_vmcnt<Sh::kDmaMin>();
            } else {
                wait_vmcnt<0>();
            }
            // a bare barrier: __syncthreads() would also wait for the stores
            // and loads of the fence it implies
            __builtin_amdgcn_s_barrier();
            if (ks + kStages - 1 < nk) issue_dma((ks + kStages - 1) * kRB, (ks + kStages - 1) % kStages);
            if (live) {
#pragma unroll
                for (int kp = 0; kp < kRB / 32; kp += 2) compute_pair(ks % kStages, kp);
            }
        }
    } else {
        // two buffers: slice ks + 2 is in registers while slice ks is multiplied
        const int nk = tk.k / kRB;
        fetch(0);
        stash(0);
        if (nk > 1) fetch(kRB);
        __syncthreads();
        for (int ks = 0; ks < nk; ++ks) {
            if (live) compute_pair(ks & 1, 0);
            if (ks + 1 < nk) {
                stash((ks + 1) & 1);
                if (ks + 2 < nk) fetch((ks + 2) * kRB);
            }
            __syncthreads();
        }
    }

    // ---- epilogue.  Every global input of the epilogue (weight scales,
    // residual rows) is loaded before the first store: the stores may alias
    // them as far as the compiler knows, so a load after a store would wait
    // for it.
    constexpr int kF = DUAL ? kNF / 2 : kNF;
    float sw[kF], su[kF];
    int ncol[kF];
#pragma unroll
    for (int f = 0; f < kF; ++f) {
        ncol[f] = n0 + wn * kF * 32 + f * 32 + frow;
        const bool ok = ncol[f] < tk.n_out;
        sw[f] = ok ? load_global_f32(tk.s + ncol[f]) : 0.0f;
        su[f] = (DUAL && ok) ? load_global_f32(tk.s2 + ncol[f]) : 0.0f;
    }
    // row scales of the result rows this lane holds
    float sxr[kMI][16];
#pragma unroll
    for (int i = 0; i < kMI; ++i)
#pragma unroll
        for (int r = 0; r < 16; ++r)
            sxr[i][r] = lds_scale[wm * (kMI * 32) + i * 32 + (r >> 2) * 8 + half * 4 + (r & 3)];
    // complete the scale loads now: stores share the vector-memory counter,
    // so a wait placed after the first store would also wait for the stores
    __builtin_amdgcn_s_waitcnt(0);
    // 65536 hi + 256 mid + lo of one result register (the int32 sums are exact)
    auto limb_sum = [&](int i, int f, int r) -> float {
        return (float)acc[0][i][f][r] * 65536.0f +
               ((float)acc[1][i][f][r] * 256.0f + (float)acc[2][i][f][r]);
    };
    // the residual and plain paths are separate instantiations, so the plain
    // path carries no wait for residual loads (which would drain the stores)
    auto epilogue = [&](auto with_resid) {
        constexpr bool kResid = decltype(with_resid)::value;
#pragma unroll
        for (int i = 0; i < kMI; ++i) {
#pragma unroll
            for (int rg = 0; rg < 16; rg += 4) {
                // residual inputs of 4 result registers, loaded before their stores
                float res[4][kF];
                if (kResid) {
#pragma unroll
                    for (int r = rg; r < rg + 4; ++r) {
                        const int m = m0 + wm * (kMI * 32) + i * 32 + (r >> 2) * 8 + half * 4 + (r & 3);
#pragma unroll
                        for (int f = 0; f < kF; ++f)
                            res[r - rg][f] = (m < tk.rows && ncol[f] < tk.n_out)
                                                 ? load_global_f32(tk.resid +
                                                                   (long)m * tk.resid_stride +
                                                                   ncol[f])
                                                 : 0.0f;
                    }
                }
#pragma unroll
                for (int r = rg; r < rg + 4; ++r) {
                    const int m = m0 + wm * (kMI * 32) + i * 32 + (r >> 2) * 8 + half * 4 + (r & 3);
                    if (m >= tk.rows) continue;
                    const float sx = sxr[i][r];
                    float *yrow = tk.y + (long)m * tk.y_stride;
                    if (DUAL) {
#pragma unroll
                        for (int f = 0; f < kF; ++f) {
                            if (ncol[f] < tk.n_out) {
                                const float g = limb_sum(i, f, r) * sx * sw[f];
                                const float u = limb_sum(i, f + kF, r) * sx * su[f];
                                store_global(yrow + ncol[f], silu(g) * u);
                            }
                        }
                    } else {
#pragma unroll
                        for (int f = 0; f < kF; ++f) {
                            if (ncol[f] < tk.n_out) {
                                float v = limb_sum(i, f, r) * sx * sw[f];
                                if (kResid) v = res[r - rg][f] + v;
                                store_global(yrow + ncol[f], v);
                            }
                        }
                    }
                }
            }
        }
    };
    if (!DUAL && tk.resid) epilogue(std::true_type{});
    else epilogue(std::false_type{});
}

// ---------------------------------------------------------------------------
// Weight-streaming tile (launches whose tasks hold few token rows, e.g. the
// MoE layer of a decode batch): BM = 16 * MB token rows x 256 weight rows per
// workgroup, each of its 4 waves owning 64 weight rows (4 blocks of 16) for
// all BM rows, with no barrier.  Weights, read once, are the stream: a wave
// copies its rows into a private LDS ring by DMA, 128 contiguous bytes of a
// row per lane group (a DMA instruction covers 8 rows x 128 bytes: on MI355X
// a plain read of such runs moves ~6 TB/s, of the 64-byte pieces an MFMA
// fragment holds ~4.2 TB/s), kStages steps of 128 k ahead; the activation
// limbs of the BM rows (L2-resident, shared by every tile of the task) load
// straight into registers.  Products on v_mfma_i32_16x16x64_i8: lane l
// supplies row / column l % 16 and the 16 k values 16 (l / 16) .. + 15 of a
// 64-wide step, for activations (A) and weights (B) alike; result register r
// of lane l is C[4 (l / 16) + r][l % 16].
// ---------------------------------------------------------------------------

template <int FMT, int MB> struct QsShape {
    static constexpr int kBM = 16 * MB;
    static constexpr int kStages = 2;                  // 128-k steps in flight
    static constexpr int kRowBytes = FMT == kQ8 ? 128 : 64;  // weight bytes per row and step
    static constexpr int kWaveStage = 64 * kRowBytes;        // one wave's rows per step
    static constexpr int kLds = 4 * kStages * kWaveStage;
    // per lane and step: weight DMA (64 rows of kRowBytes, 1 KB per
    // instruction) + activation loads (2 slices x 3 limbs x MB row blocks)
    static constexpr int kDma = kWaveStage / 1024;
    static constexpr int kLoads = kDma + 2 * kLimbs * MB;
    static_assert((kStages - 1) * kLoads <= 63, "vmcnt range");
};

typedef unsigned u32x2 __attribute__((ext_vector_type(2)));

template <int FMT, bool DUAL, int MB>
__global__ __launch_bounds__(256, 2) void qgemm_stream_kernel(QGemmLaunch L) {
    using Sh = QsShape<FMT, MB>;
    constexpr int BM = Sh::kBM;
    constexpr int S = Sh::kStages;
    constexpr int NL = Sh::kLoads;
    constexpr int RB = Sh::kRowBytes;
    extern __shared__ __attribute__((aligned(16))) unsigned char qs_lds[];
    GemmTask tk;
    int m0, n0;
    if (!map_tile<DUAL, BM>(L, tk, m0, n0)) return;
    const int lane = threadIdx.x & (kWave - 1);
    const int wave = threadIdx.x >> 6;
    const int l16 = lane & 15, kq = lane >> 4;
    unsigned char *my_lds = qs_lds + wave * S * Sh::kWaveStage;

    // activation rows of this lane (A row l16 of each row block); rows past
    // the task's end read its first row (their results are never stored)
    const int8_t *a_src[MB];
#pragma unroll
    for (int i = 0; i < MB; ++i) {
        const int m = m0 + 16 * i + l16;
        const int mm = m < tk.rows ? m : m0;
        const int arow = tk.a_rows ? tk.a_rows[mm] : mm;
        a_src[i] = tk.a + (long)arow * tk.a_stride + 16 * kq;
    }
    // weight row of LDS row j (0..63) of this wave: SwiGLU tiles give a wave
    // 32 gate rows (LDS rows 0..31) and the matching 32 up rows (32..63)
    const int w_ld = tk.w_ld ? tk.w_ld : tk.k;
    const long w_row_bytes = FMT == kQ8 ? w_ld : w_ld / 2;
    auto w_row = [&](int j, int &n) -> const uint8_t * {
        const uint8_t *base = tk.w;
        if (DUAL) {
            n = n0 + wave * 32 + (j & 31);
            if (j >= 32) base = tk.w2;
        } else {
            n = n0 + wave * 64 + j;
        }
        const int nn = n < tk.n_out ? n : 0;
        return base + (long)nn * w_row_bytes;
    };
    // DMA lane roles: instruction d covers LDS rows 8 d .. 8 d + 7 (q8) or
    // 16 d .. 16 d + 15 (q4), lane l row (l / (RB / 16)), physical 16-byte
    // chunk l % (RB / 16), which holds the row's logical chunk
    // (l % (RB / 16)) ^ (row & 7) (q8; q4 rows of 4 chunks XOR row & 3)
    constexpr int kChunks = RB / 16;
    constexpr int kRowsPerDma = 64 / kChunks;
    const uint8_t *dma_src[Sh::kDma];
#pragma unroll
    for (int d = 0; d < Sh::kDma; ++d) {
        const int j = d * kRowsPerDma + lane / kChunks;
        int n;
        const uint8_t *row = w_row(j, n);
        const int logical = (lane % kChunks) ^ (j & (kChunks - 1));
        dma_src[d] = row + logical * 16;
    }
    const int nsteps = tk.k / 128;  // k % 64 == 0; an odd last half-step is handled below
    const int nk = tk.k / 64;
    i32x4 ra[S][2][kLimbs][MB];
    auto issue = [&](int step, int st) {
        __attribute__((address_space(3))) unsigned char *dst =
            (__attribute__((address_space(3))) unsigned char *)(my_lds + st * Sh::kWaveStage);
        const long koff = (long)step * RB;
#pragma unroll
        for (int d = 0; d < Sh::kDma; ++d)
            __builtin_amdgcn_global_load_lds(
                (const __attribute__((address_space(1))) void *)(dma_src[d] + koff),
                dst + d * 1024, 16, 0, 0);
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const int slice = min(2 * step + h, nk - 1);
#pragma unroll
            for (int a = 0; a < kLimbs; ++a)
#pragma unroll
                for (int i = 0; i < MB; ++i) {
                    const u32x4 v =
                        load_global16(a_src[i] + a * tk.a_plane + (long)slice * 64);
                    ra[st][h][a][i] = i32x4{(int)v.x, (int)v.y, (int)v.z, (int)v.w};
                }
        }
    };
    i32x4 acc[kLimbs][MB][4];
#pragma unroll
    for (int a = 0; a < kLimbs; ++a)
#pragma unroll
        for (int i = 0; i < MB; ++i)
#pragma unroll
            for (int f = 0; f < 4; ++f) acc[a][i][f] = i32x4{0, 0, 0, 0};
    // the two 64-wide slices of a step (nh = 1: only the first exists)
    auto compute = [&](int st, int nh) {
        const unsigned char *stage = my_lds + st * Sh::kWaveStage;
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            if (h >= nh) break;  // uniform
            i32x4 bw[4];
#pragma unroll
            for (int f = 0; f < 4; ++f) {
                const int j = f * 16 + l16;
                if constexpr (FMT == kQ8) {
                    const int phys = (h * 4 + kq) ^ (j & 7);
                    const u32x4 v = *reinterpret_cast<const u32x4 *>(stage + j * RB + phys * 16);
                    bw[f] = i32x4{(int)v.x, (int)v.y, (int)v.z, (int)v.w};
                } else {
                    // 8 packed bytes = the 16 k values of this lane
                    const int phys = (h * 2 + (kq >> 1)) ^ (j & 3);
                    const u32x2 v = *reinterpret_cast<const u32x2 *>(stage + j * RB + phys * 16 +
                                                                    (kq & 1) * 8);
                    unsigned o0, o1, o2, o3;
                    unpack_q4_word(v.x, o0, o1);
                    unpack_q4_word(v.y, o2, o3);
                    bw[f] = i32x4{(int)o0, (int)o1, (int)o2, (int)o3};
                }
            }
#pragma unroll
            for (int f = 0; f < 4; ++f)
#pragma unroll
                for (int i = 0; i < MB; ++i)
#pragma unroll
                    for (int a = 0; a < kLimbs; ++a)
                        acc[a][i][f] = __builtin_amdgcn_mfma_i32_16x16x64_i8(
                            ra[st][h][a][i], bw[f], acc[a][i][f], 0, 0, 0);
        }
    };
    const int steps = (nk + 1) / 2;  // the last step may hold one slice
    (void)nsteps;
#pragma unroll
    for (int j = 0; j < S; ++j)
        if (j < steps) issue(j, j);
    for (int t0 = 0; t0 < steps; t0 += S) {
#pragma unroll
        for (int j = 0; j < S; ++j) {
            const int t = t0 + j;
            if (t < steps) {  // uniform
                if (t + S - 1 < steps) wait_vmcnt<(S - 1) * NL>();
                else wait_vmcnt<0>();
                compute(j, min(2, nk - 2 * t));
                if (t + S < steps) issue(t + S, j);
            }
        }
    }

    // ---- epilogue: lane l holds C[4 (l / 16) + r][l % 16] of each block
    constexpr int kF = DUAL ? 2 : 4;
    int ncol[kF];
    float sw[kF], su[kF];
#pragma unroll
    for (int f = 0; f < kF; ++f) {
        w_row(f * 16 + l16, ncol[f]);
        const bool ok = ncol[f] < tk.n_out;
        sw[f] = ok ? load_global_f32(tk.s + ncol[f]) : 0.0f;
        su[f] = (DUAL && ok) ? load_global_f32(tk.s2 + ncol[f]) : 0.0f;
    }
    float sx[MB][4];
#pragma unroll
    for (int i = 0; i < MB; ++i)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int m = m0 + 16 * i + 4 * kq + r;
            const int mm = m < tk.rows ? m : m0;
            sx[i][r] = load_global_f32(tk.a_scale + (tk.a_rows ? tk.a_rows[mm] : mm));
        }
    __builtin_amdgcn_s_waitcnt(0);
    auto limb_sum = [&](int i, int f, int r) -> float {
        return (float)acc[0][i][f][r] * 65536.0f +
               ((float)acc[1][i][f][r] * 256.0f + (float)acc[2][i][f][r]);
    };
    const bool resid = !DUAL && tk.resid;
#pragma unroll
    for (int i = 0; i < MB; ++i)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int m = m0 + 16 * i + 4 * kq + r;
            if (m >= tk.rows) continue;
            float *yrow = tk.y + (long)m * tk.y_stride;
#pragma unroll
            for (int f = 0; f < kF; ++f) {
                if (ncol[f] >= tk.n_out) continue;
                if (DUAL) {
                    const float g = limb_sum(i, f, r) * sx[i][r] * sw[f];
                    const float u = limb_sum(i, f + 2, r) * sx[i][r] * su[f];
                    store_global(yrow + ncol[f], silu(g) * u);
                } else {
                    float v = limb_sum(i, f, r) * sx[i][r] * sw[f];
                    if (resid)
                        v = load_global_f32(tk.resid + (long)m * tk.resid_stride + ncol[f]) + v;
                    store_global(yrow + ncol[f], v);
                }
            }
        }
}

template <int FMT, bool DUAL, int BM>
static void launch_qgemm(const QGemmLaunch &L, int grid, hipStream_t stream) {
    constexpr int kLds = QgShape<FMT, BM>::kLds;
    static const bool attr = [] {
        return hipFuncSetAttribute(reinterpret_cast<const void *>(&qgemm_kernel<FMT, DUAL, BM>),
                                   hipFuncAttributeMaxDynamicSharedMemorySize,
                                   kLds) == hipSuccess;
    }();
    (void)attr;
    hipLaunchKernelGGL((qgemm_kernel<FMT, DUAL, BM>), dim3((unsigned)grid),
                       dim3(QgShape<FMT, BM>::kThreads), kLds, stream, L);
}

template <int BM>
static void launch_qgemm_bm(int fmt, bool dual, const QGemmLaunch &L, int grid,
                            hipStream_t stream) {
    if (fmt == kQ8) {
        if (dual) launch_qgemm<kQ8, true, BM>(L, grid, stream);
        else launch_qgemm<kQ8, false, BM>(L, grid, stream);
    } else {
        if (dual) launch_qgemm<kQ4, true, BM>(L, grid, stream);
        else launch_qgemm<kQ4, false, BM>(L, grid, stream);
    }
}

template <int FMT, bool DUAL, int MB>
static void launch_stream(const QGemmLaunch &L, int grid, hipStream_t stream) {
    constexpr int kLds = QsShape<FMT, MB>::kLds;
    static const bool attr = [] {
        return hipFuncSetAttribute(
                   reinterpret_cast<const void *>(&qgemm_stream_kernel<FMT, DUAL, MB>),
                   hipFuncAttributeMaxDynamicSharedMemorySize, kLds) == hipSuccess;
    }();
    (void)attr;
    hipLaunchKernelGGL((qgemm_stream_kernel<FMT, DUAL, MB>), dim3((unsigned)grid), dim3(256),
                       kLds, stream, L);
}

template <int MB>
static void launch_stream_mb(int fmt, bool dual, const QGemmLaunch &L, int grid,
                             hipStream_t stream) {
    if (fmt == kQ8) {
        if (dual) launch_stream<kQ8, true, MB>(L, grid, stream);
        else launch_stream<kQ8, false, MB>(L, grid, stream);
    } else {
        if (dual) launch_stream<kQ4, true, MB>(L, grid, stream);
        else launch_stream<kQ4, false, MB>(L, grid, stream);
    }
}

// Tile kinds: the weight-streaming tile with 16 token rows, the LDS tiles
// with 32 or 128.
enum TileKind { kTileStream16 = 0, kTileLds32 = 1, kTileLds128 = 2 };

static int tile_bm(int kind) {
    return kind == kTileStream16 ? 16 : (kind == kTileLds128 ? kQgBM : kQgBMSmall);
}

// Tile choices, measured on MI355X.  A batch of at most 16 token rows streams
// the weights (every task fits one row tile); the streaming tile and the q8
// 32-row tile copy 128 k per step, so they need reductions that are whole
// multiples of 128 (`k128`; otherwise the 128-row tile runs).
// MoE layer: 16-row streaming tile up to 16 rows (T = 8: 99 against 108 us
// on the 32-row LDS tile), the 32-row LDS tile up to 80 rows per expert on
// average (T = 64: 170 against 180 us streaming), 128 rows above.  Dense
// projections: the 32-row tile up to 64 rows.
static int moe_tile(int fmt, int rows, double rows_per_expert, bool k128) {
    if (k128 && rows <= 16) return kTileStream16;
    const bool small_ok = fmt == kQ4 || k128;  // the q8 32-row tile steps 128 k
    return small_ok && rows_per_expert <= 80.0 ? kTileLds32 : kTileLds128;
}
// Dense projections whose 128-row tiles would cover at most half the CUs
// (o_proj and the dense down projection at 2048 rows: 128 tiles) take the
// 32-row tile too: 52.8 against 58.4 us for o_proj at 2048 rows; at 240
// tiles (`[q; kv_a]`) the 32-row tile measured 75.1 against 51.1 us.
static int dense_tile(int fmt, int rows, bool k128, int n_out, bool dual) {
    if (k128 && rows <= 16) return kTileStream16;
    const bool small_ok = fmt == kQ4 || k128;
    const int outw = dual ? kQgBW / 2 : kQgBW;
    const long t128 = (long)((rows + kQgBM - 1) / kQgBM) * ((n_out + outw - 1) / outw);
    return small_ok && (rows <= 2 * kQgBMSmall || t128 <= 128) ? kTileLds32 : kTileLds128;
}

static int launch_qgemm_fmt(int fmt, bool dual, int kind, const QGemmLaunch &L, int tiles_bound,
                            hipStream_t stream) {
    if (tiles_bound <= 0) return kOk;
    if (fmt != kQ8 && fmt != kQ4) return kErrArgs;
    const int grid = ((tiles_bound + 7) / 8) * 8;
    switch (kind) {
    case kTileStream16: launch_stream_mb<1>(fmt, dual, L, grid, stream); break;
    case kTileLds32: launch_qgemm_bm<kQgBMSmall>(fmt, dual, L, grid, stream); break;
    case kTileLds128: launch_qgemm_bm<kQgBM>(fmt, dual, L, grid, stream); break;
    default: return kErrArgs;
    }
    return hipGetLastError() == hipSuccess ? kOk : kErrLaunch;
}

static int host_tiles(bool dual, int rows, int n_out, int bm) {
    const int outw = dual ? kQgBW / 2 : kQgBW;
    return ((rows + bm - 1) / bm) * ((n_out + outw - 1) / outw);
}

int qgemm_single(int fmt, bool dual, const GemmTask &task, hipStream_t stream) {
    if (!qgemm_shape_ok(fmt, task.k) || task.rows <= 0 || task.n_out <= 0 || !task.w ||
        !task.s || !task.a || task.a_plane < (long)task.rows * task.a_stride || !task.a_scale ||
        !task.y ||
        (dual && (!task.w2 || !task.s2)) || task.a_stride % 16)
        return kErrArgs;
    QGemmLaunch L;
    L.single = task;
    const int kind = dense_tile(fmt, task.rows, task.k % 128 == 0, task.n_out, dual);
    return launch_qgemm_fmt(fmt, dual, kind, L,
                            host_tiles(dual, task.rows, task.n_out, tile_bm(kind)), stream);
}

// ---------------------------------------------------------------------------
// MoE prefill: device-built task tables
// ---------------------------------------------------------------------------

struct MoeScheduleParams {
    MoeGemmParams p;
    int bm;  // token rows per tile of the launches that read the tables
};

// Tasks of the shared down projection: 2 k halves when its width is twice
// inter and a second output exists, else 1.
__host__ __device__ inline int moe_shared_down_parts(const MoeGemmParams &p) {
    return p.has_shared && p.shared_out2 && p.shared_width == 2 * p.inter ? 2 : 1;
}

// With L (routing in the same workgroup) the route tables and the expert
// table (ew_lds, [experts]) come from LDS instead of global memory.  Called
// by whole workgroups of at least two waves.
__device__ __forceinline__ void moe_schedule_body(const MoeScheduleParams &sp,
                                                  const RouteLds *L = nullptr,
                                                  const ExpertWeights *ew_lds = nullptr) {
    const MoeGemmParams &p = sp.p;
    const int bm = sp.bm;
    auto tiles_rt = [bm](bool dual, int rows, int n_out) {
        const int outw = dual ? kQgBW / 2 : kQgBW;
        return ((rows + bm - 1) / bm) * ((n_out + outw - 1) / outw);
    };
    __shared__ int tiles[2][kQgMaxTasks];
    const int nr = L ? L->unique_total : *p.n_unique;
    GemmTask *t0 = p.tasks;
    GemmTask *t1 = p.tasks + kQgMaxTasks;
    for (int u = threadIdx.x; u < nr; u += blockDim.x) {
        const int e = L ? L->unique[u] : p.unique[u];
        const int cnt = L ? L->counts[e] : p.counts[e], off = L ? L->offsets[e] : p.offsets[e];
        const ExpertWeights ew = ew_lds ? ew_lds[e] : p.expert_table[e];
        GemmTask a;
        a.w = ew.gate;
        a.w2 = ew.up;
        a.s = ew.gate_s;
        a.s2 = ew.up_s;
        a.rows = cnt;
        a.n_out = p.inter;
        a.k = p.hidden;
        a.a = p.xq;
        a.a_plane = p.xq_plane;
        a.a_scale = p.xq_scale;
        a.a_stride = p.hidden;
        a.a_rows = p.list_rows + off;
        a.y = p.expert_hidden + (long)off * p.inter;
        a.y_stride = p.inter;
        t0[u] = a;
        tiles[0][u] = tiles_rt(true, cnt, p.inter);
        GemmTask b;
        b.w = ew.down;
        b.s = ew.down_s;
        b.rows = cnt;
        b.n_out = p.hidden;
        b.k = p.inter;
        b.a = p.hq + (long)off * p.inter;
        b.a_plane = p.hq_plane;
        b.a_scale = p.hq_scale + off;
        b.a_stride = p.inter;
        b.y = p.expert_out + (long)off * p.hidden;
        b.y_stride = p.hidden;
        t1[u] = b;
        tiles[1][u] = tiles_rt(false, cnt, p.hidden);
    }
    const int nsd = moe_shared_down_parts(p);  // shared down tasks (k parts)
    if (threadIdx.x == 0) {
        tiles[0][nr] = 0;
        for (int i = 0; i < nsd; ++i) tiles[1][nr + i] = 0;
        if (p.has_shared) {
            GemmTask a;
            a.w = p.shared_gate;
            a.w2 = p.shared_up;
            a.s = p.shared_gate_s;
            a.s2 = p.shared_up_s;
            a.rows = p.rows;
            a.n_out = p.shared_width;
            a.k = p.hidden;
            a.a = p.xq;
            a.a_plane = p.xq_plane;
            a.a_scale = p.xq_scale;
            a.a_stride = p.hidden;
            a.y = p.shared_hidden;
            a.y_stride = p.shared_width;
            t0[nr] = a;
            tiles[0][nr] = tiles_rt(true, p.rows, p.shared_width);
            // the shared down projection as nsd k parts of `inter` columns
            // (its tiles then last as long as the routed ones'), part i into
            // shared_out (i = 0) or shared_out2 (i = 1)
            const int kpart = p.shared_width / nsd;
            for (int i = 0; i < nsd; ++i) {
                GemmTask b;
                const long col = (long)i * kpart;
                b.w = p.shared_down + (p.shared_fmt == kQ8 ? col : col / 2);
                b.s = p.shared_down_s;
                b.rows = p.rows;
                b.n_out = p.hidden;
                b.k = kpart;
                b.w_ld = p.shared_width;
                b.a = p.sq + col;
                b.a_plane = p.sq_plane;
                b.a_scale = p.sq_scale;
                b.a_stride = p.shared_width;
                b.y = i == 0 ? p.shared_out : p.shared_out2;
                b.y_stride = p.hidden;
                t1[nr + i] = b;
                tiles[1][nr + i] = tiles_rt(false, p.rows, p.hidden);
            }
        }
    }
    lds_barrier();  // the tables are read by the next launch
    // tile prefix sums tile_start[u] = sum of tiles[s][v < u], u = 0..n: wave
    // s scans stage s, kPer consecutive entries per lane (one round of
    // independent LDS reads) and a wave scan over the lanes' sums (a loop of
    // dependent LDS reads per entry waited for each read in turn)
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    if (wave < 2) {
        const int s = wave;
        const int n = nr + (s == 0 ? 1 : nsd);  // tiles[s][0 .. n - 1] are set
        constexpr int kPer = (kQgMaxTasks + 1 + 63) / 64;
        int v[kPer], local = 0;
#pragma unroll
        for (int i = 0; i < kPer; ++i) {
            const int u = lane * kPer + i;
            v[i] = tiles[s][u < n ? u : 0];
            v[i] = u < n ? v[i] : 0;
            local += v[i];
        }
        int incl = local;
#pragma unroll
        for (int o = 1; o < 64; o <<= 1) {
            const int up = __shfl_up(incl, o, 64);
            if (lane >= o) incl += up;
        }
        int run = incl - local;
#pragma unroll
        for (int i = 0; i < kPer; ++i) {
            const int u = lane * kPer + i;
            if (u <= n) p.tile_start[s * (kQgMaxTasks + 1) + u] = run;
            run += v[i];
        }
    }
}

// The token-row quantisation of the MoE input (RMSNorm'ed) and, in the last
// workgroup, the GEMM task and tile tables: one launch before stage 0.  Eight
// waves: a row each to quantise, or to route (the routing workgroup).
constexpr int kPrepWaves = 8;
static_assert(kPrepWaves >= 2, "moe_schedule_body scans with two waves");
template <bool REG>
__global__ __launch_bounds__(64 * kPrepWaves) void moe_prep_kernel(QuantSeg a, MoeScheduleParams sp,
                                                                   int blocks_a) {
    if ((int)blockIdx.x == blocks_a) {
        if (sp.p.route_in_prep) {
            // route_kernel's work: selection (wave w: row w), the route tables
            // kept in LDS for the schedule, the expert table staged in LDS
            // meanwhile
            __shared__ RouteLds L;
            __shared__ ExpertWeights ew[64];
            __shared__ __align__(16) unsigned long long keys[kPrepWaves][64];
            const RouteParams &rp = sp.p.route;  // rows <= kPrepWaves, experts <= 64
            const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
            if (wave == 0 && lane < rp.experts) ew[lane] = sp.p.expert_table[lane];
            if (wave < rp.rows) (void)select_row_64(rp, wave, lane, L.ids, keys[wave]);
            lds_barrier();
            small_tables(rp, L);
            lds_barrier();
            moe_schedule_body(sp, &L, ew);
            return;
        }
        moe_schedule_body(sp);
        return;
    }
    const int row = (int)blockIdx.x * kPrepWaves + (int)(threadIdx.x >> 6);
    if (row >= a.rows) return;
    quantize_row<REG>(a, row);
}


int moe_gemm(const MoeGemmParams &p, hipStream_t stream) {
    if (p.rows <= 0 || p.experts <= 0 || p.experts + 2 > kQgMaxTasks || p.top_k <= 0 ||
        !qgemm_shape_ok(p.expert_fmt, p.hidden) || !qgemm_shape_ok(p.expert_fmt, p.inter) ||
        (p.has_shared && (!qgemm_shape_ok(p.shared_fmt, p.hidden) ||
                          !qgemm_shape_ok(p.shared_fmt, p.shared_width))))
        return kErrArgs;
    const int entries = p.rows * p.top_k;
    const int max_tasks = entries < p.experts ? entries : p.experts;
    // one tile kind for the whole layer, from the average rows per expert
    const bool k128 = p.hidden % 128 == 0 && p.inter % 128 == 0 &&
                      (!p.has_shared || p.shared_width % 128 == 0);
    const bool any_q8 = p.expert_fmt == kQ8 || (p.has_shared && p.shared_fmt == kQ8);
    const int kind = moe_tile(any_q8 ? kQ8 : kQ4, p.rows, (double)entries / p.experts, k128);
    const int bm = tile_bm(kind);
    MoeScheduleParams sp;
    sp.p = p;
    sp.bm = bm;
    // token rows (RMSNorm'ed) into limbs, and the task / tile tables in the
    // launch's last workgroup
    QuantSeg xs;
    xs.x = p.x;
    xs.x_stride = p.hidden;
    xs.rows = p.rows;
    xs.width = p.hidden;
    xs.norm_w = p.norm_w;
    xs.eps = p.eps;
    xs.q = p.xq;
    xs.plane = p.xq_plane;
    xs.scale = p.xq_scale;
    if (!p.x || !p.xq || !p.xq_scale || !quant_seg_ok(xs))
        return kErrArgs;
    if (p.route_in_prep &&
        (p.route.rows != p.rows || p.rows > kRouteOneGroupRows || !p.route.logits ||
         p.route.experts != p.experts || p.route.top_k != p.top_k || p.top_k > kMaxTopK ||
         p.experts > 64 || p.rows * p.top_k > kRouteFusedMaxPositions ||
         !p.route.ids || !p.route.weights || !p.route.n_unique || !p.route.unique ||
         !p.route.counts || !p.route.offsets || !p.route.list_rows || !p.route.list_slots ||
         !p.route.list_pos || !p.route.error))
        return kErrArgs;
    static_assert(kRouteOneGroupRows <= kPrepWaves, "a wave per routed row");
    const int blocks_x = (p.rows + kPrepWaves - 1) / kPrepWaves;
    if (p.hidden <= kQuantRegChunks * kWave * 4)
        hipLaunchKernelGGL(moe_prep_kernel<true>, dim3(blocks_x + 1), dim3(64 * kPrepWaves), 0,
                           stream, xs, sp, blocks_x);
    else
        hipLaunchKernelGGL(moe_prep_kernel<false>, dim3(blocks_x + 1), dim3(64 * kPrepWaves), 0,
                           stream, xs, sp, blocks_x);
    if (hipGetLastError() != hipSuccess) return kErrLaunch;
    int st = kOk;

    const bool same = !p.has_shared || p.shared_fmt == p.expert_fmt;
    for (int stage = 0; stage < 2; ++stage) {
        const bool dual = stage == 0;
        QGemmLaunch L;
        L.tasks = p.tasks + stage * kQgMaxTasks;
        L.tile_start = p.tile_start + stage * (kQgMaxTasks + 1);
        L.n_routed = p.n_unique;
        L.n_shared = dual ? 1 : moe_shared_down_parts(p);
        // upper bounds of the tile counts: sum_e ceil(n_e / BM) <= entries / BM + tasks
        const int routed_mt = entries / bm + max_tasks;
        const int routed_nt = host_tiles(dual, 1, dual ? p.inter : p.hidden, bm);
        const int shared_t =
            p.has_shared ? L.n_shared * host_tiles(dual, p.rows, dual ? p.shared_width : p.hidden, bm)
                         : 0;
        if (same) {
            L.range = 0;
            st = launch_qgemm_fmt(p.expert_fmt, dual, kind, L, routed_mt * routed_nt + shared_t,
                                  stream);
        } else {
            L.range = 1;
            st = launch_qgemm_fmt(p.expert_fmt, dual, kind, L, routed_mt * routed_nt, stream);
            if (!st) {
                L.range = 2;
                st = launch_qgemm_fmt(p.shared_fmt, dual, kind, L, shared_t, stream);
            }
        }
        if (st) return st;
        if (stage == 0) {
            // the expert hidden rows and the shared hidden rows in one launch
            QuantSeg hs, ss;
            hs.x = p.expert_hidden;
            hs.x_stride = p.inter;
            hs.rows = entries;
            hs.width = p.inter;
            hs.q = p.hq;
            hs.plane = p.hq_plane;
            hs.scale = p.hq_scale;
            if (p.has_shared) {
                ss.x = p.shared_hidden;
                ss.x_stride = p.shared_width;
                ss.rows = p.rows;
                ss.width = p.shared_width;
                ss.q = p.sq;
                ss.plane = p.sq_plane;
                ss.scale = p.sq_scale;
            }
            st = quantize_segments(hs, ss, stream);
            if (st) return st;
        }
    }
    return kOk;
}

}  // namespace mlh
