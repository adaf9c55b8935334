// W8A8 fp8 GEMM with the weights pre-arranged in MFMA fragment order:
//   out[m, n] = (sum_k a[m, k] * w[n, k]) * sa[m] * sb[n]
// Same arithmetic, epilogue variants and results as gemm_fp8.hip
// (python/flashrec/kernel/sglops.py:99-140, fp8_scaled_mm); the difference
// is where the weight bytes travel.
//
// Weights are static, so they are rearranged once (fr_fp8_weight_prearrange)
// into blocks of 32 rows x 64 bytes of K, each block stored as the two 1 KB
// halves a wave's MFMA operand registers hold:
//   pre[((n / 32) * KT + k / 64) * 2048 + h * 1024 + l * 16 + b]
//     = w[32 * (n / 32) + l % 32][64 * (k / 64) + 32 * (l / 32) + 16 * h + b]
// for lane l, half h, byte b (KT = K steps rounded up to a multiple of 4,
// rows and K past the matrix zero).  Every weight load is then one 1 KB
// contiguous run straight into VGPRs: no LDS write, no LDS read, and a
// wave's next three steps of weights in flight in registers.
//
// Design (gfx950):
//  * Persistent, one 256-thread workgroup per CU, XCD-aware tile order (as
//    gemm_fp8.hip).
//  * 4 waves side by side along n: wave w owns weight rows [w*WN, w*WN+WN)
//    of the tile and all BM activation rows, so no two waves need the same
//    weight bytes and only the activations are shared through LDS.
//  * Activations: an LDS ring of NSL slots of BM rows x 128 bytes of K
//    (two MFMA steps per slot), filled by direct-to-LDS loads; half the
//    direct-to-LDS traffic of the two-operand ring, and a ring twice as
//    deep in the same LDS.
//  * MFMA v_mfma_scale_f32_32x32x64_f8f6f4, weights as the A operand (rows =
//    output columns), activations as B.  Per step a wave issues FN x FM MFMAs
//    activation-block-major; each activation block's next-step fragment is
//    read from LDS right after its last MFMA of the step (one register set).
//  * Weights: 4 register sets; step s issues the loads of step s + 3.
//  * Multi-round launches give each XCD a slice of n-tiles, walked m-major.
#include "gemm_common.h"

namespace fr {

constexpr int kPreBlockBytes = 2048;  // 32 rows x 64 bytes of K
constexpr int kPreSteps = 4;          // K steps per prearranged group (KT is a multiple)

// KT for a K: 64-byte steps, rounded up to a multiple of kPreSteps.
inline int64_t pre_k_steps(int64_t K) { return ((K + 64 * kPreSteps - 1) / (64 * kPreSteps)) * kPreSteps; }

// One thread per 16-byte chunk of the prearranged buffer.
__global__ __launch_bounds__(256) void fp8_weight_prearrange(const uint8_t* __restrict__ w, int64_t ldw, int64_t N,
                                                             int64_t K, int64_t KT, uint8_t* __restrict__ out,
                                                             int64_t chunks) {
  const int64_t c = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (c >= chunks) return;
  const int l = static_cast<int>(c & 63);
  const int h = static_cast<int>((c >> 6) & 1);
  const int64_t bk = c >> 7;  // block * KT + k step
  const int64_t blk = bk / KT, kt = bk % KT;
  const int64_t n = 32 * blk + (l & 31);
  const int64_t k0 = 64 * kt + 32 * (l >> 5) + 16 * h;
  u32x4 v = {0u, 0u, 0u, 0u};
  if (n < N) {
    const uint8_t* src = w + n * ldw + k0;
    if (k0 + 16 <= K && (reinterpret_cast<uintptr_t>(src) & 15u) == 0) {
      v = *reinterpret_cast<const u32x4*>(src);
    } else {
      uint8_t b[16];
#pragma unroll
      for (int i = 0; i < 16; ++i) b[i] = k0 + i < K ? src[i] : 0;
      v = __builtin_bit_cast(u32x4, b);
    }
  }
  *reinterpret_cast<u32x4*>(out + 16 * c) = v;
}

// Tile order of a multi-round launch: XCD x (workgroups i with i % 8 == x)
// owns the n-tiles [x * tilesN / 8, (x + 1) * tilesN / 8) over all m-tiles,
// walked m-major, so every round of that XCD revisits one weight slice (3 MB
// at the config-1 shape) while the activation panels stream past (1-6 %
// faster than the m-grouped order on the multi-round shapes measured).
// Single-round launches (and n-tile counts that do not split over 8
// XCDs) keep the m-grouped order of tile_coords.
__device__ __forceinline__ void tile_coords_pre(int64_t pid, int64_t nt, int64_t tilesM, bool multi_round,
                                                int64_t& tm, int64_t& tn) {
  const int64_t tilesN = nt / tilesM;
  if (multi_round && (tilesN & 7) == 0) {
    const int64_t x = pid & 7, p = pid >> 3, nper = tilesN >> 3;
    tn = x * nper + p % nper;
    tm = p / nper;
    return;
  }
  tile_coords(pid, nt, tilesM, tm, tn);
}

// BN: weight rows (output columns) per tile, BM: activation rows, NSL: ring
// slots, KTAIL: K % 256 != 0 (activation chunks past K read as zero: the
// prearranged K steps come in groups of 4), EPI: epilogue variant, WS: weight
// register sets (step s loads step s + WS - 1's weights).
template <int BN, int BM, int NSL, int OUT, bool KTAIL, int EPI, int WS>
__global__ __launch_bounds__(256, 1) void gemm_fp8_pre(GemmArgs g) {
#if defined(__HIP_DEVICE_COMPILE__)
  constexpr int RB = 128;        // bytes of K per LDS row: two MFMA steps per slot
  constexpr int WN = BN / 4;     // output columns per wave
  constexpr int WM = BM;         // output rows per wave
  constexpr int FN = WN / 32;    // weight blocks per wave
  constexpr int FM = WM / 32;    // activation blocks
  constexpr int RPI = 1024 / RB; // rows one 1 KB direct-to-LDS load covers
  constexpr int CPR = RB / 16;   // 16-byte chunks per LDS row
  constexpr int IA = BM * RB / 4096;  // activation loads per wave per slot
  constexpr int STAGE = BM * RB;
  constexpr int WL = 2 * FN;          // weight loads per wave per step
  constexpr int EB = OutT<OUT>::kBytes;
  constexpr bool SILU = EPI == kEpiSilu;
  static_assert(!SILU || OUT == FR_DTYPE_BF16, "SiLU epilogue writes bf16");
  static_assert(FN >= 1 && FM >= 1 && BN % 128 == 0 && BM % 32 == 0, "tile shape");
  static_assert(NSL >= 3, "the slot waits below assume at least three slots");
  constexpr int kLds = 160 * 1024;
  // scale buffer per tile parity: sb[BN], then sa[BM] from the next 1 KB
  constexpr int SBB = (BN * 4 + 1023) / 1024, SAB = (BM * 4 + 1023) / 1024;  // 1 KB loads of each
  constexpr int SCB = 1024 * (SBB + SAB);
  constexpr bool kNarrow = NSL * STAGE + 2 * SCB + 4 * 32 * 128 > kLds || WN % (128 / EB) != 0;
  constexpr int SRB = kNarrow ? 64 : 128;
  constexpr int STG = 32 * SRB;
  static_assert(NSL * STAGE + 2 * SCB + 4 * STG <= kLds, "LDS");
  __shared__ __attribute__((aligned(1024))) uint8_t smem[NSL * STAGE + 2 * SCB + 4 * STG];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wn = wave, wm = 0;

  const int64_t tilesN = (g.N + BN - 1) / BN;
  const int64_t tilesM = (g.M + BM - 1) / BM;
  const int64_t nt = tilesN * tilesM;
  const int64_t G = gridDim.x;
  const int64_t my_tiles = (nt - blockIdx.x + G - 1) / G;
  const bool multi_round = nt > G && (G & 7) == 0;
  // K steps per tile: the prearranged layout's (a multiple of 4, >= K / 64)
  const uint32_t wblk = static_cast<uint32_t>(g.ldb);  // bytes per 32-row weight block
  const int KT = static_cast<int>(wblk / kPreBlockBytes);
  const int KS = KT / 2;  // ring slots per tile
  if (my_tiles <= 0 || KT <= 0) return;

  const int64_t nblk = (g.N + 31) / 32;
  const __amdgpu_buffer_rsrc_t rw = make_rsrc(g.b, static_cast<uint32_t>(nblk * wblk));
  const __amdgpu_buffer_rsrc_t ra = make_rsrc(g.a, static_cast<uint32_t>((g.M - 1) * g.lda + g.K));

  // ---- activation ring (as gemm_fp8.hip with 128-byte rows): lane L of a
  // 1 KB load lands in row L / 8, chunk slot L % 8, fetching global chunk
  // (L % 8) ^ ((row / 2) % 8); row bit 3 is the wave's parity.
  const int lrow = lane / CPR;
  const int lchunk = (lane % CPR) ^ swz_g8(lrow + 8 * (wave & 1));
  constexpr uint32_t kOOB = 0x80000000u;
  uint32_t loa[IA];
#pragma unroll
  for (int i = 0; i < IA; ++i) loa[i] = static_cast<uint32_t>(((i * 4 + wave) * RPI + lrow) * g.lda + lchunk * 16);
  // scalar activation tile bases, per-lane weight offsets (lane * 16 plus
  // the wave's first weight block of the tile), for the current and next tile
  uint32_t ba_cur, ba_nxt, wv_cur, wv_nxt;
  auto tile_bases = [&](int64_t local, uint32_t& ba, uint32_t& wv) __attribute__((always_inline)) {
    if (local >= my_tiles) {
      ba = wv = kOOB;
      return;
    }
    int64_t tm, tn;
    tile_coords_pre(blockIdx.x + local * G, nt, tilesM, multi_round, tm, tn);
    ba = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(tm * BM * g.lda));
    wv = static_cast<uint32_t>((tn * (BN / 32) + wave * FN) * wblk) + 16 * lane_id_here();
  };
  auto issue_a = [&](int slot, int lk, bool next, int i) __attribute__((always_inline)) {
    uint8_t* sa = smem + slot * STAGE;
    const uint32_t k0 = static_cast<uint32_t>(lk) * RB;
    const bool kin = !KTAIL || (k0 + lchunk * 16 < static_cast<uint64_t>(g.K));
    const uint32_t o = loa[i] + (next ? ba_nxt : ba_cur);
    __builtin_amdgcn_raw_ptr_buffer_load_lds(ra, (lds_ptr_t)(sa + (i * 4 + wave) * 1024), 16, kin ? o : kOOB, k0,
                                             0, 0);
  };

  // ---- weight registers: wr[set][block][half]
  u32x4 wr[WS][FN][2];
  // load `l` (block l / 2, half l % 2) of K step kt of the cur / nxt tile
  auto issue_w = [&](int set, int kt, bool next, int l) __attribute__((always_inline)) {
    const int i = l >> 1, h = l & 1;
    // the block offset rides in the per-lane offset, which the buffer range
    // check covers (a block past the last one reads zeros); the K step in
    // the scalar offset stays inside its block
    const uint32_t vo = (next ? wv_nxt : wv_cur) + i * wblk + h * 1024;
    wr[set][i][h] = __builtin_bit_cast(
        u32x4, __builtin_amdgcn_raw_buffer_load_b128(rw, vo, static_cast<int>(kt * kPreBlockBytes), 0));
  };

  // ---- activation fragments (one set; block j of the next step is read
  // right after the last MFMA that uses block j of the current one)
  const int fr = lane & 31;
  const int c0 = (lane >> 5) * 2;
  u32x4 fa[FM][2];
  auto read_a = [&](int slot, int sub, int j) __attribute__((always_inline)) {
    const uint8_t* sa = smem + slot * STAGE;
#pragma unroll
    for (int h = 0; h < 2; ++h)
      fa[j][h] = *reinterpret_cast<const u32x4*>(sa + swz_row<RB>(j * 32 + fr, 4 * sub + c0 + h));
  };
  v16f acc[FN][FM];
  auto mfma_one = [&](int set, int i, int j, bool first) __attribute__((always_inline)) {
    const v8i wv = (v8i)__builtin_shufflevector(wr[set][i][0], wr[set][i][1], 0, 1, 2, 3, 4, 5, 6, 7);
    const v8i av = (v8i)__builtin_shufflevector(fa[j][0], fa[j][1], 0, 1, 2, 3, 4, 5, 6, 7);
    const v16f zero = {};
    acc[i][j] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(wv, av, first ? zero : acc[i][j], 0, 0, 0, 0, 0, 0);
  };

  // ---- scales and epilogue (shared with gemm_fp8.hip)
  uint8_t* const scl = smem + NSL * STAGE;
  uint8_t* const stg = smem + NSL * STAGE + 2 * SCB + wave * STG;
  const bool sa_vec = g.sa_stride != 0, sb_vec = g.sb_stride != 0;
  const float sa0 = sa_vec ? 0.0f : __uint_as_float(__builtin_amdgcn_readfirstlane(__float_as_uint(g.sa[0])));
  const float sb0 = sb_vec ? 0.0f : __uint_as_float(__builtin_amdgcn_readfirstlane(__float_as_uint(g.sb[0])));
  auto load_scales = [&](int64_t local) __attribute__((always_inline)) {
    if (local >= my_tiles) return;
    int64_t tm, tn;
    tile_coords_pre(blockIdx.x + local * G, nt, tilesM, multi_round, tm, tn);
    uint8_t* dst = scl + (local & 1) * SCB;
    const uint32_t l16 = 16 * lane_id_here();
    // 1 KB chunks: sb's on waves 0, 2, ..., sa's on waves 1, 3, ...
#pragma unroll
    for (int c = 0; c < SBB; ++c)
      if (wave == (2 * c) % 4 && sb_vec)
        lds_dma_b128(g.sb, static_cast<uint32_t>(g.N * 4), lds_addr(dst + 1024 * c),
                     static_cast<uint32_t>(tn * BN * 4 + 1024 * c) + l16);
#pragma unroll
    for (int c = 0; c < SAB; ++c)
      if (wave == (2 * c + 1) % 4 && sa_vec)
        lds_dma_b128(g.sa, static_cast<uint32_t>(g.M * 4), lds_addr(dst + 1024 * (SBB + c)),
                     static_cast<uint32_t>(tm * BM * 4 + 1024 * c) + l16);
  };
  auto epilogue = [&](int64_t local) __attribute__((always_inline)) {
    int64_t tm, tn;
    tile_coords_pre(blockIdx.x + local * G, nt, tilesM, multi_round, tm, tn);
    gemm_epilogue<BN, BM, WN, WM, OUT, EPI, SRB>(g, acc, tm, tn, wn, wm, scl + (local & 1) * SCB, stg, sa_vec,
                                                 sb_vec, sa0, sb0);
  };

  // ---- step schedule.  Step s (K step kt of its tile, ring slot s / 2,
  // weight set s % WS).  Unit u = j * FN + i: MFMA (i, j), then, if it was
  // block j's last, block j's next-step activation reads; the step's share
  // of the weight loads of step s + WS - 1 and, on a slot's second step, of the
  // slot's refill.  The second step of a slot opens with a barrier (every
  // wave is done reading the slot, which may then be refilled with the slot
  // NSL ahead) and at unit MW waits for the next slot (own loads, then a
  // barrier for everyone's) before its activation reads start.
  constexpr int NMF = FN * FM;
  constexpr int MW = 3 * NMF / 8;
  // weight and refill loads spread evenly over their step's units (a
  // slot's refill all in its second step: splitting it over that step and
  // the next measured the same)
  auto w_at = [](int l) constexpr { return l * NMF / WL; };
  auto a_at = [](int i) constexpr { return i * NMF / IA; };
  // vmcnt of the slot waits: the fewest vm ops issued after the last load of
  // the slot waited for, over the prologue and the first steps (the stream
  // is periodic from there; epilogue stores between tiles only add ops and
  // make the wait more conservative), found by replaying the issue order
  constexpr int kWaitN = [w_at, a_at] {
    constexpr int S = 2 * NSL + 24;
    int last_of[S / 2 + NSL + 2] = {};
    int idx = 0;
    for (int q = 0; q < NSL; ++q) {
      idx += IA;
      last_of[q] = idx - 1;
    }
    idx += (WS - 1) * WL;
    int best = 1 << 30;
    for (int st = 0; st < S; ++st) {
      const bool lst = st & 1;
      for (int u = 0; u < NMF; ++u) {
        if (lst && u == MW) {
          const int c = idx - 1 - last_of[(st + 1) / 2];
          best = c < best ? c : best;
        }
        for (int l = 0; l < WL; ++l)
          if (w_at(l) == u) ++idx;
        if (lst)
          for (int i = 0; i < IA; ++i)
            if (a_at(i) == u) {
              ++idx;
              if (i == IA - 1) last_of[st / 2 + NSL] = idx - 1;
            }
      }
    }
    return best;
  }();
  static_assert(kWaitN >= 0 && kWaitN < 64, "vmcnt range");

  auto step = [&](int set, int64_t s, int kt, bool first) __attribute__((always_inline)) {
    __builtin_amdgcn_sched_barrier(0);
    const bool last = (set & 1) != 0;  // second step of its slot
    const int slot = static_cast<int>((s >> 1) % NSL);
    const int nslot = static_cast<int>(((s + 1) >> 1) % NSL);
    const int nsub = static_cast<int>((s + 1) & 1);
    // refill (second step of a slot): slot kt/2 + NSL of this tile, or of
    // the next
    const int lq0 = kt / 2 + NSL;
    const int lq = lq0 < KS ? lq0 : lq0 - KS;
    const bool lnx = lq0 >= KS;
    // weights of step s + WS - 1
    const int wk0 = kt + WS - 1;
    const int wk = wk0 < KT ? wk0 : wk0 - KT;
    const bool wnx = wk0 >= KT;
    const int wset = (set + WS - 1) % WS;
    if (last) lds_barrier();
#pragma unroll
    for (int u = 0; u < NMF; ++u) {
      const int j = u / FN, i = u % FN;
      if (last && u == MW) {
        waitcnt_vm<kWaitN>();
        lds_barrier();
        // blocks whose last MFMA is already issued
#pragma unroll
        for (int jj = 0; jj < FM; ++jj)
          if (jj * FN + FN - 1 < MW) read_a(nslot, nsub, jj);
      }
      mfma_one(set, i, j, first);
      if (i == FN - 1 && !(last && u < MW)) read_a(nslot, nsub, j);
#pragma unroll
      for (int l = 0; l < WL; ++l)
        if (w_at(l) == u) issue_w(wset, wk, wnx, l);
      if (last) {
#pragma unroll
        for (int a = 0; a < IA; ++a)
          if (a_at(a) == u) issue_a(slot, lq, lnx, a);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
  };

  // ---- prologue: activation slots 0..NSL-1 (past a one-tile workgroup's
  // end: the next tile's, i.e. zeros), then weights of steps 0..2; slot 0
  // landed, and its first step's fragments read.
  tile_bases(0, ba_cur, wv_cur);
  tile_bases(1, ba_nxt, wv_nxt);
  load_scales(0);
#pragma unroll
  for (int st = 0; st < NSL; ++st)
#pragma unroll
    for (int a = 0; a < IA; ++a) issue_a(st, st < KS ? st : st - KS, st >= KS, a);
#pragma unroll
  for (int st = 0; st < WS - 1; ++st)
#pragma unroll
    for (int l = 0; l < WL; ++l) issue_w(st, st < KT ? st : st - KT, st >= KT, l);
  waitcnt_vm<((NSL - 1) * IA + (WS - 1) * WL < 63 ? (NSL - 1) * IA + (WS - 1) * WL : 63)>();
  lds_barrier();
#pragma unroll
  for (int j = 0; j < FM; ++j) read_a(0, 0, j);

  // steps run in groups of WS (KT is a multiple of WS), so step s uses weight
  // set s % WS and loads set (s + WS - 1) % WS, both known at compile time
  int64_t s = 0;
  for (int64_t tile = 0; tile < my_tiles; ++tile) {
#pragma unroll
    for (int u = 0; u < WS; ++u) step(u, s + u, u, u == 0);
    s += WS;
    for (int kt = WS; kt < KT; kt += WS, s += WS) {
#pragma unroll
      for (int u = 0; u < WS; ++u) step(u, s + u, kt + u, false);
    }
    // the tile's scales (a direct-to-LDS load issued before its first step,
    // with KT * WL weight loads behind it) have landed
    if (KT * WL >= 64) waitcnt_vm<63>();
    else waitcnt_vm<0>();
    lds_barrier();
    epilogue(tile);
    load_scales(tile + 1);
    ba_cur = ba_nxt;
    wv_cur = wv_nxt;
    tile_bases(tile + 2, ba_nxt, wv_nxt);
  }
  waitcnt_vm<0>();  // drain the trailing loads before the LDS is released
#endif  // __HIP_DEVICE_COMPILE__
}

template <int BN, int BM, int OUT, int EPI>
static hipError_t launch_pre(const GemmArgs& g, hipStream_t st) {
  constexpr int RB = 128;
  constexpr int stage = BM * RB;
  constexpr int scb = 1024 * ((BN * 4 + 1023) / 1024 + (BM * 4 + 1023) / 1024);
  constexpr int fit = (160 * 1024 - 2 * scb - 4 * 32 * 128) / stage;
  constexpr int NSL = fit > 4 ? 4 : fit;
  const int64_t nt = ((g.N + BN - 1) / BN) * ((g.M + BM - 1) / BM);
  const int64_t cus = num_cus();
  // the ring runs NSL slots ahead, which may only reach into the next tile:
  // with fewer slots per tile than that, every tile gets its own workgroup
  const int64_t slots = pre_k_steps(g.K) / 2;
  const unsigned grid = static_cast<unsigned>(nt < cus || slots < NSL ? nt : cus);
  // steps past K (K not a multiple of the 256-byte step group) must read
  // zero activations: the weights there are zero, but a stray e4m3 NaN
  // would still poison the sum
  // four weight register sets (loads 3 steps ahead); eight on the smaller
  // tiles, whose steps are half as long, measured 2-5 % slower on the down
  // and o shapes
  if (g.K % (64 * kPreSteps) == 0)
    hipLaunchKernelGGL((gemm_fp8_pre<BN, BM, NSL, OUT, false, EPI, 4>), dim3(grid), dim3(256), 0, st, g);
  else
    hipLaunchKernelGGL((gemm_fp8_pre<BN, BM, NSL, OUT, true, EPI, 4>), dim3(grid), dim3(256), 0, st, g);
  return hipGetLastError();
}

// Tile choice: the least estimated time, rounds of tiles over the CUs
// (persistent workgroups: a partial round costs a full one) times a tile's
// MFMA work over its relative efficiency, measured with each tile forced
// (operands rotated through HBM): 256x256 1.0; 256x128 0.75 (the down and o
// projections: 2218-2243 and 1553-1738 TFLOP/s against 1506-1605 and
// 1225-1267 on 256x256 tiles, which leave half the CUs idle there); 128x128
// 0.6 (slower than 256x128 on every shape measured; taken by small launches).
template <int OUT, int EPI>
static hipError_t dispatch_pre(const GemmArgs& g, hipStream_t st) {
  const int64_t cus = num_cus();
  auto cost = [&](int bn, int bm, double eff) {
    const int64_t tiles = ((g.N + bn - 1) / bn) * ((g.M + bm - 1) / bm);
    return static_cast<double>((tiles + cus - 1) / cus) * bn * bm / eff;
  };
  const double c0 = cost(256, 256, 1.0), c1 = cost(256, 128, 0.75), c3 = cost(128, 128, 0.6);
  if (c0 <= c1 && c0 <= c3) return launch_pre<256, 256, OUT, EPI>(g, st);
  if (c1 <= c3) return launch_pre<256, 128, OUT, EPI>(g, st);
  return launch_pre<128, 128, OUT, EPI>(g, st);
}

}  // namespace fr

using namespace fr;

extern "C" int64_t fr_fp8_weight_prearranged_bytes(int64_t N, int64_t K) {
  if (N <= 0 || K <= 0) return N == 0 || K == 0 ? 0 : -1;
  return ((N + 31) / 32) * pre_k_steps(K) * kPreBlockBytes;
}

extern "C" int fr_fp8_weight_prearrange(const void* w, int64_t ldw, int64_t N, int64_t K, void* out,
                                        void* stream) {
  if (N < 0 || K < 0 || (N > 0 && ldw < K)) return FR_EINVAL;
  if (N == 0 || K == 0) return FR_OK;
  if (!w || !out) return FR_EINVAL;
  const int64_t bytes = fr_fp8_weight_prearranged_bytes(N, K);
  if (bytes >= (int64_t(1) << 31)) return FR_EUNSUPPORTED;
  const int64_t chunks = bytes / 16;
  hipLaunchKernelGGL(fp8_weight_prearrange, dim3(static_cast<unsigned>((chunks + 255) / 256)), dim3(256), 0,
                     static_cast<hipStream_t>(stream), static_cast<const uint8_t*>(w), ldw, N, K, pre_k_steps(K),
                     static_cast<uint8_t*>(out), chunks);
  return hipGetLastError() == hipSuccess ? FR_OK : FR_ELAUNCH;
}

extern "C" int fr_fp8_scaled_mm_prearranged(const void* a, int64_t lda, const void* w_pre, const float* scale_a,
                                            int64_t scale_a_numel, const float* scale_b, int64_t scale_b_numel,
                                            const void* residual, int64_t ldr, void* out, int64_t ldo, int64_t M,
                                            int64_t N, int64_t K, int out_dtype, int silu, void* stream) {
  if (M < 0 || N < 0 || K < 0) return FR_EINVAL;
  if (M == 0 || N == 0) return FR_OK;
  if (!a || !w_pre || !scale_a || !scale_b || !out) return FR_EINVAL;
  if (silu && (N % 16 != 0 || out_dtype != FR_DTYPE_BF16 || residual)) return FR_EINVAL;
  if (lda < K || ldo < (silu ? N / 2 : N)) return FR_EINVAL;
  if (!(scale_a_numel == 1 || scale_a_numel == M) || !(scale_b_numel == 1 || scale_b_numel == N)) return FR_EINVAL;
  if (residual && (out_dtype == FR_DTYPE_FP32 || ldr < N || (residual == out && ldr != ldo))) return FR_EINVAL;
  auto al16 = [](const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; };
  // the activation ring's operand conditions (there is no scalar variant
  // here: prearranged weights exist only for the MFMA kernel)
  if (K == 0 || K % 16 != 0 || lda % 16 != 0 || !al16(a) || !al16(w_pre) ||
      (M - 1) * lda + K >= (int64_t(1) << 31) || fr_fp8_weight_prearranged_bytes(N, K) >= (int64_t(1) << 31))
    return FR_EUNSUPPORTED;
  GemmArgs g{};
  g.a = static_cast<const uint8_t*>(a);
  g.lda = lda;
  g.b = static_cast<const uint8_t*>(w_pre);
  g.ldb = pre_k_steps(K) * kPreBlockBytes;
  g.sa = scale_a;
  g.sa_stride = scale_a_numel == 1 && M != 1 ? 0 : 1;
  g.sb = scale_b;
  g.sb_stride = scale_b_numel == 1 && N != 1 ? 0 : 1;
  g.out = out;
  g.ldo = ldo;
  g.M = M;
  g.N = N;
  g.K = K;
  g.res = residual;
  g.ldr = ldr;
  g.silu = silu ? 1 : 0;
  hipStream_t st = static_cast<hipStream_t>(stream);
  hipError_t err;
  switch (out_dtype) {
    case FR_DTYPE_BF16:
      err = silu ? dispatch_pre<FR_DTYPE_BF16, kEpiSilu>(g, st)
                 : (residual ? dispatch_pre<FR_DTYPE_BF16, kEpiRes>(g, st) : dispatch_pre<FR_DTYPE_BF16, kEpiPlain>(g, st));
      break;
    case FR_DTYPE_FP16:
      err = residual ? dispatch_pre<FR_DTYPE_FP16, kEpiRes>(g, st) : dispatch_pre<FR_DTYPE_FP16, kEpiPlain>(g, st);
      break;
    case FR_DTYPE_FP32: err = dispatch_pre<FR_DTYPE_FP32, kEpiPlain>(g, st); break;
    default: return FR_EINVAL;
  }
  return err == hipSuccess ? FR_OK : FR_ELAUNCH;
}
