// W8A8 fp8 GEMM on CDNA4 OCP-FP8 MFMA:
//   out[m, n] = (sum_k a[m, k] * b[k, n]) * sa[m] * sb[n] (+ bias[n])
// a: [M, K] e4m3 row-major (activations, per-row scale sa)
// b: [K, N] e4m3 column-major, i.e. N rows of K contiguous bytes
//    (weights, per-output-channel scale sb)
// Replaces python/flashrec/kernel/sglops.py:99-140 (fp8_scaled_mm), called
// from python/flashrec/layers/linear.py:153-172.
//
// Design (gfx950):
//  * Persistent: one 256-thread workgroup per CU walks its share of the
//    output tiles.  The K steps of consecutive tiles form one continuous
//    stream, so the direct-to-LDS loads for the next tile's first K steps
//    are in flight while the current tile finishes and stores its output.
//  * 4 wave64 in a 2x2 grid; each wave owns a (BN/2) x (BM/2) sub-tile of
//    32x32 blocks of v_mfma_f32_32x32x64_f8f6f4 (A-operand = weight rows,
//    B-operand = activation rows).  The K order inside one MFMA does not
//    matter as long as both operands use the same (lane group, byte) -> k
//    assignment: lane l supplies row l%32 and bytes (l/32)*32 .. +31 of the
//    64-byte K step, for both operands.
//  * K is consumed in 64-byte MFMA steps from an LDS ring whose rows hold
//    128 bytes of K (two steps per slot), filled by buffer_load ... lds (no
//    VGPR staging; rows past M/N and the K tail read as zero through the
//    buffer range check).  Each 1 KB load then covers 8 whole 128-byte
//    lines, which the direct-to-LDS path moves much faster than 16 half
//    lines.  One barrier per slot.
//  * Fragments of step s+1 are read from LDS while the MFMAs of step s run
//    (register double buffering).
//  * Epilogue: scales applied in fp32, converted, transposed through a
//    per-wave LDS staging tile and written as whole 128- (or 64-) byte row
//    segments through a buffer resource with scalar offsets, the passes
//    software-pipelined.
//  * Workgroup -> tile mapping is XCD aware: dispatch places workgroup i on
//    XCD i % 8; tiles are renumbered so each XCD walks a contiguous, m-grouped
//    range and its 32 CUs share weight/activation panels in their L2.
#include "gemm_common.h"

namespace fr {

// BN: weight rows (output columns) per tile, BM: activation rows per tile,
// RB: bytes of K per LDS row (64: one MFMA K step per ring slot, 128: two,
// so each direct-to-LDS load covers whole 128-byte lines), NSL: ring depth
// in slots, KTAIL: K % 128 != 0 (the last K steps are partly or wholly
// zero-filled).  EPI: kEpiPlain, kEpiRes or kEpiSilu.
template <int BN, int BM, int NSL, int RB, int OUT, bool KTAIL, int EPI>
__global__ __launch_bounds__(256, 1) void gemm_fp8_mfma(GemmArgs g) {
  // The host pass only needs the kernel's signature (for its launch stub);
  // the body uses device-only buffer-resource builtins.
#if defined(__HIP_DEVICE_COMPILE__)
  constexpr int FN = BN / 64;  // 32-row blocks per wave along n
  constexpr int FM = BM / 64;  // 32-row blocks per wave along m
  constexpr int WN = BN / 2;   // wave sub-tile: WN output columns ...
  constexpr int WM = BM / 2;   // ... x WM output rows
  constexpr int SPS = RB / kBK;       // MFMA K steps per ring slot
  constexpr int RPI = 1024 / RB;      // rows one 1 KB direct-to-LDS load covers
  constexpr int CPR = RB / 16;        // 16-byte chunks per LDS row
  constexpr int IB = BN * RB / 4096;  // 1 KB loads per wave per slot (weights)
  constexpr int IA = BM * RB / 4096;  // ... (activations)
  constexpr int STAGE = (BN + BM) * RB;
  constexpr int LOADS = IB + IA;  // vmcnt units one slot adds per wave
  constexpr int EB = OutT<OUT>::kBytes;
  constexpr bool RES = EPI == kEpiRes;
  // SiLU-and-mul (bf16 only): the weight rows come in chunks of 16, the
  // gate rows of 8 output columns followed by their 8 up rows; the product
  // column c of chunk k is bf16(bf16(silu(gate)) * up) of chunk columns c
  // and 8 + c, written at output column 8k + c (the output is N / 2 wide).
  constexpr bool SILU = EPI == kEpiSilu;
  static_assert(!SILU || OUT == FR_DTYPE_BF16, "SiLU epilogue writes bf16");
  // LDS: the slot ring, two 2 KB scale buffers, per-wave epilogue staging of
  // 32 rows x 128 bytes, or x 64 bytes where the wider staging does not fit
  // (narrow also when a wave's columns are not whole 128-byte staging rows:
  // the 192-column tile with 16-bit outputs)
  constexpr bool kNarrow =
      NSL * STAGE + 2 * 2048 + 4 * 32 * 128 > 160 * 1024 || (BN / 2) % (128 / OutT<OUT>::kBytes) != 0;
  constexpr int SRB = kNarrow ? 64 : 128;  // staging row bytes
  constexpr int STG = 32 * SRB;
  __shared__ __attribute__((aligned(1024))) uint8_t smem[NSL * STAGE + 2 * 2048 + 4 * STG];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  // wave index in an SGPR: LDS destinations (M0) and row bases are scalar
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wn = wave & 1, wm = wave >> 1;

  const int64_t tilesN = (g.N + BN - 1) / BN;
  const int64_t tilesM = (g.M + BM - 1) / BM;
  const int64_t nt = tilesN * tilesM;
  const int64_t G = gridDim.x;
  const int64_t my_tiles = (nt - blockIdx.x + G - 1) / G;
  // K steps per tile, rounded up to even (steps run in pairs); steps past
  // K read zeros through the buffer range check.
  const int KT = static_cast<int>((g.K + 2 * kBK - 1) / (2 * kBK)) * 2;
  const int KS = KT / SPS;  // ring slots per tile
  const int64_t S = my_tiles * KT;  // K steps this workgroup runs
  if (S == 0) return;

  const __amdgpu_buffer_rsrc_t rb =
      make_rsrc(g.b, static_cast<uint32_t>((g.N - 1) * g.ldb + g.K));
  const __amdgpu_buffer_rsrc_t ra =
      make_rsrc(g.a, static_cast<uint32_t>((g.M - 1) * g.lda + g.K));

  // ---- direct-to-LDS loads.  One wave instruction fills 1 KB = RPI rows of
  // RB bytes; lane L lands in row L/CPR, chunk slot L%CPR, so it fetches the
  // global chunk (L%CPR) ^ g(L/CPR).  Per-lane row offsets are kept for the
  // tile being computed (cur) and the next one (nxt): the ring runs NSL slots
  // ahead, so the last NSL slots of a tile load the first ones of the next.
  // Offsets of a tile past the end are out of range (loads return zeros,
  // touch nothing).
  // The swizzle depends on row bits 0-3.  A load covers 16 (RB = 64) or 8
  // (RB = 128) rows starting at a multiple of 16 or 8: in the second case
  // bit 3 of the row is the parity of the load's index l*4 + wave, i.e. of
  // the wave.
  const int lrow = lane / CPR;
  const int lchunk = (lane % CPR) ^ (RB == 64 ? swz_g(lrow) : swz_g8(lrow + 8 * (wave & 1)));
  constexpr uint32_t kOOB = 0x80000000u;
  // Per-lane part of each load's offset (the same for every tile) and the
  // scalar tile bases of the current and the next tile; a tile past the end
  // gets base kOOB (the sum is then past the buffer: zeros, no access).
  uint32_t lob[IB], loa[IA];
#pragma unroll
  for (int i = 0; i < IB; ++i) lob[i] = static_cast<uint32_t>(((i * 4 + wave) * RPI + lrow) * g.ldb + lchunk * 16);
#pragma unroll
  for (int i = 0; i < IA; ++i) loa[i] = static_cast<uint32_t>(((i * 4 + wave) * RPI + lrow) * g.lda + lchunk * 16);
  uint32_t bb_cur, ba_cur, bb_nxt, ba_nxt;
  auto tile_bases = [&](int64_t local, uint32_t& bb, uint32_t& ba) __attribute__((always_inline)) {
    if (local >= my_tiles) {
      bb = ba = kOOB;
      return;
    }
    int64_t tm, tn;
    tile_coords(blockIdx.x + local * G, nt, tilesM, tm, tn);
    bb = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(tn * BN * g.ldb));
    ba = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(tm * BM * g.lda));
  };
  // Load `l` (0..LOADS-1: weight blocks, then activation blocks) of ring
  // slot `lk` (0..KS-1, RB bytes of K) of the cur or nxt tile into `slot`.
  auto issue_one = [&](int slot, int lk, bool next, int l) __attribute__((always_inline)) {
    uint8_t* sb = smem + slot * STAGE;
    uint8_t* sa = sb + BN * RB;
    const uint32_t k0 = static_cast<uint32_t>(lk) * RB;
    const bool kin = !KTAIL || (k0 + lchunk * 16 < static_cast<uint64_t>(g.K));
    if (l < IB) {
      const uint32_t o = lob[l] + (next ? bb_nxt : bb_cur);
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rb, (lds_ptr_t)(sb + (l * 4 + wave) * 1024), 16,
                                               kin ? o : kOOB, k0, 0, 0);
    } else {
      const int i = l - IB;
      const uint32_t o = loa[i] + (next ? ba_nxt : ba_cur);
      __builtin_amdgcn_raw_ptr_buffer_load_lds(ra, (lds_ptr_t)(sa + (i * 4 + wave) * 1024), 16,
                                               kin ? o : kOOB, k0, 0, 0);
    }
  };
  auto issue = [&](int slot, int lk, bool next) __attribute__((always_inline)) {
#pragma unroll
    for (int l = 0; l < LOADS; ++l) issue_one(slot, lk, next, l);
  };

  // ---- fragments and MFMAs
  const int fr = lane & 31;        // fragment row inside a 32-row block
  const int c0 = (lane >> 5) * 2;  // first 16-byte chunk of this lane's 32 bytes
  // Fragments as 16-byte halves.  Activation fragments are used by every
  // MFMA row and have two register sets (current step, next step).  Weight
  // fragments have two sets too, except on the 256x256 tile, where registers
  // are short: there block i of the next step is read right after the last
  // MFMA that uses block i of the current one.  Read r (0..2*(FN+FM)-1) fills
  // half r%2 of weight block r/2, then of activation block r/2 - FN.
  constexpr bool kOneB = BN == 256 && BM == 256;
  struct Frags {
    u32x4 b[FN][2], a[FM][2];
  };
  u32x4 fb1[kOneB ? FN : 1][2];  // the single weight set (kOneB)
  auto breg = [&](Frags& f, int i, int h) -> u32x4& __attribute__((always_inline)) {
    if constexpr (kOneB) return fb1[i][h];
    else return f.b[i][h];
  };
  // Fragments of MFMA K step `sub` (0..SPS-1) of a ring slot.
  auto read_one = [&](Frags& f, int slot, int sub, int r) __attribute__((always_inline)) {
    const uint8_t* sb = smem + slot * STAGE;
    const uint8_t* sa = sb + BN * RB;
    const int h = r & 1;
    const int c = 4 * sub + c0 + h;
    if (r < 2 * FN) {
      const int i = r >> 1;
      breg(f, i, h) = *reinterpret_cast<const u32x4*>(sb + swz_row<RB>(wn * WN + i * 32 + fr, c));
    } else {
      const int j = (r >> 1) - FN;
      f.a[j][h] = *reinterpret_cast<const u32x4*>(sa + swz_row<RB>(wm * WM + j * 32 + fr, c));
    }
  };
  auto read_frags = [&](Frags& f, int slot, int sub) __attribute__((always_inline)) {
#pragma unroll
    for (int r = 0; r < 2 * (FN + FM); ++r) read_one(f, slot, sub, r);
  };
  v16f acc[FN][FM];
  // A tile's first K step starts its accumulators from the constant 0
  // (the MFMA's inline-constant C operand) instead of clearing 256 AGPRs.
  auto mfma_one = [&](Frags& f, int i, int j, bool first) __attribute__((always_inline)) {
    const v8i bv = (v8i)__builtin_shufflevector(breg(f, i, 0), breg(f, i, 1), 0, 1, 2, 3, 4, 5, 6, 7);
    const v8i av = (v8i)__builtin_shufflevector(f.a[j][0], f.a[j][1], 0, 1, 2, 3, 4, 5, 6, 7);
    const v16f zero = {};
    acc[i][j] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(bv, av, first ? zero : acc[i][j], 0, 0, 0, 0, 0, 0);
  };

  // ---- epilogue of one tile.  Lane l holds, per block (i, j), output row
  // m = l%32 of block j and the 4 consecutive columns n = 8q + 4(l/32) + t of
  // block i (q, t = 0..3).  Fast path: (acc * sa[m]) * sb[n] is converted and
  // written to a per-wave staging tile of 32 rows x 128 bytes per pass (16-byte
  // chunk c of row r at slot c ^ (r % 8)), read back as 16 consecutive bytes
  // per lane and stored as whole 128-byte row segments.  The tile's scales
  // are brought into LDS by direct loads when the tile starts (load_scales),
  // so the epilogue issues no global load (a load here would queue behind
  // the next tile's ring loads: vmcnt retires in order) and holds no scale
  // registers through the K loop.
  uint8_t* const scl = smem + NSL * STAGE;
  uint8_t* const stg = smem + NSL * STAGE + 2 * 2048 + wave * STG;
  // scales: sb[BN] (1 KB) then sa[BM] (1 KB) as fp32, one buffer per tile parity
  const bool sa_vec = g.sa_stride != 0, sb_vec = g.sb_stride != 0;
  // per-tensor scales, read once up front (never a load in the epilogue)
  const float sa0 = sa_vec ? 0.0f : __uint_as_float(__builtin_amdgcn_readfirstlane(__float_as_uint(g.sa[0])));
  const float sb0 = sb_vec ? 0.0f : __uint_as_float(__builtin_amdgcn_readfirstlane(__float_as_uint(g.sb[0])));
  auto load_scales = [&](int64_t local) __attribute__((always_inline)) {
    if (local >= my_tiles) return;
    int64_t tm, tn;
    tile_coords(blockIdx.x + local * G, nt, tilesM, tm, tn);
    uint8_t* dst = scl + (local & 1) * 2048;
    const uint32_t l16 = 16 * lane_id_here();
    if (wave == 0 && sb_vec)
      lds_dma_b128(g.sb, static_cast<uint32_t>(g.N * 4), lds_addr(dst), static_cast<uint32_t>(tn * BN * 4) + l16);
    if (wave == 1 && sa_vec)
      lds_dma_b128(g.sa, static_cast<uint32_t>(g.M * 4), lds_addr(dst + 1024),
                   static_cast<uint32_t>(tm * BM * 4) + l16);
  };
  // bf16/fp16 outputs leave the epilogue through an LDS staging tile as
  // 16-byte row segments.  8-byte stores straight from the accumulator
  // layout need no LDS round trips but twice the store instructions;
  // measured in one process against the staged form, they were 1-12 %
  // slower on every tile shape.
  // stores per wave per tile on the fast paths (fp32: 16 bytes per (i, j, q))
  constexpr int kStagedStores = gemm_staged_stores<OUT, EPI, FN, FM>();
  // Returns whether a fast path ran (and so issued exactly kStagedStores
  // stores per wave).
  auto epilogue = [&](int64_t local) -> bool __attribute__((always_inline)) {
    int64_t tm, tn;
    tile_coords(blockIdx.x + local * G, nt, tilesM, tm, tn);
    return gemm_epilogue<BN, BM, WN, WM, OUT, EPI, SRB>(g, acc, tm, tn, wn, wm, scl + (local & 1) * 2048, stg,
                                                         sa_vec, sb_vec, sa0, sb0);
  };

  // ---- prologue: the first NSL slots in flight; all but the last landed.
  // With more than one tile per workgroup KS >= NSL (see launch_mfma), so
  // the prologue stays inside tile 0; with one tile, slots past its end are
  // all-zero dummies.
  tile_bases(0, bb_cur, ba_cur);
  tile_bases(1, bb_nxt, ba_nxt);
  load_scales(0);
#pragma unroll
  for (int st = 0; st < NSL; ++st) issue(st, st < KS ? st : st - KS, st >= KS);
  waitcnt_vm<LOADS>();
  lds_barrier();
  Frags f0, f1;
  read_frags(f0, 0, 0);

  // ---- main loop.  Step s (tile s / KT, K step kt = s % KT; ring slot
  // q = s / SPS, step s % SPS inside it) holds its fragments in `cur` and
  // reads step s+1's into `nxt`.  The last step of a slot opens with a
  // barrier that retires every wave's reads of slot q (whose steps are all in
  // registers by then), refills slot q with slot q+NSL, spreading those loads
  // over its MFMAs, and a few MFMAs in waits for the next slot (own loads,
  // then everyone's through a second barrier) before reading from it.  Each
  // MFMA is followed by its share of the next step's fragment reads (over
  // three quarters of the MFMAs that follow the wait) and of the refill
  // loads, so the LDS reads of the CU's four waves overlap the matrix work
  // instead of stalling the next step.  Past the end the ring loads zeros
  // and the last fragment read is discarded.
  //
  // vmcnt retires loads and stores in issue order, so a plain load wait issued
  // while the epilogue's stores are in flight would also wait for them.
  // Before a tile's epilogue every ring load but the newest slot's is drained
  // (waitcnt_vm<LOADS>): slots 0..NSL-2 of the next tile have landed and
  // need no wait; slot NSL-1 is waited for with a count that also leaves the
  // epilogue's stores in flight (wait kind 2 below) when their number is
  // known.
  static_assert(NSL >= 2, "ring of at least two slots");
  constexpr int NMF = FN * FM;                   // MFMAs per step
  constexpr int NRD = 2 * (FN + FM);             // 16-byte LDS reads per step
  // Fragment reads over the first three quarters of the step's MFMAs, the
  // refill loads over all of them.  Measured with 128-byte rows on the
  // 4096-row gate_up, qkv and down shapes against reads over 1/2, 5/8, 7/8
  // or all MFMAs and loads from 1/8, 1/4 or 1/2 on, or ending at 1/2 or
  // 3/4: this placement was best or within 1 % on each (gate_up +4 % over
  // loads from 1/4 on).
  constexpr int RDU = NMF * 3 / 4;  // MFMAs the fragment reads spread over
  constexpr int LD0 = 0;            // first MFMA followed by a ring load
  constexpr int LDE = NMF;          // loads spread over MFMAs LD0 .. LDE-1
  // Wait kinds: 0 none, 1 the slot's loads (the NSL-2 newer slots' loads may
  // be in flight), 2 the same with the previous tile's staged stores also
  // allowed in flight (they were issued after the loads waited for).  The
  // count is capped at vmcnt's 63: a smaller count only waits for the
  // oldest few stores as well (conservative).
  // The slot-final step opens with a barrier (every wave is done reading the
  // slot, so its refill may start) and waits for the next slot only at MFMA
  // MW, its fragment reads following from there: the newest refill loads get
  // MW MFMAs more time to land.  Measured with MW at 1/4, 3/8, 1/2, 5/8 and 3/4
  // of the step on the 4096-row gate_up, qkv, down and o shapes, M = 512 and
  // fp32 outputs: 3/8 best or within 1 % on each, 2-7 % over waiting at the
  // start (0 restores that).
  constexpr int MW = 3 * NMF / 8;
  // refill loads of the same step issued before that point
  constexpr int kEarly = [] {
    int n = 0;
    for (int l = 0; l < LOADS; ++l)
      if (LD0 + l * (LDE - LD0) / LOADS < MW) ++n;
    return n;
  }();
  constexpr int kWait1 = (NSL - 2) * LOADS + kEarly;
  constexpr int kAdjN = kWait1 + kStagedStores < 63 ? kWait1 + kStagedStores : 63;
  auto step = [&](Frags& cur, Frags& nxt, int64_t s, int kt, int wait, bool first, bool last)
      __attribute__((always_inline)) {
    __builtin_amdgcn_sched_barrier(0);
    auto slot_wait = [&]() __attribute__((always_inline)) {
      if (wait == 2)
        waitcnt_vm<kAdjN>();
      else if (wait != 0)
        waitcnt_vm<kWait1>();
      lds_barrier();
    };
    if (last) {
      if (MW == 0) slot_wait();
      else lds_barrier();
    }
    const int lq0 = kt / SPS + NSL;
    const int lq = lq0 < KS ? lq0 : lq0 - KS;
    const bool nx = lq0 >= KS;
    const int slot = static_cast<int>((s / SPS) % NSL);
    const int nslot = static_cast<int>(((s + 1) / SPS) % NSL);
    const int nsub = static_cast<int>((s + 1) % SPS);
    // Unit u: its share of step s+1's fragment reads, MFMA u of step s
    // (weight block u / FM), with a single weight set the next weight block's
    // reads once its last MFMA is issued, its share of the refill loads.  The
    // sched_barrier keeps units in order, so the loads leave at the rate the
    // step consumes data and the wave never stalls on a full load queue while
    // it has MFMAs to issue.
#pragma unroll
    for (int u = 0; u < NMF; ++u) {
      // reads of a slot-final step start at MFMA R0 (after the wait)
      const int R0 = last ? MW : 0;
      const int RU = last && MW > 0 ? (NMF - MW) * 3 / 4 : RDU;
      if (last && MW > 0 && u == MW) {
        slot_wait();
        if constexpr (kOneB) {
          // weight blocks whose last MFMA is already issued
#pragma unroll
          for (int i = 0; i < FN; ++i)
            if (i * FM + FM - 1 < MW) {
              read_one(nxt, nslot, nsub, 2 * i);
              read_one(nxt, nslot, nsub, 2 * i + 1);
            }
        }
      }
      if constexpr (kOneB) {
#pragma unroll
        for (int r = 0; r < 2 * FM; ++r)
          if (R0 + r * RU / (2 * FM) == u) read_one(nxt, nslot, nsub, 2 * FN + r);
      } else {
#pragma unroll
        for (int r = 0; r < NRD; ++r)
          if (R0 + r * RU / NRD == u) read_one(nxt, nslot, nsub, r);
      }
      mfma_one(cur, u / FM, u % FM, first);
      if (kOneB && u % FM == FM - 1 && !(last && MW > 0 && u < MW)) {
        read_one(nxt, nslot, nsub, 2 * (u / FM));
        read_one(nxt, nslot, nsub, 2 * (u / FM) + 1);
      }
      if (last) {
#pragma unroll
        for (int l = 0; l < LOADS; ++l)
          if (LD0 + l * (LDE - LD0) / LOADS == u) issue_one(slot, lq, nx, l);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
  };
  // Wait kind of the slot-final step kt of a tile: the slot after it is
  // slot kt / SPS + 1 of the tile.
  auto wait_kind = [&](int kt, bool staged_prev) __attribute__((always_inline)) -> int {
    const int nq = kt / SPS + 1;
    if (nq <= NSL - 2) return 0;
    if (nq == NSL - 1) return staged_prev ? 2 : 1;
    return 1;
  };
  int64_t s = 0;
  bool staged_prev = false;
  for (int64_t tile = 0; tile < my_tiles; ++tile) {
    // steps run in pairs (f0, f1); with two steps per slot the second of a
    // pair ends the slot
    step(f0, f1, s, 0, SPS == 1 ? wait_kind(0, staged_prev) : 0, true, SPS == 1);
    step(f1, f0, s + 1, 1, wait_kind(1, staged_prev), false, true);
    s += 2;
    for (int kt = 2; kt < KT; kt += 2, s += 2) {
      step(f0, f1, s, kt, SPS == 1 ? wait_kind(kt, staged_prev) : 0, false, SPS == 1);
      step(f1, f0, s + 1, kt + 1, wait_kind(kt + 1, staged_prev), false, true);
    }
    waitcnt_vm<LOADS>();
    staged_prev = epilogue(tile);
    load_scales(tile + 1);
    bb_cur = bb_nxt;
    ba_cur = ba_nxt;
    tile_bases(tile + 2, bb_nxt, ba_nxt);
  }
  waitcnt_vm<0>();  // drain the trailing dummy loads before the LDS is released
#endif  // __HIP_DEVICE_COMPILE__
}

// Scalar fallback for shapes/strides the MFMA kernel does not take
// (K not a multiple of 16, unaligned operands).  One thread per output.
template <int OUT>
__global__ __launch_bounds__(256) void gemm_fp8_scalar(GemmArgs g) {
  const int64_t idx = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (idx >= g.M * g.N) return;
  const int64_t m = idx / g.N, n = idx % g.N;
  const uint8_t* ar = g.a + m * g.lda;
  const uint8_t* br = g.b + n * g.ldb;
  float acc = 0.0f;
  for (int64_t k = 0; k < g.K; ++k)
    acc += __builtin_amdgcn_cvt_f32_fp8(ar[k], 0) * __builtin_amdgcn_cvt_f32_fp8(br[k], 0);
  float v[4] = {(acc * g.sa[m * g.sa_stride]) * g.sb[n * g.sb_stride], 0.f, 0.f, 0.f};
  // store one element through the 4-wide helper with N clipped to n + 1
  store4<OUT>(g.out, g.ldo, m, n, n + 1, v, g.bias, g.res, g.ldr);
}


// Bytes of K per LDS row: 128 for every tile shape (each direct-to-LDS load
// then covers whole 128-byte lines; 64-byte rows measured slower on every
// shape).
template <int BN, int BM>
constexpr int tile_rb() {
  return 128;
}
// Ring slots: the deepest ring that fits next to the scale buffers and the
// epilogue staging (32 x 128 bytes per wave, or 32 x 64 where that buys a
// needed slot).  The loads are latency-bound (about 1.3 us from issue to LDS on a
// busy chip); at 64-byte rows this gives 4, 5 and 8 slots for the 256x256,
// 256x128 and 128x128 tiles.
template <int BN, int BM, int RB>
constexpr int ring_slots() {
  constexpr int stage = (BN + BM) * RB;
  constexpr int wide = (160 * 1024 - 2 * 2048 - 4 * 32 * 128) / stage;
  constexpr int narrow = (160 * 1024 - 2 * 2048 - 4 * 32 * 64) / stage;
  // (at 64-byte rows a sixth 256x128 slot bought with narrow staging measured
  // no faster, so narrow staging is taken only below three slots)
  constexpr int n = wide >= 3 || narrow == wide ? wide : narrow;
  constexpr int cap = 8 * kBK / RB;
  return n > cap ? cap : n;
}

template <int BN, int BM, int OUT, int EPI>
static hipError_t launch_mfma(const GemmArgs& g, hipStream_t st) {
  constexpr int RB = tile_rb<BN, BM>();
  constexpr int NSL = ring_slots<BN, BM, RB>();
  const int64_t nt = ((g.N + BN - 1) / BN) * ((g.M + BM - 1) / BM);
  const int64_t cus = num_cus();
  // The ring runs NSL slots ahead, which may only reach into the next tile:
  // with fewer K steps per tile than that, give every tile its own workgroup.
  const int64_t kt = ((g.K + 2 * kBK - 1) / (2 * kBK)) * 2;
  const unsigned grid = static_cast<unsigned>(nt < cus || kt < NSL * (RB / kBK) ? nt : cus);
  if (g.K % (2 * kBK) == 0)
    hipLaunchKernelGGL((gemm_fp8_mfma<BN, BM, NSL, RB, OUT, false, EPI>), dim3(grid), dim3(256), 0, st, g);
  else
    hipLaunchKernelGGL((gemm_fp8_mfma<BN, BM, NSL, RB, OUT, true, EPI>), dim3(grid), dim3(256), 0, st, g);
  return hipGetLastError();
}

template <int OUT>
static hipError_t dispatch(const GemmArgs& g, hipStream_t st) {
  auto al16 = [](const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; };
  // Buffer offsets are 32-bit: each operand must span < 2 GiB; the K == 0
  // case has nothing to load.
  const bool mfma_ok = g.K > 0 && g.K % 16 == 0 && g.lda % 16 == 0 && g.ldb % 16 == 0 &&
                       al16(g.a) && al16(g.b) && (g.M - 1) * g.lda + g.K < (int64_t(1) << 31) &&
                       (g.N - 1) * g.ldb + g.K < (int64_t(1) << 31);
  if (!mfma_ok) {
    const int64_t total = g.M * g.N;
    hipLaunchKernelGGL((gemm_fp8_scalar<OUT>), dim3(static_cast<unsigned>((total + 255) / 256)),
                       dim3(256), 0, st, g);
    return hipGetLastError();
  }
  // Tile choice: the shape with the least estimated time, rounds of tiles
  // over the CUs (persistent workgroups: a partial round costs a full one)
  // times a tile's MFMA work over its relative efficiency (256x256 1.0,
  // 256x128 0.75, 192x128 0.72, 128x128 0.6), fitted so that the choice is
  // the fastest of the four, timed with every tile forced, on the config
  // shapes and on M = 768..3072 x N = 12288, M = 1024 x N = 4096 and
  // M = 2048 x N = 2048 (K = 2048 or 6144).  E.g. M=4096, N=12288 takes
  // 256x256 (3 rounds); N=2048 takes 256x128 (one round); M=512, N=12288
  // takes 192x128 (256 tiles: one round on every CU, where 256x128 leaves 64
  // CUs idle); M=1024..3072, N=12288 take 256x256 (3-10 % over the smaller
  // tiles' extra rounds).
  const int64_t cus = num_cus();
  auto tiles = [&](int bn, int bm) __attribute__((always_inline)) { return ((g.N + bn - 1) / bn) * ((g.M + bm - 1) / bm); };
  auto cost = [&](int bn, int bm, double eff) __attribute__((always_inline)) {
    return static_cast<double>((tiles(bn, bm) + cus - 1) / cus) * bn * bm / eff;
  };
  const double c256 = cost(256, 256, 1.0), c2561 = cost(256, 128, 0.75), c192 = cost(192, 128, 0.72),
               c128 = cost(128, 128, 0.6);
  // the residual add and SiLU-and-mul are variants of their own, so the
  // plain kernels carry none of their code (measured 1-3 % on every tile
  // shape when the residual was a runtime branch); only 16-bit outputs take
  // a residual, only bf16 takes SiLU (never on the 192-column tile, whose
  // wave sub-tiles are not whole gate/up chunk pairs)
  if constexpr (OUT == FR_DTYPE_BF16) {
    if (g.silu) {
      if (c256 <= c2561 && c256 <= c128) return launch_mfma<256, 256, OUT, kEpiSilu>(g, st);
      if (c2561 <= c128) return launch_mfma<256, 128, OUT, kEpiSilu>(g, st);
      return launch_mfma<128, 128, OUT, kEpiSilu>(g, st);
    }
  }
  constexpr int kRes = OUT != FR_DTYPE_FP32 ? kEpiRes : kEpiPlain;
  const bool res = OUT != FR_DTYPE_FP32 && g.res;
  if (c256 <= c2561 && c256 <= c192 && c256 <= c128)
    return res ? launch_mfma<256, 256, OUT, kRes>(g, st) : launch_mfma<256, 256, OUT, kEpiPlain>(g, st);
  if (c2561 <= c192 && c2561 <= c128)
    return res ? launch_mfma<256, 128, OUT, kRes>(g, st) : launch_mfma<256, 128, OUT, kEpiPlain>(g, st);
  if (c192 <= c128)
    return res ? launch_mfma<192, 128, OUT, kRes>(g, st) : launch_mfma<192, 128, OUT, kEpiPlain>(g, st);
  return res ? launch_mfma<128, 128, OUT, kRes>(g, st) : launch_mfma<128, 128, OUT, kEpiPlain>(g, st);
}

}  // namespace fr

using namespace fr;

static int gemm_entry(const void* a, int64_t lda, const void* b, int64_t ldb, const float* scale_a,
                      int64_t scale_a_numel, const float* scale_b, int64_t scale_b_numel, const void* bias,
                      int64_t bias_numel, const void* res, int64_t ldr, void* out, int64_t ldo, int64_t M,
                      int64_t N, int64_t K, int out_dtype, void* stream, bool silu = false) {
  if (M < 0 || N < 0 || K < 0) return FR_EINVAL;
  if (M == 0 || N == 0) return FR_OK;
  if (!a || !b || !scale_a || !scale_b || !out) return FR_EINVAL;
  if (lda < K || ldb < K || ldo < (silu ? N / 2 : N)) return FR_EINVAL;
  if (!(scale_a_numel == 1 || scale_a_numel == M)) return FR_EINVAL;
  if (!(scale_b_numel == 1 || scale_b_numel == N)) return FR_EINVAL;
  if (bias && bias_numel != N) return FR_EINVAL;  // the epilogue reads bias[0..N)
  if (M * N > (int64_t)0x7FFFFFFF * 256) return FR_EUNSUPPORTED;
  GemmArgs g{};
  g.a = static_cast<const uint8_t*>(a);
  g.lda = lda;
  g.b = static_cast<const uint8_t*>(b);
  g.ldb = ldb;
  g.sa = scale_a;
  g.sa_stride = scale_a_numel == 1 && M != 1 ? 0 : 1;
  g.sb = scale_b;
  g.sb_stride = scale_b_numel == 1 && N != 1 ? 0 : 1;
  g.bias = bias;
  g.out = out;
  g.ldo = ldo;
  g.M = M;
  g.N = N;
  g.K = K;
  g.res = res;
  g.ldr = ldr;
  g.silu = silu ? 1 : 0;
  hipStream_t st = static_cast<hipStream_t>(stream);
  hipError_t err;
  switch (out_dtype) {
    case FR_DTYPE_BF16: err = dispatch<FR_DTYPE_BF16>(g, st); break;
    case FR_DTYPE_FP16: err = dispatch<FR_DTYPE_FP16>(g, st); break;
    case FR_DTYPE_FP32: err = dispatch<FR_DTYPE_FP32>(g, st); break;
    default: return FR_EINVAL;
  }
  return err == hipSuccess ? FR_OK : FR_ELAUNCH;
}

extern "C" int fr_fp8_scaled_mm(const void* a, int64_t lda, const void* b, int64_t ldb,
                                const float* scale_a, int64_t scale_a_numel,
                                const float* scale_b, int64_t scale_b_numel, const void* bias,
                                int64_t bias_numel, void* out, int64_t ldo, int64_t M, int64_t N, int64_t K,
                                int out_dtype, void* stream) {
  return gemm_entry(a, lda, b, ldb, scale_a, scale_a_numel, scale_b, scale_b_numel, bias, bias_numel, nullptr, 0,
                    out, ldo, M, N, K, out_dtype, stream);
}

extern "C" int fr_fp8_scaled_mm_residual(const void* a, int64_t lda, const void* b, int64_t ldb,
                                         const float* scale_a, int64_t scale_a_numel, const float* scale_b,
                                         int64_t scale_b_numel, const void* residual, int64_t ldr, void* out,
                                         int64_t ldo, int64_t M, int64_t N, int64_t K, int out_dtype,
                                         void* stream) {
  if (out_dtype != FR_DTYPE_BF16 && out_dtype != FR_DTYPE_FP16) return out_dtype == FR_DTYPE_FP32 ? FR_EUNSUPPORTED
                                                                                                    : FR_EINVAL;
  if (M > 0 && N > 0 && (!residual || ldr < N)) return FR_EINVAL;
  // in place only row for row: an aliased residual must share the output's stride
  if (residual == out && ldr != ldo) return FR_EINVAL;
  return gemm_entry(a, lda, b, ldb, scale_a, scale_a_numel, scale_b, scale_b_numel, nullptr, 0, residual, ldr, out,
                    ldo, M, N, K, out_dtype, stream);
}

// out[m, 8k + c] = bf16(bf16(silu(p[m, 16k + c])) * p[m, 16k + 8 + c]) for
// the bf16-rounded scaled product p (c < 8): SiLU-and-mul in the epilogue,
// with the weight rows given in gate/up chunks of 8 (see gemm_fp8_mfma).
extern "C" int fr_fp8_scaled_mm_silu(const void* a, int64_t lda, const void* b, int64_t ldb, const float* scale_a,
                                     int64_t scale_a_numel, const float* scale_b, int64_t scale_b_numel, void* out,
                                     int64_t ldo, int64_t M, int64_t N, int64_t K, void* stream) {
  if (M < 0 || N < 0 || K < 0 || N % 16 != 0) return FR_EINVAL;
  // the MFMA kernel's operand conditions (there is no scalar SiLU variant)
  auto al16 = [](const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; };
  if (M > 0 && N > 0 &&
      (K == 0 || K % 16 != 0 || lda % 16 != 0 || ldb % 16 != 0 || !al16(a) || !al16(b) ||
       (M - 1) * lda + K >= (int64_t(1) << 31) || (N - 1) * ldb + K >= (int64_t(1) << 31)))
    return FR_EUNSUPPORTED;
  return gemm_entry(a, lda, b, ldb, scale_a, scale_a_numel, scale_b, scale_b_numel, nullptr, 0, nullptr, 0, out, ldo,
                    M, N, K, FR_DTYPE_BF16, stream, true);
}
