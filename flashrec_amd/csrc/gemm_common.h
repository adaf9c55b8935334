// Shared pieces of the W8A8 fp8 GEMM kernels (gemm_fp8.hip: weights as
// [N, K] rows staged through LDS; gemm_fp8_pre.hip: weights pre-arranged in
// MFMA fragment order and loaded straight into registers): the argument
// block, LDS swizzles, barrier and wait helpers, the epilogue's LDS accesses
// as inline asm, buffer resources, the XCD-aware tile order.
#pragma once

#include <type_traits>

#include "fr_common.h"

namespace fr {

typedef int v8i __attribute__((ext_vector_type(8)));
typedef float v16f __attribute__((ext_vector_type(16)));
typedef __attribute__((address_space(3))) void* lds_ptr_t;

struct GemmArgs {
  const uint8_t* a;
  int64_t lda;
  const uint8_t* b;
  int64_t ldb;
  const float* sa;
  int64_t sa_stride;  // 1: per-row, 0: per-tensor
  const float* sb;
  int64_t sb_stride;  // 1: per-channel, 0: per-tensor
  const void* bias;   // out dtype, [N] or null
  void* out;
  int64_t ldo;
  int64_t M, N, K;
  // residual rows (out dtype, 16-bit outputs only) added to the rounded
  // product: out = rnd(rnd(product) + res); may alias out (same ldo), or null
  const void* res;
  int64_t ldr;
  // SiLU-and-mul epilogue: out is [M, N / 2] bf16 (see gemm_fp8_mfma)
  int silu;
};

constexpr int kBK = 64;  // bytes of K per MFMA step
// Epilogue variants (a compile-time kernel parameter, so the plain kernels
// carry none of the others' code): the scaled product; the same plus a
// residual added after rounding; SiLU-and-mul of gate/up column pairs.
constexpr int kEpiPlain = 0, kEpiRes = 1, kEpiSilu = 2;
constexpr int kNT = 2;   // buffer-instruction cache policy bit: nontemporal (gfx950)

// LDS rows are 64 bytes (4 chunks of 16 B); chunk c of row r lives in slot
// c ^ g(r) with g(r) = r2 | (r1 ^ r3) << 1 (r_i = bit i of r).  For the
// 16-byte fragment reads (lane l reads row l % 32) this spreads every group
// of 8 consecutive rows over the 8 distinct 16-byte bank groups of a
// 128-byte bank line, and every group of 16 rows over the 16 of a 256-byte
// line, so the reads are conflict free whether the LDS serves 128 or 256
// bytes per clock.
__device__ __forceinline__ int swz_g(int r) {
  return ((r >> 2) & 1) | ((((r >> 1) ^ (r >> 3)) & 1) << 1);
}
__device__ __forceinline__ int swz(int r, int c) { return r * 64 + ((c ^ swz_g(r)) << 4); }
// 128-byte rows (8 chunks): chunk c of row r in slot c ^ ((r / 2) % 8).  A
// 256-byte bank line holds two rows, so any 16 consecutive rows read at one
// logical chunk fall on 16 distinct 16-byte bank groups.
__device__ __forceinline__ int swz_g8(int r) { return (r >> 1) & 7; }
template <int RB>
__device__ __forceinline__ int swz_row(int r, int c) {
  if constexpr (RB == 64) return swz(r, c);
  else return r * 128 + ((c ^ swz_g8(r)) << 4);
}

// Workgroup barrier that orders LDS accesses only.  __syncthreads() would
// also wait for every outstanding global->LDS load (vmcnt(0)) and so drain
// the prefetch ring; the explicit waitcnt_vm<> calls do that part.  The asm
// memory clobber keeps the compiler from moving memory accesses across it,
// lgkmcnt(0) retires this wave's LDS reads first (no wave can then overwrite
// a slot another wave is still reading), and sched_barrier(0) pins every
// other instruction to its side.
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_sched_barrier(0);
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
  __builtin_amdgcn_sched_barrier(0);
}

// s_waitcnt with only the vector-memory counter constrained (gfx9 encoding:
// vmcnt[3:0] | expcnt[6:4] | lgkmcnt[11:8] | vmcnt_hi[15:14]).
template <int N>
__device__ __forceinline__ void waitcnt_vm() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | (15 << 8) | ((N >> 4) << 14));
}

// LDS accesses of the epilogue, written as inline asm: the compiler cannot
// tell plain LDS accesses from the ring's direct-to-LDS writes, so before each
// one it would wait for vmcnt(0) -- all ring loads and every output store
// issued so far.  These need no such wait (the scales landed long before, and
// the staging area is never a direct-load target); their lgkmcnt waits are
// explicit (lds_wait_all, the pass loop's wait).
__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return static_cast<uint32_t>(reinterpret_cast<uintptr_t>((__attribute__((address_space(3))) const void*)p));
}
__device__ __forceinline__ void lds_write_b64(uint32_t a, uint32_t lo, uint32_t hi) {
  asm volatile("ds_write_b64 %0, %1" ::"v"(a), "v"(make_uint2(lo, hi)) : "memory");
}
__device__ __forceinline__ void lds_write_b128(uint32_t a, u32x4 v) {
  asm volatile("ds_write_b128 %0, %1" ::"v"(a), "v"(v) : "memory");
}
// Reads without their wait; lds_wait_all() then retires them all and, by
// taking the registers as operands, keeps every use after it.
__device__ __forceinline__ u32x4 lds_read_b128_nw(uint32_t a) {
  u32x4 r;
  asm volatile("ds_read_b128 %0, %1" : "=v"(r) : "v"(a) : "memory");
  return r;
}
__device__ __forceinline__ float lds_read_f32_nw(uint32_t a) {
  float r;
  asm volatile("ds_read_b32 %0, %1" : "=v"(r) : "v"(a) : "memory");
  return r;
}
// The same reads with their wait inside the asm: the register is final when
// the statement ends.  A read without its wait is only safe while nothing
// touches its register before lds_wait_all; where the compiler spills in the
// epilogue it could store such a register before the data arrived.
__device__ __forceinline__ u32x4 lds_read_b128_wait(uint32_t a) {
  u32x4 r;
  asm volatile("ds_read_b128 %0, %1\n\ts_waitcnt lgkmcnt(0)" : "=v"(r) : "v"(a) : "memory");
  return r;
}
__device__ __forceinline__ float lds_read_f32_wait(uint32_t a) {
  float r;
  asm volatile("ds_read_b32 %0, %1\n\ts_waitcnt lgkmcnt(0)" : "=v"(r) : "v"(a) : "memory");
  return r;
}
template <int NV, int NF>
__device__ __forceinline__ void lds_wait_all(u32x4 (&v)[NV], float (&f)[NF]) {
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
#pragma unroll
  for (int i = 0; i < NV; ++i) asm volatile("" : "+v"(v[i]));
#pragma unroll
  for (int i = 0; i < NF; ++i) asm volatile("" : "+v"(f[i]));
}

// Lane id, computed where it is written (a volatile asm is never hoisted
// out of the tile loop, where holding it would cost a register).
__device__ __forceinline__ int lane_id_here() {
  int l;
  asm volatile("v_mbcnt_lo_u32_b32 %0, -1, 0\n\tv_mbcnt_hi_u32_b32 %0, -1, %0" : "=v"(l));
  return l;
}

// A 16-byte-per-lane direct-to-LDS load written as inline asm, for the tile
// scales: issued through the builtin, the compiler would treat every later
// LDS read as possibly aliasing it and wait for vmcnt(0) first -- at the
// next tile's first fragment read, that is for all of the previous tile's
// output stores.  The K loop's own waits cover this load.
typedef int v4i __attribute__((ext_vector_type(4)));
__device__ __forceinline__ void lds_dma_b128(const void* base, uint32_t bytes, uint32_t lds_dst,
                                             uint32_t voff) {
  const uint64_t b = reinterpret_cast<uint64_t>(base);
  v4i rs;
  rs[0] = static_cast<int>(b & 0xFFFFFFFFu);
  rs[1] = static_cast<int>((b >> 32) & 0xFFFFu);
  rs[2] = static_cast<int>(bytes);
  rs[3] = 0x00020000;
  rs[0] = __builtin_amdgcn_readfirstlane(rs[0]);
  rs[1] = __builtin_amdgcn_readfirstlane(rs[1]);
  rs[2] = __builtin_amdgcn_readfirstlane(rs[2]);
  asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dwordx4 %1, %2, 0 offen lds"
               :: "s"(lds_dst), "v"(voff), "s"(rs) : "memory", "m0");
}

// Raw buffer resource over [base, base + bytes): loads past the end return 0.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, bytes, 0x00020000);
}

template <int OUT>
struct OutT {
  static constexpr int kBytes = OUT == FR_DTYPE_FP32 ? 4 : 2;
};

// Four consecutive outputs of one row, with optional bias and residual,
// bounds-checked.
template <int OUT>
__device__ __forceinline__ void store4(void* out, int64_t ldo, int64_t m, int64_t n, int64_t N,
                                       const float* v, const void* bias, const void* res, int64_t ldr) {
  float t[4] = {v[0], v[1], v[2], v[3]};
  if (OUT == FR_DTYPE_FP32) {
    float* o = static_cast<float*>(out) + m * ldo + n;
    if (bias) {
      const float* bb = static_cast<const float*>(bias) + n;
      for (int i = 0; i < 4; ++i)
        if (n + i < N) t[i] += bb[i];
    }
    for (int i = 0; i < 4; ++i)
      if (n + i < N) o[i] = t[i];
    return;
  }
  uint16_t* o = static_cast<uint16_t*>(out) + m * ldo + n;
  if (bias) {
    const uint16_t* bb = static_cast<const uint16_t*>(bias) + n;
    for (int i = 0; i < 4; ++i)
      if (n + i < N) t[i] += (OUT == FR_DTYPE_BF16) ? bf16_to_f32(bb[i]) : fp16_to_f32(bb[i]);
  }
  if (res) {
    // the product is stored in the output dtype first, then added
    const uint16_t* rr = static_cast<const uint16_t*>(res) + m * ldr + n;
    for (int i = 0; i < 4; ++i)
      if (n + i < N)
        t[i] = OUT == FR_DTYPE_BF16 ? round_bf16(t[i]) + bf16_to_f32(rr[i])
                                    : fp16_to_f32(static_cast<uint16_t>(pack_fp16x2(t[i], 0.0f) & 0xFFFFu)) +
                                          fp16_to_f32(rr[i]);
  }
  uint32_t lo = OUT == FR_DTYPE_BF16 ? pack_bf16x2(t[0], t[1]) : pack_fp16x2(t[0], t[1]);
  uint32_t hi = OUT == FR_DTYPE_BF16 ? pack_bf16x2(t[2], t[3]) : pack_fp16x2(t[2], t[3]);
  uint16_t h[4] = {(uint16_t)(lo & 0xFFFF), (uint16_t)(lo >> 16), (uint16_t)(hi & 0xFFFF),
                   (uint16_t)(hi >> 16)};
  for (int i = 0; i < 4; ++i)
    if (n + i < N) o[i] = h[i];
}

// Logical tile id -> (tm, tn): XCD-aware renumbering (workgroup i runs on XCD
// i % 8 and, being persistent, only ever sees ids == i mod 8), then groups of
// kGroupM m-tiles walked n-major so concurrent tiles share panels.
__device__ __forceinline__ void tile_coords(int64_t pid, int64_t nt, int64_t tilesM, int64_t& tm,
                                            int64_t& tn) {
  if ((nt & 7) == 0) pid = (pid & 7) * (nt >> 3) + (pid >> 3);
  constexpr int64_t kGroupM = 8;
  const int64_t tilesN = nt / tilesM;
  const int64_t width = kGroupM * tilesN;
  const int64_t gid = pid / width;
  const int64_t first_m = gid * kGroupM;
  const int64_t gsz = (tilesM - first_m) < kGroupM ? (tilesM - first_m) : kGroupM;
  tm = first_m + (pid % width) % gsz;
  tn = (pid % width) / gsz;
}

// Epilogue of one tile, shared by both GEMM kernels.  Lane l of wave (wn, wm)
// holds, per 32x32 block (i, j) of its WN x WM sub-tile, output row
// m = l%32 of block j and the 4 consecutive columns n = 8q + 4(l/32) + t of
// block i (q, t = 0..3).  Fast path: (acc * sa[m]) * sb[n] is converted and
// written to a per-wave staging tile of 32 rows x SRB bytes per pass
// (16-byte chunks XOR-swizzled by row), read back as 16 consecutive bytes
// per lane and stored as whole SRB-byte row segments.  The tile's scales
// were brought into LDS (`scl`: sb[BN], then sa[BM] from the next 1 KB
// boundary, as fp32) by direct loads
// when the tile started, so the epilogue issues no global load (a load here
// would queue behind the next tile's ring loads: vmcnt retires in order)
// and holds no scale registers through the K loop.  Returns whether a fast
// path ran (and so issued exactly gemm_staged_stores<> stores per wave).
template <int OUT, int EPI, int FN, int FM>
constexpr int gemm_staged_stores() {
  return OUT == FR_DTYPE_FP32 ? 4 * FN * FM : (EPI == kEpiSilu ? FN * FM : 2 * FN * FM);
}

template <int BN, int BM, int WN, int WM, int OUT, int EPI, int SRB>
__device__ __forceinline__ bool gemm_epilogue(const GemmArgs& g, v16f (&acc)[WN / 32][WM / 32], int64_t tm,
                                              int64_t tn, int wn, int wm, uint8_t* scl, uint8_t* stg,
                                              bool sa_vec, bool sb_vec, float sa0, float sb0) {
  constexpr int FN = WN / 32, FM = WM / 32;
  constexpr int EB = OutT<OUT>::kBytes;
  constexpr bool RES = EPI == kEpiRes;
  constexpr bool SILU = EPI == kEpiSilu;
  constexpr int kStagedStores = gemm_staged_stores<OUT, EPI, FN, FM>();
  const int64_t m0 = tm * BM + wm * WM;
  const int64_t n0 = tn * BN + wn * WN;
  // the residual add is compiled into the fast path of the tiles that have
  // registers to spare for it (not the 256 x 256 tile); others take the
  // bounds-checked path for it
  constexpr bool kResFast = !(BN == 256 && BM == 256);
  const bool fast = tm * BM + BM <= g.M && tn * BN + BN <= g.N && g.bias == nullptr &&
                    (!RES || (kResFast && (g.ldr * EB) % 16 == 0 &&
                              (reinterpret_cast<uintptr_t>(g.res) & 15) == 0 && g.ldr < (int64_t(1) << 22))) &&
                    (g.ldo * EB) % 16 == 0 && (reinterpret_cast<uintptr_t>(g.out) & 15) == 0 &&
                    g.ldo < (int64_t(1) << 22);  // tile offsets fit the 32-bit store offsets
  if (!fast && SILU) {
    // gate columns n .. n+3 and their up columns n+8 .. n+11 (N is a
    // multiple of 16, so a chunk is never cut by the edge)
    const int ls = lane_id_here();
    uint16_t* const o16 = static_cast<uint16_t*>(g.out);
#pragma unroll
    for (int j = 0; j < FM; ++j) {
      const int64_t m = m0 + j * 32 + (ls & 31);
      if (m >= g.M) continue;
      const float sam = g.sa[m * g.sa_stride];
#pragma unroll
      for (int i = 0; i < FN; ++i)
#pragma unroll
        for (int q = 0; q < 4; q += 2) {
          const int64_t n = n0 + i * 32 + 8 * q + 4 * (ls >> 5);
          if (n >= g.N) continue;
#pragma unroll
          for (int t = 0; t < 4; ++t) {
            const float gt = round_bf16((acc[i][j][4 * q + t] * sam) * g.sb[(n + t) * g.sb_stride]);
            const float up = round_bf16((acc[i][j][4 * q + 4 + t] * sam) * g.sb[(n + 8 + t) * g.sb_stride]);
            const float sg = __builtin_fabsf(gt) <= 80.0f ? silu_in_range(gt) : gt / (1.0f + expf(-gt));
            o16[m * g.ldo + (n / 16) * 8 + 4 * (ls >> 5) + t] =
                static_cast<uint16_t>(pack_bf16x2(round_bf16(sg) * up, 0.0f) & 0xFFFFu);
          }
        }
    }
    waitcnt_vm<0>();
    return false;
  }
  if (!fast) {
    const int ls = lane_id_here();
#pragma unroll
    for (int j = 0; j < FM; ++j) {
      const int64_t m = m0 + j * 32 + (ls & 31);
      if (m >= g.M) continue;
      const float sam = g.sa[m * g.sa_stride];
#pragma unroll
      for (int i = 0; i < FN; ++i)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const int64_t n = n0 + i * 32 + 8 * q + 4 * (ls >> 5);
          if (n >= g.N) continue;
          float v[4];
#pragma unroll
          for (int t = 0; t < 4; ++t) {
            const int64_t nn = n + t < g.N ? n + t : g.N - 1;
            v[t] = (acc[i][j][4 * q + t] * sam) * g.sb[nn * g.sb_stride];
          }
          store4<OUT>(g.out, g.ldo, m, n, g.N, v, g.bias, RES ? g.res : nullptr, g.ldr);
        }
    }
    // Retire this path's scale and bias loads here: the compiler's wait
    // tracking otherwise carries them around the tile loop and makes the
    // fast path wait for every load in flight before reusing a register.
    waitcnt_vm<0>();
    return false;
  }
  // lane-derived values are formed here from a freshly computed lane id,
  // not hoisted out of the tile loop (held across it they would be
  // spilled, and a reload's vmcnt wait would drain the load ring)
  const int lx = lane_id_here();
  const int row = lx & 31;
  const int h4 = 4 * (lx >> 5);
  const uint32_t sbl = lds_addr(scl) + 4 * (wn * WN + h4);
  // sa[] follows sb[] at the next 1 KB boundary
  const uint32_t sal = lds_addr(scl + ((BN * 4 + 1023) / 1024) * 1024) + 4 * (wm * WM + row);
  // Passes of 32 rows x SRB bytes: pass t = (column group cg, block row j),
  // cg outer, covering CPP output columns (NQ groups u of 8: lane l holds
  // columns 8u + 4(l/32) .. +3 of its row l%32).  The converted outputs go
  // to the wave's staging tile (16-byte chunk c of row r at slot
  // c ^ ((r / RPL) % CPRS), RPL = staging rows per 256-byte bank line: a
  // write of one column group by all 64 lanes then hits each bank at most
  // twice), are read back as 16 consecutive bytes per lane and
  // stored as whole SRB-byte row segments.  Passes are software-pipelined:
  // pass t+1 is scaled and converted while pass t's reads are in flight.
  constexpr int CPP = SRB / EB;        // output columns per pass
  constexpr int NQ = CPP / 8;          // 8-column groups per pass
  constexpr int NCG = WN / CPP;        // column groups per wave
  constexpr int NP = NCG * FM;         // passes
  constexpr int CPRS = SRB / 16;       // 16-byte chunks per staging row (= lanes per row on read-back)
  constexpr int RPL = 256 / SRB;       // staging rows per 256-byte LDS bank line
  constexpr int RPR = 64 / CPRS;       // rows per read-back instruction
  constexpr int NR = 32 / RPR;         // read-backs (and stores) per pass
  // Output side of a pass: the same, except that SiLU passes write half
  // as many columns (CPPO), staged in rows of SRBO bytes.
  constexpr int OD = SILU ? 2 : 1;
  constexpr int CPPO = CPP / OD;
  constexpr int NQO = NQ / OD;
  constexpr int SRBO = CPPO * EB;
  constexpr int CPRSO = SRBO / 16;
  constexpr int RPLO = 256 / SRBO;
  constexpr int RPRO = 64 / CPRSO;
  constexpr int NRO = 32 / RPRO;
  static_assert(!SILU || CPP % 16 == 0, "SiLU passes hold whole gate/up chunks");
  static_assert(NP * NRO == kStagedStores, "store count per tile");
  using PkT = typename std::conditional<EB == 4, u32x4, u32x2>::type;
  const uint32_t stg_base = lds_addr(stg);
  // stores through a buffer resource based at this wave's sub-tile: the
  // lane's offset is formed once, each store's row/column step is a scalar
  // offset (no 64-bit address arithmetic per store)
  const uint64_t obase = reinterpret_cast<uint64_t>(static_cast<uint8_t*>(g.out) + (m0 * g.ldo + n0 / OD) * EB);
  const uint32_t olo = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(obase));
  const uint32_t ohi = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(obase >> 32));
  const __amdgpu_buffer_rsrc_t ro =
      make_rsrc(reinterpret_cast<const void*>((static_cast<uint64_t>(ohi) << 32) | olo), 0xFFFFFFFFu);
  const uint32_t ldo32 = static_cast<uint32_t>(g.ldo);
  const uint32_t vo = ((lx / CPRSO) * ldo32 + (lx % CPRSO) * (16 / EB)) * EB;
  uint32_t ra[NRO];
#pragma unroll
  for (int rr = 0; rr < NRO; ++rr) {
    const int r = rr * RPRO + lx / CPRSO;
    ra[rr] = stg_base + r * SRBO + (((lx % CPRSO) ^ ((r / RPLO) % CPRSO)) << 4);
  }
  // scales: sa of the wave's rows up front, sb per column group
  u32x4 sb4[NQ];
  float sam_r[FM];
  // fp16 outputs: the conversion's extra registers make the compiler spill
  // in this epilogue, and a spilled register of a read still in flight would
  // be stored stale, so that variant waits inside each read
  constexpr bool kSafeReads = OUT == FR_DTYPE_FP16;
  auto load_sb = [&](int cg) __attribute__((always_inline)) {
#pragma unroll
    for (int u = 0; u < NQ; ++u) {
      if (sb_vec) {
        if constexpr (kSafeReads) sb4[u] = lds_read_b128_wait(sbl + 4 * (cg * CPP + 8 * u));
        else sb4[u] = lds_read_b128_nw(sbl + 4 * (cg * CPP + 8 * u));
      } else {
        const uint32_t b0 = __float_as_uint(sb0);
        sb4[u] = u32x4{b0, b0, b0, b0};
      }
    }
  };
#pragma unroll
  for (int j = 0; j < FM; ++j)
    sam_r[j] = sa_vec ? (kSafeReads ? lds_read_f32_wait(sal + 128 * j) : lds_read_f32_nw(sal + 128 * j)) : sa0;
  load_sb(0);
  lds_wait_all(sb4, sam_r);
  PkT pk[NQO];
  auto compute = [&](int t) __attribute__((always_inline)) {
    const int cg = t / FM, j = t % FM;
    if constexpr (SILU) {
      // 8-column groups 2k (gate) and 2k + 1 (up) of the pass are one chunk
      float gt[NQO][4], up[NQO][4], sg[NQO][4];
      float gmax = 0.0f;  // max |gate| (NaN-propagating)
#pragma unroll
      for (int k = 0; k < NQO; ++k) {
        const int col = cg * CPP + 16 * k;
        const int i = col / 32, q = (col % 32) / 8;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          gt[k][e] = (acc[i][j][4 * q + e] * sam_r[j]) * __uint_as_float(sb4[2 * k][e]);
          up[k][e] = (acc[i][j][4 * q + 4 + e] * sam_r[j]) * __uint_as_float(sb4[2 * k + 1][e]);
        }
#pragma unroll
        for (int e = 0; e < 4; e += 2) {
          round_bf16x2(gt[k][e], gt[k][e + 1]);
          round_bf16x2(up[k][e], up[k][e + 1]);
        }
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          gmax = maxnan(gmax, __builtin_fabsf(gt[k][e]));
          sg[k][e] = silu_in_range(gt[k][e]);
        }
      }
      // gates beyond the in-range form (|g| > 80, inf, NaN): torch's formula
      if (__builtin_expect(__ballot(!(gmax <= 80.0f)) != 0, 0)) {
#pragma unroll
        for (int k = 0; k < NQO; ++k)
#pragma unroll
          for (int e = 0; e < 4; ++e)
            if (!(__builtin_fabsf(gt[k][e]) <= 80.0f)) sg[k][e] = gt[k][e] / (1.0f + expf(-gt[k][e]));
      }
#pragma unroll
      for (int k = 0; k < NQO; ++k) {
        round_bf16x2(sg[k][0], sg[k][1]);
        round_bf16x2(sg[k][2], sg[k][3]);
        pk[k][0] = pack_bf16x2(sg[k][0] * up[k][0], sg[k][1] * up[k][1]);
        pk[k][1] = pack_bf16x2(sg[k][2] * up[k][2], sg[k][3] * up[k][3]);
      }
      return;
    }
#pragma unroll
    for (int u = 0; u < NQ; ++u) {
      const int col = cg * CPP + 8 * u;
      const int i = col / 32, q = (col % 32) / 8;
      float v[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) v[e] = (acc[i][j][4 * q + e] * sam_r[j]) * __uint_as_float(sb4[u][e]);
      if constexpr (EB == 4) {
#pragma unroll
        for (int e = 0; e < 4; ++e) pk[u][e] = __float_as_uint(v[e]);
      } else {
        pk[u][0] = OUT == FR_DTYPE_BF16 ? pack_bf16x2(v[0], v[1]) : pack_fp16x2(v[0], v[1]);
        pk[u][1] = OUT == FR_DTYPE_BF16 ? pack_bf16x2(v[2], v[3]) : pack_fp16x2(v[2], v[3]);
      }
    }
  };
  auto stage = [&]() __attribute__((always_inline)) {
#pragma unroll
    for (int u = 0; u < NQO; ++u) {
      const int byte = (8 * u + h4) * EB;  // inside the staging row
      const uint32_t ad = stg_base + row * SRBO + ((((byte >> 4) ^ ((row / RPLO) % CPRSO))) << 4) + (byte & 15);
      if constexpr (EB == 4) lds_write_b128(ad, pk[u]);
      else lds_write_b64(ad, pk[u][0], pk[u][1]);
    }
  };
  u32x4 w[NRO];
  // residual rows (16-bit outputs): read with the same segment layout as
  // the stores, one pass ahead, and added to the converted product
  constexpr bool has_res = RES && kResFast && EB == 2;
  const uint64_t rbase =
      has_res ? reinterpret_cast<uint64_t>(static_cast<const uint8_t*>(g.res) + (m0 * g.ldr + n0) * EB) : 0;
  // (readfirstlane returns int: each word goes through uint32_t before it
  // is widened, or a low word with bit 31 set would sign-extend into the
  // high word)
  const uint32_t rlo = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(rbase));
  const uint32_t rhi = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(rbase >> 32));
  const __amdgpu_buffer_rsrc_t rres =
      make_rsrc(reinterpret_cast<const void*>((static_cast<uint64_t>(rhi) << 32) | rlo), 0xFFFFFFFFu);
  const uint32_t ldr32 = static_cast<uint32_t>(g.ldr);
  const uint32_t vr = ((lx / CPRS) * ldr32 + (lx % CPRS) * (16 / EB)) * EB;
  u32x4 rv[2][NR];
  auto load_res = [&](int t) __attribute__((always_inline)) {
    const int cg = t / FM, j = t % FM;
#pragma unroll
    for (int rr = 0; rr < NR; ++rr)
      rv[t & 1][rr] = __builtin_bit_cast(
          u32x4, __builtin_amdgcn_raw_buffer_load_b128(
                     rres, vr, static_cast<int>(((j * 32 + rr * RPR) * ldr32 + cg * CPP) * EB), 0));
  };
  auto add_res = [&](int t) __attribute__((always_inline)) {
#pragma unroll
    for (int rr = 0; rr < NR; ++rr)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const uint32_t pw = w[rr][e], rw = rv[t & 1][rr][e];
        if constexpr (OUT == FR_DTYPE_BF16) {
          w[rr][e] = pack_bf16x2(__uint_as_float(pw << 16) + __uint_as_float(rw << 16),
                                 __uint_as_float(pw & 0xFFFF0000u) + __uint_as_float(rw & 0xFFFF0000u));
        } else {
          w[rr][e] = pack_fp16x2(fp16_to_f32(static_cast<uint16_t>(pw & 0xFFFFu)) +
                                     fp16_to_f32(static_cast<uint16_t>(rw & 0xFFFFu)),
                                 fp16_to_f32(static_cast<uint16_t>(pw >> 16)) +
                                     fp16_to_f32(static_cast<uint16_t>(rw >> 16)));
        }
      }
  };
  auto read_back = [&]() __attribute__((always_inline)) {
#pragma unroll
    for (int rr = 0; rr < NRO; ++rr) w[rr] = kSafeReads ? lds_read_b128_wait(ra[rr]) : lds_read_b128_nw(ra[rr]);
  };
  // one wait for the reads, taking the next pass's values as operands so
  // their arithmetic stays ahead of it
  auto wait_reads = [&]() __attribute__((always_inline)) {
    if constexpr (NRO == 4 && NQO == 8)
      asm volatile("s_waitcnt lgkmcnt(0)"
                   : "+v"(w[0]), "+v"(w[1]), "+v"(w[2]), "+v"(w[3]), "+v"(pk[0]), "+v"(pk[1]), "+v"(pk[2]),
                     "+v"(pk[3]), "+v"(pk[4]), "+v"(pk[5]), "+v"(pk[6]), "+v"(pk[7])
                   :
                   : "memory");
    else if constexpr (NRO == 4 && NQO == 4)
      asm volatile("s_waitcnt lgkmcnt(0)"
                   : "+v"(w[0]), "+v"(w[1]), "+v"(w[2]), "+v"(w[3]), "+v"(pk[0]), "+v"(pk[1]), "+v"(pk[2]),
                     "+v"(pk[3])
                   :
                   : "memory");
    else if constexpr (NRO == 2 && NQO == 4)
      asm volatile("s_waitcnt lgkmcnt(0)"
                   : "+v"(w[0]), "+v"(w[1]), "+v"(pk[0]), "+v"(pk[1]), "+v"(pk[2]), "+v"(pk[3])
                   :
                   : "memory");
    else if constexpr (NRO == 2 && NQO == 2)
      asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(w[0]), "+v"(w[1]), "+v"(pk[0]), "+v"(pk[1]) : : "memory");
    else if constexpr (NRO == 1 && NQO == 2)
      asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(w[0]), "+v"(pk[0]), "+v"(pk[1]) : : "memory");
    else
      static_assert(NRO == 0, "pass shape");
  };
  if constexpr (has_res) load_res(0);
  compute(0);
  stage();
  read_back();
#pragma unroll
  for (int t = 0; t < NP; ++t) {
    if constexpr (has_res) {
      if (t + 1 < NP) load_res(t + 1);
    }
    if (t + 1 < NP && (t + 1) % FM == 0) {
      // next column group: its scales replace this group's (already applied)
      load_sb((t + 1) / FM);
      lds_wait_all(sb4, sam_r);
    }
    if (t + 1 < NP) compute(t + 1);
    wait_reads();
    if constexpr (has_res) add_res(t);
    const int cg = t / FM, j = t % FM;
    // nontemporal stores (cache policy NT): the output is written once and
    // not read back by this kernel; 2-3 % faster on the 4096-row gate_up,
    // down and M = 512 shapes, the decode step unchanged
#pragma unroll
    for (int rr = 0; rr < NRO; ++rr)
      __builtin_amdgcn_raw_buffer_store_b128(w[rr], ro, vo,
                                             static_cast<int>(((j * 32 + rr * RPRO) * ldo32 + cg * CPPO) * EB), kNT);
    if (t + 1 < NP) {
      stage();
      read_back();
    }
  }
  return true;
}

inline int num_cus() {
  static int cached[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (cached[dev] == 0) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0)
      n = 256;
    cached[dev] = n;
  }
  return cached[dev];
}

}  // namespace fr
