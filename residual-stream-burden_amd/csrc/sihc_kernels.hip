// SiHC hyper-connection read/write path for MI355X (gfx950, CDNA4, wave64).
//
// All kernels here are weighted stream reductions and broadcasts over a packed NHWC
// carrier and packed [tokens, channels] workspace tensors, HBM-bound at 4-slot cells.
// There is no matrix-core work: per element the path does at most 2*E*S flops per
// 2*(S+E) bytes.
//
// Thread mapping of most kernels: a block is (BCG channel groups) x (TL token lanes).
// A lane owns V adjacent channels (up to one 16-byte vector) and walks a run of tokens
// with stride TL, so each wave issues fully coalesced vector loads, and the per-channel
// weights of its channel group are fetched once per block: into LDS when the kernel
// handles many events (read / write / triangular), into registers when it handles one
// (per-event fused kernels). Runs are short (16-64 tokens for the per-event forward,
// read and triangular) or, where a run is one reduction chunk (per-event backward),
// interleaved groups of 32-64 tokens, so the blocks resident at one time stream through
// a narrow window of each array; loads and stores carry non-temporal hints where that
// measured faster. Every token is processed as "issue all loads, then
// compute, then store" with no data-dependent branches in the loop body, so each lane
// keeps all of a token's loads in flight at once (the write also issues the next event
// group's loads early). The pipelined carrier weight gradient instead gives each lane
// one channel and stages whole tiles of rows in LDS with 16-byte loads, one tile ahead.
// All sums are fp32 with a single round-to-nearest-even per stored element. Reductions
// over tokens (weight gradients) are per-lane fp32 partials (for the per-event backward,
// one LDS pass per block), a per-block partial row, then a fixed-order sum over blocks:
// no atomics, bitwise deterministic.
//
// Reference (behaviour, not code): tongtongliang/residual-stream-burden,
// sihc/models/sihc/sublayer_kernels.py (Triton `_read`, `_write`, `_weight_grad`,
// `_triangular`, `_triangular_gamma_grad`) and sihc/bench/fusion_controls.py:14-85.

#include <hip/hip_runtime.h>

#include <algorithm>
#include <atomic>
#include <map>
#include <mutex>
#include <tuple>
#include <cstdarg>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <string>
#include <type_traits>

#include "sihc_hip.h"

// Launch-shape defaults (compile-time constants of the library).
#ifndef SIHC_EV_VEC  // max channels per lane in the per-event kernels (4-slot cells)
#define SIHC_EV_VEC 4
#endif
#ifndef SIHC_EV_BCG  // channel-group lanes per block, per-event kernels
#define SIHC_EV_BCG 32
#endif
#ifndef SIHC_EV_TPT  // tokens per lane, per-event forward
#define SIHC_EV_TPT 2
#endif
#ifndef SIHC_EV_UNROLL  // tokens per lane per loop iteration, per-event kernels
#define SIHC_EV_UNROLL 2
#endif
#ifndef SIHC_EV_FWD16  // 1: 16-slot bf16 per-event forward on the register-lean kernel
#define SIHC_EV_FWD16 1
#endif
#ifndef SIHC_EV_BWD16  // 1: 16-slot bf16 per-event backward on the register-lean kernel
#define SIHC_EV_BWD16 1
#endif
#ifndef SIHC_EV16_MINW  // occupancy hint (min waves per SIMD) of the 16-slot per-event backward
#define SIHC_EV16_MINW 2
#endif
#ifndef SIHC_EV_FWD_THREADS  // threads per one-shot block of the per-event forward (256 or 512)
#define SIHC_EV_FWD_THREADS 256
#endif
#ifndef SIHC_EV_FWD_ROWS  // 1: 4-slot bf16 per-event forward over whole channel rows (k_event_fwd_rows)
#define SIHC_EV_FWD_ROWS 1
#endif
#ifndef SIHC_EV_ROW_THREADS  // target threads per block of k_event_fwd_rows (whole tokens of C/8 lanes)
#define SIHC_EV_ROW_THREADS 720
#endif
#ifndef SIHC_EV_MINW  // occupancy hint (min waves per SIMD) of the per-event kernels
#define SIHC_EV_MINW 1
#endif
#ifndef SIHC_EV_CHUNK  // tokens per reduction chunk, per-event backward (4-slot cells)
#define SIHC_EV_CHUNK 64
#endif
#ifndef SIHC_EV_MAXCHUNKS  // most reduction chunks (partial rows) of the per-event backward (4-slot cells)
#define SIHC_EV_MAXCHUNKS 1024
#endif
#ifndef SIHC_EV_CHUNK_K4  // the same for 16-slot cells, whose partial rows are 4x larger per chunk
#define SIHC_EV_CHUNK_K4 256
#endif
#ifndef SIHC_EV_MAXCHUNKS_K4
#define SIHC_EV_MAXCHUNKS_K4 512
#endif
#ifndef SIHC_EV_GROUP  // tokens per interleaved group of a backward chunk (0: contiguous)
#define SIHC_EV_GROUP 32
#endif
#ifndef SIHC_EV_GROUP_K4  // the same for 16-slot cells
#define SIHC_EV_GROUP_K4 64
#endif
#ifndef SIHC_EV_BWD_NT  // non-temporal hints in the per-event backward: 1 loads, 2 stores, 3 both
#define SIHC_EV_BWD_NT 3
#endif
#ifndef SIHC_EV_FWD_NT  // non-temporal hints in the per-event forward: 1 loads, 2 stores, 3 both
#define SIHC_EV_FWD_NT 3
#endif
// Non-temporal hint modes (1 loads, 2 stores, 3 both) of the stage kernels; -1 selects
// by launch shape.
#ifndef SIHC_RD_NTM
#define SIHC_RD_NTM -1
#endif
#ifndef SIHC_WR_NTM
#define SIHC_WR_NTM -1
#endif
#ifndef SIHC_TRI_NTM
#define SIHC_TRI_NTM -1
#endif
#ifndef SIHC_TRIB_NTM  // the fused triangular backward (weight-gradient kernels storing d)
#define SIHC_TRIB_NTM -1
#endif
#ifndef SIHC_CELLS_NTM  // gather / scatter of cells (both hinted: 7% faster)
#define SIHC_CELLS_NTM 3
#endif
#ifndef SIHC_COPY_NTM  // the library's copy (both hinted: 16% faster)
#define SIHC_COPY_NTM 3
#endif
#ifndef SIHC_RW_BCG  // channel-group lanes per block, read / write / triangular
#define SIHC_RW_BCG 16
#endif
#ifndef SIHC_RW_UNROLL  // tokens per lane per loop iteration, read / write / triangular
#define SIHC_RW_UNROLL 2
#endif
#ifndef SIHC_RW_TPT  // tokens per lane, write (4-slot cells) and 16-slot read / write with few events
#define SIHC_RW_TPT 8
#endif
// 16-slot cells: a lane holds 16 slot vectors per token and reads 16 weights per event
// and channel from LDS, so read / write use narrow vectors and 2 tokens per lane (wider
// shapes exceed 256 VGPRs), and a smaller LDS budget per block keeps 3+ blocks per CU.
#ifndef SIHC_RW_UNROLL_K4  // tokens per lane per iteration of k_read / k_write, 16 slots
#define SIHC_RW_UNROLL_K4 2
#endif
#ifndef SIHC_RW_VEC_K4  // widest vector of k_read / k_write, 16 slots
#define SIHC_RW_VEC_K4 2
#endif
#ifndef SIHC_RW_BCG_K4  // channel-group lanes per block of k_read / k_write, 16 slots
#define SIHC_RW_BCG_K4 32
#endif
#ifndef SIHC_K4_BF16W  // 1: 16-slot read / write stage bf16 weights packed as bf16 in LDS
#define SIHC_K4_BF16W 1
#endif
#ifndef SIHC_K4_DOT2  // 1: 16-slot bf16 read / write / weight gradient sum bf16 pairs with v_dot2c_f32_bf16
#define SIHC_K4_DOT2 1
#endif
#ifndef SIHC_RDW_MINE  // 4-slot bf16 reads with at least this many events: k_read_w (0: never)
#define SIHC_RDW_MINE 17  // XL shape: E = 16 k_read 573 vs 582 us, E = 20 743 vs 710, 8-12 equal
#endif
#ifndef SIHC_RD2_U  // tokens per lane per iteration of the 16-slot dot2 read
#define SIHC_RD2_U 4
#endif
#ifndef SIHC_WR2_U  // tokens per lane per iteration of the 16-slot dot2 write
#define SIHC_WR2_U 2
#endif
#ifndef SIHC_K2_BF16W  // the same for 4-slot read / write (8-channel lanes)
#define SIHC_K2_BF16W 1
#endif
#ifndef SIHC_RW_LDS_K4  // LDS bytes per block for staged weights, 16 slots (of 160 KB per CU):
#define SIHC_RW_LDS_K4 (80 * 1024)  // 32 channel lanes up to 32 events (48 KB: 16 lanes past 24
#endif                              // events, read E = 28 1916 -> 1406 us, write 2290 -> 2129)
#ifndef SIHC_WG_CHUNK  // tokens per reduction chunk, weight / gamma gradients
#define SIHC_WG_CHUNK 512
#endif
#ifndef SIHC_WG_CHUNK_K4  // the same for 16-slot carriers (XL shape, E = 24: 1214 -> 1163 us against 512)
#define SIHC_WG_CHUNK_K4 1024
#endif
#ifndef SIHC_WG_PAD  // most idle event lanes added to make k_wgrad blocks 4 whole waves
#define SIHC_WG_PAD 4
#endif
#ifndef SIHC_TRIB_WAVES  // fused triangular backward: k_trib_waves from this many updates (0: never)
#define SIHC_TRIB_WAVES 3  // A = 3: 229 -> 224 us against the LDS-tile kernel (XL shape)
#endif
#ifndef SIHC_TRIB_CHUNK  // tokens per reduction chunk, fused triangular backward
#define SIHC_TRIB_CHUNK 64
#endif
#ifndef SIHC_WG_TT  // most tokens per staged LDS tile of the weight / gamma gradients
#define SIHC_WG_TT 64
#endif
#ifndef SIHC_WG_BCG  // most channel-group lanes per weight-gradient block
#define SIHC_WG_BCG 64
#endif

#ifndef SIHC_LOAD_FENCE  // 1: keep each token's loads ahead of its arithmetic (see load_fence)
#define SIHC_LOAD_FENCE 1
#endif
#ifndef SIHC_HW_BF16  // 1: fp32 -> bf16 stores through the hardware conversion instruction
#define SIHC_HW_BF16 1
#endif
#ifndef SIHC_RW_MINW  // minimum waves per SIMD read / write are compiled for (caps VGPRs)
#define SIHC_RW_MINW 3
#endif
#ifndef SIHC_C16Z  // 1: pipelined carrier weight gradient (k_wgradz) where it applies
#define SIHC_C16Z 1
#endif
#ifndef SIHC_WR_PF  // 1: k_write prefetches the next event group's update rows
#define SIHC_WR_PF 1
#endif
#ifndef SIHC_XCD_MAP  // 1: XCD-contiguous logical block order (see logical_block)
#define SIHC_XCD_MAP 1
#endif

namespace {

using bf16_t = uint16_t;  // bfloat16 storage (upper 16 bits of an IEEE fp32)

template <int N>
using IC = std::integral_constant<int, N>;

// ----------------------------------------------------------------------------------
// element conversion
// ----------------------------------------------------------------------------------
__device__ __forceinline__ float to_f32(float v) { return v; }
__device__ __forceinline__ float to_f32(bf16_t v) { return __uint_as_float(uint32_t(v) << 16); }

template <typename T>
__device__ __forceinline__ T from_f32(float v);
template <>
__device__ __forceinline__ float from_f32<float>(float v) { return v; }
template <>
__device__ __forceinline__ bf16_t from_f32<bf16_t>(float v) {
#if SIHC_HW_BF16
  // gfx950's v_cvt_pk_bf16_f32 (the compiler pairs adjacent conversions): round to
  // nearest, ties to even, identical to the software path below for every non-NaN
  // input; a NaN keeps its sign and top payload bits (quieted).
  return __builtin_bit_cast(bf16_t, static_cast<__bf16>(v));
#else
  // Round to nearest, ties to even; every NaN becomes the canonical quiet NaN 0x7fc0
  // (the same bits torch's float->bfloat16 conversion produces).
  uint32_t u = __float_as_uint(v);
  if ((u & 0x7fffffffu) > 0x7f800000u) return bf16_t(0x7fc0);
  u += 0x7fffu + ((u >> 16) & 1u);
  return bf16_t(u >> 16);
#endif
}
// Scheduling fence between a token's load phase and its arithmetic. Without it the
// compiler interleaves loads with the math that consumes them to save registers,
// leaving only two or three loads per lane in flight; with it every load of the
// token is issued before the first wait.
__device__ __forceinline__ void load_fence() {
#if SIHC_LOAD_FENCE
  __builtin_amdgcn_sched_barrier(0);
#endif
}

// Value of v after a round trip through T (what a stored-then-reloaded element holds).
template <typename T>
__device__ __forceinline__ float round_as(float v) { return to_f32(from_f32<T>(v)); }

// ----------------------------------------------------------------------------------
// vector load/store of V elements of T as fp32
// ----------------------------------------------------------------------------------
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
template <int BYTES> struct RawT;
template <> struct RawT<16> { using type = u32x4; };
template <> struct RawT<8> { using type = u32x2; };
template <> struct RawT<4> { using type = uint32_t; };
template <> struct RawT<2> { using type = uint16_t; };

// Stream access. NT = non-temporal hint (the `nt` bit of the global load / store). Chosen
// per kernel and launch shape from measurements: loads and stores together speed up the
// balanced streams (per-event kernels 3-6%, writes 3-7%, cell copies 7%, the copy 16%);
// read-dominated streams gain from hinted loads alone (gamma and weight gradients,
// triangular with 7+ updates); hinted loads without hinted stores slow the balanced
// streams down (1-3%); slices narrower than a 128-byte line take no hint (16-slot
// read/write with 16+ events: 7-60% slower).
template <bool NT = false, typename R>
__device__ __forceinline__ R ld(const R* p) {
  if constexpr (NT) {
    return __builtin_nontemporal_load(p);
  } else {
    return *p;
  }
}
template <bool NT = false, typename R>
__device__ __forceinline__ void st(R* p, R v) {
  if constexpr (NT) {
    // An empty register constraint keeps the stored words opaque: otherwise the
    // optimizer folds the bf16 conversion into the store, retypes it as a bfloat
    // vector store and drops the non-temporal hint (checked in the generated code).
    asm volatile("" : "+v"(v));
    __builtin_nontemporal_store(v, p);
  } else {
    *p = v;
  }
}

template <typename T, int V, bool NT = false>
__device__ __forceinline__ void load_vec(const T* __restrict__ p, float* o) {
  constexpr int BYTES = V * int(sizeof(T));
  constexpr int CH = BYTES >= 16 ? 16 : BYTES;
  constexpr int EPC = CH / int(sizeof(T));
  using R = typename RawT<CH>::type;
#pragma unroll
  for (int q = 0; q < BYTES / CH; ++q) {
    R r = ld<NT>(reinterpret_cast<const R*>(p) + q);
    T e[EPC];
    __builtin_memcpy(e, &r, CH);
#pragma unroll
    for (int i = 0; i < EPC; ++i) o[q * EPC + i] = to_f32(e[i]);
  }
}

template <typename T, int V, bool NT = false>
__device__ __forceinline__ void store_vec(T* __restrict__ p, const float* v) {
  constexpr int BYTES = V * int(sizeof(T));
  constexpr int CH = BYTES >= 16 ? 16 : BYTES;
  constexpr int EPC = CH / int(sizeof(T));
  using R = typename RawT<CH>::type;
#pragma unroll
  for (int q = 0; q < BYTES / CH; ++q) {
    T e[EPC];
#pragma unroll
    for (int i = 0; i < EPC; ++i) e[i] = from_f32<T>(v[q * EPC + i]);
    R r;
    __builtin_memcpy(&r, e, CH);
    st<NT>(reinterpret_cast<R*>(p) + q, r);
  }
}

// Weights are tiny and reused by every block: plain cached loads.
template <typename T, int V>
__device__ __forceinline__ void load_vec_cached(const T* __restrict__ p, float* o) {
  constexpr int BYTES = V * int(sizeof(T));
  constexpr int CH = BYTES >= 16 ? 16 : BYTES;
  constexpr int EPC = CH / int(sizeof(T));
  using R = typename RawT<CH>::type;
#pragma unroll
  for (int q = 0; q < BYTES / CH; ++q) {
    R r = reinterpret_cast<const R*>(p)[q];
    T e[EPC];
    __builtin_memcpy(e, &r, CH);
#pragma unroll
    for (int i = 0; i < EPC; ++i) o[q * EPC + i] = to_f32(e[i]);
  }
}

// V elements of T as the raw words a vector load returns: loaded now, converted later
// (a prefetch held in registers costs half the VGPRs of its fp32 values for bf16).
template <typename T, int V>
struct RawVec {
  static constexpr int BYTES = V * int(sizeof(T));
  static constexpr int CH = BYTES >= 16 ? 16 : BYTES;
  using R = typename RawT<CH>::type;
  R r[BYTES / CH];
};
template <typename T, int V, bool NT = false>
__device__ __forceinline__ void load_raw(const T* __restrict__ p, RawVec<T, V>& o) {
  using RV = RawVec<T, V>;
#pragma unroll
  for (int q = 0; q < RV::BYTES / RV::CH; ++q) o.r[q] = ld<NT>(reinterpret_cast<const typename RV::R*>(p) + q);
}
template <typename T, int V>
__device__ __forceinline__ void raw_to_f32(const RawVec<T, V>& in, float* o) {
  using RV = RawVec<T, V>;
  constexpr int EPC = RV::CH / int(sizeof(T));
#pragma unroll
  for (int q = 0; q < RV::BYTES / RV::CH; ++q) {
    T e[EPC];
    __builtin_memcpy(e, &in.r[q], RV::CH);
#pragma unroll
    for (int i = 0; i < EPC; ++i) o[q * EPC + i] = to_f32(e[i]);
  }
}

// ----------------------------------------------------------------------------------
// geometry
// ----------------------------------------------------------------------------------
// Exact unsigned division of n < 2^31 by a runtime divisor d >= 1 as one 64-bit
// multiply and a shift (Granlund & Montgomery, "Division by invariant integers using
// multiplication", 1994): with l = ceil(log2 d), p = 31 + l and m = ceil(2^p / d),
// m * d - 2^p < d <= 2^l, so floor(n * m / 2^p) = floor(n / d) for every n < 2^31, and
// m < 2^32 (m = 2^31 for powers of two). The constants are set once per launch on the
// host; per token this replaces two emulated 32-bit divisions of ~12 instructions each.
struct FastDiv {
  uint32_t m;  // ceil(2^p / d)
  uint32_t p;  // 31 + ceil(log2 d)
};
inline FastDiv make_fastdiv(uint32_t d) {
  uint32_t l = 0;
  while ((uint64_t(1) << l) < d) ++l;
  const uint32_t p = 31 + l;
  const uint64_t num = uint64_t(1) << p;
  return FastDiv{uint32_t((num + d - 1) / d), p};
}
__host__ __device__ __forceinline__ uint32_t fast_div(uint32_t n, FastDiv f) {
  return uint32_t((uint64_t(n) * f.m) >> f.p);
}

struct Geo {
  int M;    // tokens = batch * grid * grid
  int GG;   // grid * grid
  int G;    // workspace grid
  int K;    // cell edge (slots = K*K)
  int GK;   // carrier edge = G*K
  int C;    // channels
  FastDiv divGG, divG;  // division by GG and by G (set_divisors)
};

// Fill the division constants of a geometry whose GG and G are set.
inline void set_divisors(Geo& g) {
  g.divGG = make_fastdiv(uint32_t(g.GG));
  g.divG = make_fastdiv(uint32_t(g.G));
}

struct PtrPack {
  const void* p[SIHC_MAX_EVENTS];
};

// Logical block index of this workgroup in a 1-D grid of n blocks. The dispatcher
// hands workgroups to the 8 XCDs round-robin (workgroup b runs on XCD b % 8), and each
// XCD has its own L2. With XCD set, the remap gives XCD x a contiguous run of logical
// blocks, so the neighbouring channel slices of one token chunk run on one XCD: where
// a slice row is narrower than a 128-byte line (16 lanes x 4 bytes in the 16-slot
// read / write), the two slices that share the line are fetched through one L2
// instead of once per XCD (measured: 2.06x -> 1.18x the algorithmic bytes fetched).
// Kernels whose slice rows are whole lines keep the plain order, which measured
// faster for the 4-slot per-event kernels. A bijection on [0, n) whatever the actual
// placement, so only speed depends on the round-robin.
// logical_block_of(n): the same order over the first n blocks of the grid (blocks past
// them do other work).
template <bool XCD>
__device__ __forceinline__ int logical_block_of(int n) {
  if constexpr (XCD && SIHC_XCD_MAP) {
    const int b = int(blockIdx.x);
    const int q = n >> 3, r = n & 7;  // XCDs 0..r-1 run q+1 blocks, the others q
    const int x = b & 7, i = b >> 3;
    return x < r ? x * (q + 1) + i : r * (q + 1) + (x - r) * q + i;
  } else {
    return int(blockIdx.x);
  }
}
template <bool XCD>
__device__ __forceinline__ int logical_block() {
  return logical_block_of<XCD>(int(gridDim.x));
}

// (slice, chunk) of block blk in a slices-fastest grid, the slice rotated by the chunk. The
// hardware deals consecutive blocks to the 8 XCDs in turn, so with the plain order a slice
// count that shares factors with 8 pins each XCD to a few slices of every row (C = 1024 in
// 128-channel slices: XCD x always takes slice x) and its traffic to a fixed part of every
// 2 KB row; the per-event backward ran 366.6 against 349.0 us at C = 1024 and 746 against
// 684 at C = 2048 (C = 1152, 9 slices: the same). Each chunk still runs every slice once,
// so the partial rows and all sums are unchanged.
__device__ __forceinline__ void slice_chunk(int blk, int nslices, int& slice, int& chunk) {
  chunk = blk / nslices;
  slice = (blk - chunk * nslices + chunk) % nslices;
}
// The same, rotated only for slice counts that are not a multiple of 8: the 4-slot read and
// weight gradient ran slower rotated at C = 1024 (8 / 16 slices: read E = 24 727 -> 759 us,
// gradient E = 16 532 -> 550) and faster at 768, 1152 and 1280 (gradient E = 16 673 -> 653 at
// 1280, read E = 24 812 -> 797 at 1152).
__device__ __forceinline__ void slice_chunk_unless8(int blk, int nslices, int& slice, int& chunk) {
  chunk = blk / nslices;
  const int r = blk - chunk * nslices;
  slice = (nslices & 7) == 0 ? r : (r + chunk) % nslices;
}

// Carrier pixel of slot 0 of the cell token m reads/writes. Token m = b*GG + n owns
// cell n of batch b, or cell index[m] in the spatially indexed variant.
// cell_pixel0_at: the same with the cell already known (`cell` = the clamped index[m]
// when `indexed`, ignored otherwise), for kernels that load the index ahead of use.
__device__ __forceinline__ int64_t cell_pixel0_at(int m, uint32_t cell, bool indexed, const Geo& g) {
  const uint32_t b = fast_div(uint32_t(m), g.divGG);
  const uint32_t n = indexed ? cell : uint32_t(m) - b * uint32_t(g.GG);
  const uint32_t wy = fast_div(n, g.divG);
  const uint32_t wx = n - wy * uint32_t(g.G);
  return (int64_t(b) * g.GK + int64_t(wy) * g.K) * g.GK + int64_t(wx) * g.K;
}
// Out-of-range indices (rejected by the host wrappers) are clamped so that no access can
// leave the carrier.
__device__ __forceinline__ uint32_t index_cell(int m, const Geo& g, const int32_t* __restrict__ index) {
  return min(uint32_t(index[m]), uint32_t(g.GG) - 1u);
}
__device__ __forceinline__ int64_t cell_pixel0(int m, const Geo& g, const int32_t* __restrict__ index) {
  return cell_pixel0_at(m, index ? index_cell(m, g, index) : 0u, index != nullptr, g);
}

// Element offset of (pixel0 + slot s) at channel c, s = uy*K + ux.
template <int K>
__device__ __forceinline__ int64_t slot_offset(int64_t pix0, int s, const Geo& g, int c) {
  return (pix0 + int64_t(s / K) * g.GK + (s % K)) * g.C + c;
}

// LDS layout of a staged weight slice: row r = e*S + s, channel cl = cg*V + v of the
// block's slice. For V >= 4 the row is stored as [V/4][BCG][4] so that the BCG lanes of
// a wave read 16 consecutive bytes each from consecutive addresses (one conflict-free
// ds_read_b128 per 4 channels); narrower vectors use the plain [BCG*V] row.
template <int V>
__device__ __forceinline__ int lds_w(int row, int cg, int v, int BCG) {
  if constexpr (V >= 4) {
    return ((row * (V / 4) + v / 4) * BCG + cg) * 4 + (v & 3);
  } else {
    return row * BCG * V + cg * V + v;
  }
}

// Stage a [E, C, S] weight stack's channel slice [cs, cs+BCG*V) into LDS (layout of
// lds_w, rows e*S+s for e < Epad), zero-filling padded events (e >= E) and channels
// past C.
template <int V, typename TW>
__device__ __forceinline__ void stage_weights(float* lds, const TW* __restrict__ w, int E, int Epad, int S, int BCG,
                                              int cs, int C) {
  const int BC = BCG * V;
  const int tid = threadIdx.y * blockDim.x + threadIdx.x;
  const int nthr = blockDim.x * blockDim.y;
  for (int i = tid; i < Epad * BC * S; i += nthr) {  // global [e][c][s], read coalesced
    const int e = i / (BC * S);
    const int r = i - e * BC * S;
    const int cl = r / S;
    const int s = r - cl * S;
    const int c = cs + cl;
    const int cg = cl / V;
    lds[lds_w<V>(e * S + s, cg, cl - cg * V, BCG)] = (e < E && c < C) ? to_f32(w[(int64_t(e) * C + c) * S + s]) : 0.f;
  }
  __syncthreads();
}

// bf16 weights (V = 2 or 8 channels per lane): the same slice as stage_weights in half
// the LDS, V/2 32-bit words per (row, lane) holding the lane's channels as bf16 pairs
// (low half: the even channel), so a lane reads its row with one 4- or 16-byte access and
// consecutive lanes read consecutive words. Exact: a bf16 weight widens to the same fp32
// value either way.
template <int V>
__device__ __forceinline__ void stage_weights_bf16(uint32_t* lds, const bf16_t* __restrict__ w, int E, int Epad,
                                                   int S, int BCG, int cs, int C) {
  constexpr int NW = V / 2;  // words per (row, lane)
  const int tid = threadIdx.y * blockDim.x + threadIdx.x;
  const int nthr = blockDim.x * blockDim.y;
  const int BP = BCG * NW;  // channel pairs per block
  for (int i = tid; i < Epad * BP * S; i += nthr) {  // [e][pair][s]
    const int e = i / (BP * S);
    const int r = i - e * BP * S;
    const int pr = r / S;
    const int s = r - pr * S;
    const int c = cs + 2 * pr;
    const uint32_t lo = (e < E && c < C) ? uint32_t(w[(int64_t(e) * C + c) * S + s]) : 0u;
    const uint32_t hi = (e < E && c + 1 < C) ? uint32_t(w[(int64_t(e) * C + c + 1) * S + s]) : 0u;
    const int cg = pr / NW, q = pr - cg * NW;
    lds[((e * S + s) * BCG + cg) * NW + q] = lo | (hi << 16);
  }
  __syncthreads();
}
// The V weights of weight row `row` for lane cg from either LDS layout.
template <int V, bool WB>
__device__ __forceinline__ void lds_weights(const float* lds, int row, int cg, int BCG, float (&a)[V]) {
  if constexpr (WB) {
    static_assert(V == 2 || V == 8, "packed bf16 weights: 2 or 8 channels per lane");
    using W = typename RawT<2 * V>::type;
    const W w = reinterpret_cast<const W*>(lds)[row * BCG + cg];
    uint32_t u[V / 2];
    __builtin_memcpy(u, &w, 2 * V);
#pragma unroll
    for (int q = 0; q < V / 2; ++q) {
      a[2 * q] = __uint_as_float(u[q] << 16);
      a[2 * q + 1] = __uint_as_float(u[q] & 0xffff0000u);
    }
  } else {
#pragma unroll
    for (int v = 0; v < V; ++v) a[v] = lds[lds_w<V>(row, cg, v, BCG)];
  }
}

// ----------------------------------------------------------------------------------
// read: out_e[m,c] = sum_s alpha[e,c,s] * x[m,s,c]
// 1-D grid of (slices x chunks), block (BCG, TL); LDS holds alpha as [E][S][BC] fp32.
// ----------------------------------------------------------------------------------
template <typename T, int V, int K, int BCGT, int NTM, bool WB>
__global__ void __launch_bounds__(256, SIHC_RW_MINW) k_read(const T* __restrict__ x, const T* __restrict__ alpha,
                                              PtrPack out, const int32_t* __restrict__ index,
                                              int E, Geo g, int gs, int nchunks, int nslices) {
  constexpr int S = K * K;
  constexpr bool NTL = (NTM & 1) != 0, NTS = (NTM & 2) != 0;  // hints: loads, stores
  // tokens per lane per iteration: each LDS weight feeds U tokens
  constexpr int U = K == 2 ? SIHC_RW_UNROLL : SIHC_RW_UNROLL_K4;
  extern __shared__ float lds[];
  // BCGT: channel-group lanes known at compile time (0: blockDim.x), so LDS row strides
  // fold into the ds_read immediate offsets instead of costing an add per weight row
  const int BCG = BCGT ? BCGT : int(blockDim.x), TL = blockDim.y;
  const int BC = BCG * V;
  const int blk = logical_block<true>(), slice = blk % nslices, chunk = blk / nslices;
  const int cs = slice * BC;
  if constexpr (WB) {
    stage_weights_bf16<V>(reinterpret_cast<uint32_t*>(lds), reinterpret_cast<const bf16_t*>(alpha), E, E, S, BCG,
                          cs, g.C);
  } else {
    stage_weights<V>(lds, alpha, E, E, S, BCG, cs, g.C);
  }
  const int c0 = cs + threadIdx.x * V;
  if (c0 >= g.C) return;
  // The block's tokens: groups of gs tokens (a multiple of U * TL), group `chunk` and
  // every nchunks-th one after it (the launchers pass gs = the block's whole run).
  for (int64_t m0 = int64_t(chunk) * gs; m0 < g.M; m0 += int64_t(nchunks) * gs) {
   const int64_t m_end = min(m0 + gs, int64_t(g.M));
   for (int64_t mi = m0; mi < m_end; mi += U * TL) {
    const int64_t m = mi + threadIdx.y;
    bool ok[U];
    int64_t zoff[U];
    float xv[U][S][V];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      ok[u] = m + u * TL < m_end;
      const int mu = int(ok[u] ? m + u * TL : mi);  // tail: reload a valid token, store nothing
      const int64_t p0 = cell_pixel0(mu, g, index);
      zoff[u] = int64_t(mu) * g.C + c0;
#pragma unroll
      for (int s = 0; s < S; ++s) load_vec<T, V, NTL>(x + slot_offset<K>(p0, s, g, c0), xv[u][s]);
    }
    load_fence();
    for (int e = 0; e < E; ++e) {
      float acc[U][V];
#pragma unroll
      for (int u = 0; u < U; ++u)
#pragma unroll
        for (int v = 0; v < V; ++v) acc[u][v] = 0.f;
#pragma unroll
      for (int s = 0; s < S; ++s) {
        float a[V];
        lds_weights<V, WB>(lds, e * S + s, threadIdx.x, BCG, a);
#pragma unroll
        for (int v = 0; v < V; ++v)
#pragma unroll
          for (int u = 0; u < U; ++u) acc[u][v] = fmaf(a[v], xv[u][s][v], acc[u][v]);
      }
      T* dst = static_cast<T*>(const_cast<void*>(out.p[e]));
#pragma unroll
      for (int u = 0; u < U; ++u)
        if (ok[u]) store_vec<T, V, NTS>(dst + zoff[u], acc[u]);
    }
  }
  }
}

// ----------------------------------------------------------------------------------
// bf16 pair arithmetic (16-slot cells). A 32-bit word holds two bf16 values; pair_lo /
// pair_hi gather the low / high halves of two words into one word (v_perm_b32), and
// dot2 adds both products of two such words to an fp32 accumulator (v_dot2c_f32_bf16:
// the bf16 products are exact in fp32), so one VALU instruction does two multiply-adds.
// ----------------------------------------------------------------------------------
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t pair_lo(uint32_t a, uint32_t b) {  // a.lo | b.lo << 16
  return __builtin_amdgcn_perm(b, a, 0x05040100u);
}
__device__ __forceinline__ uint32_t pair_hi(uint32_t a, uint32_t b) {  // a.hi | b.hi << 16
  return __builtin_amdgcn_perm(b, a, 0x07060302u);
}
__device__ __forceinline__ float dot2(uint32_t a, uint32_t b, float acc) {
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, a), __builtin_bit_cast(bf16x2_t, b), acc,
                                         false);
}

// Stage the read weights of a 2-channel-lane slice [cs, cs + 2*BCG) for the dot2 read:
// alpha [E][C][16] bf16 holds, for each (e, c), the 8 slot-pair words (slots 2p, 2p+1)
// the read multiplies against. LDS layout [e][q][lane][4]: words (pair 2q, channel 0),
// (2q, 1), (2q + 1, 0), (2q + 1, 1), so a lane reads an event's 16 words with four
// consecutive-address 16-byte reads. Channels past C get zero words.
__device__ __forceinline__ void stage_read_pairs(uint32_t* lds, const bf16_t* __restrict__ alpha, int E, int BCG,
                                                 int cs, int C) {
  const uint32_t* w = reinterpret_cast<const uint32_t*>(alpha);
  const int BC = 2 * BCG;
  const int tid = threadIdx.y * blockDim.x + threadIdx.x;
  const int nthr = blockDim.x * blockDim.y;
  for (int i = tid; i < E * BC * 8; i += nthr) {  // global [e][c][pair]: coalesced
    const int e = i / (BC * 8);
    const int r = i - e * BC * 8;
    const int cl = r >> 3, pr = r & 7;
    const int c = cs + cl;
    lds[((e * 4 + (pr >> 1)) * BCG + (cl >> 1)) * 4 + (pr & 1) * 2 + (cl & 1)] =
        c < C ? w[(int64_t(e) * C + c) * 8 + pr] : 0u;
  }
  __syncthreads();
}

// ----------------------------------------------------------------------------------
// 16-slot read in bf16: out_e[m,c] = sum_s alpha[e,c,s] * x[m,s,c] with the slot sum done
// in pairs by dot2. A lane owns 2 channels (one word per token and slot) and U tokens;
// each token's 16 slot words become 8 pair words per channel (pair_lo / pair_hi), which
// then serve all E events. Per event and token a lane issues 16 dot2 (the fp32 kernel:
// 32 FMAs plus the bf16 -> fp32 unpacking of its weights), and each 16-byte LDS weight
// read feeds U tokens. Same block shape, token runs and hints as k_read.
// ----------------------------------------------------------------------------------
template <int U, int BCGT, int NTM>
__global__ void __launch_bounds__(256, SIHC_RW_MINW) k_read_d2(const bf16_t* __restrict__ x,
                                                 const bf16_t* __restrict__ alpha, PtrPack out,
                                                 const int32_t* __restrict__ index, int E, Geo g, int gs,
                                                 int nchunks, int nslices) {
  constexpr int K = 4, S = 16;
  constexpr bool NTL = (NTM & 1) != 0, NTS = (NTM & 2) != 0;  // hints: loads, stores
  extern __shared__ float lds[];
  const int BCG = BCGT ? BCGT : int(blockDim.x), TL = blockDim.y;
  const int blk = logical_block<true>(), slice = blk % nslices, chunk = blk / nslices;
  const int cs = slice * BCG * 2;
  stage_read_pairs(reinterpret_cast<uint32_t*>(lds), alpha, E, BCG, cs, g.C);
  const u32x4* wl = reinterpret_cast<const u32x4*>(lds);
  const int c0 = cs + threadIdx.x * 2;
  if (c0 >= g.C) return;
  // slot s of a cell: carrier row s / 4, pixel s % 4 of the cell's 4-pixel run; in words
  // (2 channels each, C even on this path) a pixel is C / 2 words and a row GK * C / 2
  const int64_t row_w = int64_t(g.GK) * (g.C >> 1);
  const int pix_w = g.C >> 1;
  for (int64_t m0 = int64_t(chunk) * gs; m0 < g.M; m0 += int64_t(nchunks) * gs) {
    const int64_t m_end = min(m0 + gs, int64_t(g.M));
    for (int64_t mi = m0; mi < m_end; mi += U * TL) {
      const int64_t m = mi + threadIdx.y;
      bool ok[U];
      int64_t zoff[U];
      uint32_t xw[U][S];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        ok[u] = m + u * TL < m_end;
        const int mu = int(ok[u] ? m + u * TL : mi);  // tail: reload a valid token, store nothing
        const uint32_t* px = reinterpret_cast<const uint32_t*>(x + cell_pixel0(mu, g, index) * g.C + c0);
        zoff[u] = int64_t(mu) * g.C + c0;
#pragma unroll
        for (int uy = 0; uy < K; ++uy)
#pragma unroll
          for (int ux = 0; ux < K; ++ux) xw[u][uy * K + ux] = ld<NTL>(px + uy * row_w + ux * pix_w);
      }
      load_fence();
      uint32_t xp[U][S / 2][2];  // [token][slot pair][channel]
#pragma unroll
      for (int u = 0; u < U; ++u)
#pragma unroll
        for (int pr = 0; pr < S / 2; ++pr) {
          xp[u][pr][0] = pair_lo(xw[u][2 * pr], xw[u][2 * pr + 1]);
          xp[u][pr][1] = pair_hi(xw[u][2 * pr], xw[u][2 * pr + 1]);
        }
      for (int e = 0; e < E; ++e) {
        float acc[U][2];
#pragma unroll
        for (int u = 0; u < U; ++u) acc[u][0] = acc[u][1] = 0.f;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const u32x4 w = wl[(e * 4 + q) * BCG + threadIdx.x];
#pragma unroll
          for (int u = 0; u < U; ++u) {
            acc[u][0] = dot2(xp[u][2 * q][0], w[0], acc[u][0]);
            acc[u][1] = dot2(xp[u][2 * q][1], w[1], acc[u][1]);
            acc[u][0] = dot2(xp[u][2 * q + 1][0], w[2], acc[u][0]);
            acc[u][1] = dot2(xp[u][2 * q + 1][1], w[3], acc[u][1]);
          }
        }
        // all U chains are computed before the tail test (otherwise the compiler moves each
        // token's chain into its store's branch, leaving two dependent chains at a time)
#pragma unroll
        for (int u = 0; u < U; ++u) asm volatile("" : "+v"(acc[u][0]), "+v"(acc[u][1]));
        bf16_t* dst = static_cast<bf16_t*>(const_cast<void*>(out.p[e]));
#pragma unroll
        for (int u = 0; u < U; ++u)
          if (ok[u]) store_vec<bf16_t, 2, NTS>(dst + zoff[u], acc[u]);
      }
    }
  }
}

// ----------------------------------------------------------------------------------
// write: out[m,s,c] = (add_x ? x : 0) + sum_e beta[e,c,s] * upd_e[m,c]
// Events are consumed in groups of 4 (E padded to a multiple of 4 with zero weights
// and a repeated valid pointer), so each group's 4 update loads issue together.
// ----------------------------------------------------------------------------------
template <typename TX, typename TW, int V, int K, bool ADD_X, int BCGT, int NTM, bool WB>
__global__ void __launch_bounds__(256, SIHC_RW_MINW) k_write(const TX* __restrict__ x, PtrPack upd,
                                               const TW* __restrict__ beta, TX* __restrict__ out,
                                               const int32_t* __restrict__ index, int E, Geo g, int gs,
                                               int nchunks, int nslices) {
  constexpr int S = K * K;
  constexpr bool NTL = (NTM & 1) != 0, NTS = (NTM & 2) != 0;  // hints: loads, stores
  // tokens per lane per iteration: each LDS weight feeds U tokens
  constexpr int U = K == 2 ? SIHC_RW_UNROLL : SIHC_RW_UNROLL_K4;
  constexpr int EG = U > 1 ? 2 : 4;  // events per load group
  extern __shared__ float lds[];
  const int BCG = BCGT ? BCGT : int(blockDim.x), TL = blockDim.y;  // BCGT as in k_read
  const int BC = BCG * V;
  const int blk = logical_block<true>(), slice = blk % nslices, chunk = blk / nslices;
  const int cs = slice * BC;
  const int E4 = (E + 3) & ~3;
  if constexpr (WB) {
    stage_weights_bf16<V>(reinterpret_cast<uint32_t*>(lds), reinterpret_cast<const bf16_t*>(beta), E, E4, S, BCG,
                          cs, g.C);
  } else {
    stage_weights<V>(lds, beta, E, E4, S, BCG, cs, g.C);
  }
  const int c0 = cs + threadIdx.x * V;
  if (c0 >= g.C) return;
  // The block's tokens: groups of gs tokens (a multiple of U * TL), group `chunk` and
  // every nchunks-th one after it (the launchers pass gs = the block's whole run).
  for (int64_t m0 = int64_t(chunk) * gs; m0 < g.M; m0 += int64_t(nchunks) * gs) {
   const int64_t m_end = min(m0 + gs, int64_t(g.M));
   for (int64_t mi = m0; mi < m_end; mi += U * TL) {
    const int64_t m = mi + threadIdx.y;
    bool ok[U];
    int64_t p0[U], zoff[U];
    float acc[U][S][V];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      ok[u] = m + u * TL < m_end;
      const int mu = int(ok[u] ? m + u * TL : mi);  // tail: reload a valid token, store nothing
      p0[u] = cell_pixel0(mu, g, index);
      zoff[u] = int64_t(mu) * g.C + c0;
      if constexpr (ADD_X) {
#pragma unroll
        for (int s = 0; s < S; ++s) load_vec<TX, V, NTL>(x + slot_offset<K>(p0[u], s, g, c0), acc[u][s]);
      } else {
#pragma unroll
        for (int s = 0; s < S; ++s)
#pragma unroll
          for (int v = 0; v < V; ++v) acc[u][s][v] = 0.f;
      }
    }
    // PF: the next group's update loads are issued (raw) before this group is summed,
    // so two groups of loads are in flight (E = 24: 4-slot 1078 -> 1028 us, 16-slot
    // 2136 -> 1964 us at batch 256, D 1152)
    constexpr bool PF = SIHC_WR_PF != 0;
    RawVec<TW, V> dzr[PF ? EG : 1][PF ? U : 1];
    auto issue = [&](int e) {
#pragma unroll
      for (int q = 0; q < EG; ++q)
#pragma unroll
        for (int u = 0; u < U; ++u) load_raw<TW, V, NTL>(static_cast<const TW*>(upd.p[e + q]) + zoff[u], dzr[q][u]);
    };
    if constexpr (PF) issue(0);
    for (int e = 0; e < E4; e += EG) {
      float dz[EG][U][V];
      if constexpr (PF) {
#pragma unroll
        for (int q = 0; q < EG; ++q)
#pragma unroll
          for (int u = 0; u < U; ++u) raw_to_f32<TW, V>(dzr[q][u], dz[q][u]);
        if (e + EG < E4) issue(e + EG);
      } else {
#pragma unroll
        for (int q = 0; q < EG; ++q)
#pragma unroll
          for (int u = 0; u < U; ++u) load_vec<TW, V, NTL>(static_cast<const TW*>(upd.p[e + q]) + zoff[u], dz[q][u]);
      }
      load_fence();
      // Padded events (e + q >= E) loaded a repeated real update: zero the values
      // themselves (a zero weight times an Inf would still give NaN).
#pragma unroll
      for (int q = 0; q < EG; ++q)
        if (e + q >= E)
#pragma unroll
          for (int u = 0; u < U; ++u)
#pragma unroll
            for (int v = 0; v < V; ++v) dz[q][u][v] = 0.f;
#pragma unroll
      for (int q = 0; q < EG; ++q)
#pragma unroll
        for (int s = 0; s < S; ++s) {
          float b[V];
          lds_weights<V, WB>(lds, (e + q) * S + s, threadIdx.x, BCG, b);
#pragma unroll
          for (int v = 0; v < V; ++v)
#pragma unroll
            for (int u = 0; u < U; ++u) acc[u][s][v] = fmaf(b[v], dz[q][u][v], acc[u][s][v]);
        }
    }
#pragma unroll
    for (int u = 0; u < U; ++u)
      if (ok[u]) {
#pragma unroll
        for (int s = 0; s < S; ++s) store_vec<TX, V, NTS>(out + slot_offset<K>(p0[u], s, g, c0), acc[u][s]);
      }
  }
  }
}

// Stage the write weights of a 2-channel-lane slice for the dot2 write: word (j, s, c) =
// beta[2j][c][s] | beta[2j + 1][c][s] << 16, the event pair j's weights of slot s (a zero
// high half past the last event). LDS layout [j][s / 2][lane][4]: words (s even, channel
// 0), (s even, 1), (s odd, 0), (s odd, 1), so a lane reads a pair's 32 words with eight
// consecutive-address 16-byte reads.
__device__ __forceinline__ void stage_write_pairs(uint32_t* lds, const bf16_t* __restrict__ beta, int E, int BCG,
                                                  int cs, int C) {
  const uint16_t* w = reinterpret_cast<const uint16_t*>(beta);
  const int BC = 2 * BCG, J = (E + 1) / 2;
  const int tid = threadIdx.y * blockDim.x + threadIdx.x;
  const int nthr = blockDim.x * blockDim.y;
  for (int i = tid; i < J * BC * 16; i += nthr) {  // [j][c][s]: consecutive slots of one (e, c)
    const int j = i / (BC * 16);
    const int r = i - j * BC * 16;
    const int cl = r >> 4, sl = r & 15;
    const int c = cs + cl;
    uint32_t lo = 0u, hi = 0u;
    if (c < C) {
      lo = w[(int64_t(2 * j) * C + c) * 16 + sl];
      if (2 * j + 1 < E) hi = w[(int64_t(2 * j + 1) * C + c) * 16 + sl];
    }
    lds[((j * 8 + (sl >> 1)) * BCG + (cl >> 1)) * 4 + (sl & 1) * 2 + (cl & 1)] = lo | (hi << 16);
  }
  __syncthreads();
}

// ----------------------------------------------------------------------------------
// 16-slot write in bf16: out[m,s,c] = (add_x ? x[m,s,c] : 0) + sum_e beta[e,c,s] *
// upd_e[m,c], the event sum done in pairs by dot2. A lane owns 2 channels and U tokens
// (16 x 2 fp32 accumulators per token, started from the carrier when add_x); each event
// pair's two update words per token become one pair word per channel (pair_lo /
// pair_hi), multiplied against the staged weight pair of every slot: 32 dot2 per token
// and pair (the fp32 kernel: 64 FMAs plus weight unpacking). The next pair's update
// words are loaded before the current pair is summed. Same block shape, token runs and
// hints as k_write.
// ----------------------------------------------------------------------------------
template <int U, bool ADD_X, int BCGT, int NTM>
__global__ void __launch_bounds__(256, SIHC_RW_MINW) k_write_d2(const bf16_t* __restrict__ x, PtrPack upd,
                                                  const bf16_t* __restrict__ beta, bf16_t* __restrict__ out,
                                                  const int32_t* __restrict__ index, int E, Geo g, int gs,
                                                  int nchunks, int nslices) {
  constexpr int K = 4, S = 16;
  constexpr bool NTL = (NTM & 1) != 0, NTS = (NTM & 2) != 0;  // hints: loads, stores
  extern __shared__ float lds[];
  const int BCG = BCGT ? BCGT : int(blockDim.x), TL = blockDim.y;
  const int blk = logical_block<true>(), slice = blk % nslices, chunk = blk / nslices;
  const int cs = slice * BCG * 2;
  stage_write_pairs(reinterpret_cast<uint32_t*>(lds), beta, E, BCG, cs, g.C);
  const u32x4* wl = reinterpret_cast<const u32x4*>(lds);
  const int c0 = cs + threadIdx.x * 2;
  if (c0 >= g.C) return;
  const int J = (E + 1) / 2;
  // carrier words (2 channels each, C even on this path): a pixel is C / 2 words, a
  // carrier row GK * C / 2
  const int64_t row_w = int64_t(g.GK) * (g.C >> 1);
  const int pix_w = g.C >> 1;
  const uint32_t* xw = reinterpret_cast<const uint32_t*>(x);
  uint32_t* ow = reinterpret_cast<uint32_t*>(out);
  for (int64_t m0 = int64_t(chunk) * gs; m0 < g.M; m0 += int64_t(nchunks) * gs) {
    const int64_t m_end = min(m0 + gs, int64_t(g.M));
    for (int64_t mi = m0; mi < m_end; mi += U * TL) {
      const int64_t m = mi + threadIdx.y;
      bool ok[U];
      int64_t zoff[U], b0[U];
      float acc[U][S][2];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        ok[u] = m + u * TL < m_end;
        const int mu = int(ok[u] ? m + u * TL : mi);  // tail: reload a valid token, store nothing
        b0[u] = (cell_pixel0(mu, g, index) * g.C + c0) >> 1;
        zoff[u] = int64_t(mu) * g.C + c0;
        if constexpr (ADD_X) {
#pragma unroll
          for (int uy = 0; uy < K; ++uy)
#pragma unroll
            for (int ux = 0; ux < K; ++ux) {
              const uint32_t v = ld<NTL>(xw + b0[u] + uy * row_w + ux * pix_w);
              acc[u][uy * K + ux][0] = __uint_as_float(v << 16);
              acc[u][uy * K + ux][1] = __uint_as_float(v & 0xffff0000u);
            }
        } else {
#pragma unroll
          for (int s = 0; s < S; ++s) acc[u][s][0] = acc[u][s][1] = 0.f;
        }
      }
      uint32_t zr[2][U];  // update words of the next event pair: [event of the pair][token]
      auto issue = [&](int j) {
#pragma unroll
        for (int q = 0; q < 2; ++q) {
          const bf16_t* z = static_cast<const bf16_t*>(upd.p[min(2 * j + q, E - 1)]);
#pragma unroll
          for (int u = 0; u < U; ++u) zr[q][u] = ld<NTL>(reinterpret_cast<const uint32_t*>(z + zoff[u]));
        }
      };
      issue(0);
      for (int j = 0; j < J; ++j) {
        uint32_t d[U][2];  // [token][channel]: (event 2j, event 2j + 1) pair words
        const bool second = 2 * j + 1 < E;  // past the last event the pair's high half is zero
#pragma unroll
        for (int u = 0; u < U; ++u) {
          const uint32_t w1 = second ? zr[1][u] : 0u;
          d[u][0] = pair_lo(zr[0][u], w1);
          d[u][1] = pair_hi(zr[0][u], w1);
        }
        if (j + 1 < J) issue(j + 1);
        load_fence();
#pragma unroll
        for (int q = 0; q < 8; ++q) {
          const u32x4 w = wl[(j * 8 + q) * BCG + threadIdx.x];
#pragma unroll
          for (int u = 0; u < U; ++u) {
            acc[u][2 * q][0] = dot2(d[u][0], w[0], acc[u][2 * q][0]);
            acc[u][2 * q][1] = dot2(d[u][1], w[1], acc[u][2 * q][1]);
            acc[u][2 * q + 1][0] = dot2(d[u][0], w[2], acc[u][2 * q + 1][0]);
            acc[u][2 * q + 1][1] = dot2(d[u][1], w[3], acc[u][2 * q + 1][1]);
          }
        }
      }
#pragma unroll
      for (int u = 0; u < U; ++u)
        if (ok[u]) {
#pragma unroll
          for (int uy = 0; uy < K; ++uy)
#pragma unroll
            for (int ux = 0; ux < K; ++ux)
              store_vec<bf16_t, 2, NTS>(reinterpret_cast<bf16_t*>(ow + b0[u] + uy * row_w + ux * pix_w),
                                        acc[u][uy * K + ux]);
        }
    }
  }
}

// ----------------------------------------------------------------------------------
// 4-slot bf16 read with many events, one output array per wave at a time:
// out_e[m,c] = sum_s alpha[e,c,s] * x[m,s,c]. A block (4 waves) owns 128 channels (16
// lanes x 8) and RDW_TT tokens. It stages its cell tile in LDS once, already as slot-pair
// words (word (t, p, c) = x[t, 2p, c] | x[t, 2p + 1, c] << 16) and the weights' own pair
// words alpha[e][c][2p..2p+1]; then wave w writes events w, w + 4, ... one at a time, each
// as RDW_TT / 4 consecutive stores of 4 token rows x 256 bytes to that event's array
// (k_read's lanes store all E arrays for every token pair: 24 arrays at once per wave).
// The slot sum is two dot2 per channel.
// ----------------------------------------------------------------------------------
#ifndef RDW_TT  // tokens per block of k_read_w
#define RDW_TT 32
#endif
template <int NTM>
__global__ void __launch_bounds__(256) k_read_w(const bf16_t* __restrict__ x, const bf16_t* __restrict__ alpha,
                                                PtrPack out, const int32_t* __restrict__ index, int E, Geo g,
                                                int nslices) {
  constexpr int K = 2, LX = 16, V = 8, BC = LX * V, RY = 4;
  constexpr bool NTL = (NTM & 1) != 0, NTS = (NTM & 2) != 0;
  extern __shared__ __align__(16) unsigned char smem_rw[];
  uint32_t* xp = reinterpret_cast<uint32_t*>(smem_rw);  // [RDW_TT][2][BC] pair words
  uint32_t* ap = xp + RDW_TT * 2 * BC;                   // [E][2][BC] pair words
  const int blk = int(blockIdx.x);
  int slice, chunk;
  slice_chunk_unless8(blk, nslices, slice, chunk);
  const int cs = slice * BC;
  const int tid = int(threadIdx.x), wave = tid / 64, lane = tid % 64;
  const int lx = lane % LX, ly = lane / LX;
  const int m0 = chunk * RDW_TT;
  const int tn = min(RDW_TT, g.M - m0);
  // weights: word (e, p, c) = alpha[e][c][2p..2p+1] (zero past C)
  const uint32_t* aw = reinterpret_cast<const uint32_t*>(alpha);
  for (int i = tid; i < E * BC * 2; i += 256) {
    const int e = i / (BC * 2), r = i - e * BC * 2, cl = r >> 1, pr = r & 1;
    const int c = cs + cl;
    ap[(e * 2 + pr) * BC + cl] = c < g.C ? aw[(int64_t(e) * g.C + c) * 2 + pr] : 0u;
  }
  // cell tile: unit u = (token t, channel group j): 4 slot vectors of 8 channels ->
  // 8 pair words per slot pair
  for (int u = tid; u < RDW_TT * LX; u += 256) {
    const int t = u / LX, j = u % LX, c = cs + j * V;
    if (t < tn && c < g.C) {
      const int64_t p0 = cell_pixel0(m0 + t, g, index);
      u32x4 v[4];
#pragma unroll
      for (int sl = 0; sl < 4; ++sl) v[sl] = ld<NTL>(reinterpret_cast<const u32x4*>(x + slot_offset<K>(p0, sl, g, c)));
#pragma unroll
      for (int pr = 0; pr < 2; ++pr) {
        const u32x4 a = v[2 * pr], b = v[2 * pr + 1];
        u32x4 lo, hi;  // channels 0..3 and 4..7 of the group
        lo[0] = pair_lo(a[0], b[0]);
        lo[1] = pair_hi(a[0], b[0]);
        lo[2] = pair_lo(a[1], b[1]);
        lo[3] = pair_hi(a[1], b[1]);
        hi[0] = pair_lo(a[2], b[2]);
        hi[1] = pair_hi(a[2], b[2]);
        hi[2] = pair_lo(a[3], b[3]);
        hi[3] = pair_hi(a[3], b[3]);
        u32x4* dst = reinterpret_cast<u32x4*>(xp + (t * 2 + pr) * BC + j * V);
        dst[0] = lo;
        dst[1] = hi;
      }
    }
  }
  __syncthreads();
  const int c0 = cs + lx * V;
  if (c0 >= g.C) return;  // no barrier below
  for (int e = wave; e < E; e += 4) {
    const u32x4* ae = reinterpret_cast<const u32x4*>(ap + e * 2 * BC + lx * V);
    const u32x4 w00 = ae[0], w01 = ae[1];                       // pair 0, channels 0..3, 4..7
    const u32x4 w10 = ae[BC / 4], w11 = ae[BC / 4 + 1];         // pair 1
    bf16_t* dst = static_cast<bf16_t*>(const_cast<void*>(out.p[e]));
#pragma unroll 2
    for (int t = ly; t < tn; t += RY) {
      const u32x4* xt = reinterpret_cast<const u32x4*>(xp + t * 2 * BC + lx * V);
      const u32x4 x00 = xt[0], x01 = xt[1], x10 = xt[BC / 4], x11 = xt[BC / 4 + 1];
      float acc[V];
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        acc[k] = dot2(x10[k], w10[k], dot2(x00[k], w00[k], 0.f));
        acc[4 + k] = dot2(x11[k], w11[k], dot2(x01[k], w01[k], 0.f));
      }
      store_vec<bf16_t, V, NTS>(dst + int64_t(m0 + t) * g.C + c0, acc);
    }
  }
}

// ----------------------------------------------------------------------------------
// Block reduction helper: sums W = (blockDim.x * NV) floats per thread over threadIdx.y
// and hands each (lane-major) sum to `emit(i, value)`. red must hold TL * W floats.
// ----------------------------------------------------------------------------------
template <int NV, typename Emit>
__device__ __forceinline__ void block_reduce_rows(const float* acc, float* red, Emit&& emit) {
  const int W = blockDim.x * NV;
  const int TL = blockDim.y;
  const int tid = threadIdx.y * blockDim.x + threadIdx.x;
  const int nthr = blockDim.x * TL;
#pragma unroll
  for (int v = 0; v < NV; ++v) red[threadIdx.y * W + threadIdx.x * NV + v] = acc[v];
  __syncthreads();
  for (int i = tid; i < W; i += nthr) {
    float sum = 0.f;
    for (int ty = 0; ty < TL; ++ty) sum += red[ty * W + i];
    emit(i, sum);
  }
  __syncthreads();
}

// ----------------------------------------------------------------------------------
// weight gradient partials: part[chunk][e][s][c] = sum_{m in chunk} x[m,s,c] * z_e[m,c]
// CARRIER: x is the NHWC carrier with S = K*K slots; otherwise x is a workspace
// [M, C] tensor (S = 1; the triangular gamma gradient).
// STORE_D (workspace mode only): also write d_e[m,c] = x[m,c] * gamma[e,c] (the
// triangular update gradients) from the staged x tile, so one pass reads x once, each
// z_e once and writes each d_e once.
// Block = (BCG channel groups) x (E event lanes): lane (e, cg) owns the S x V outputs
// of event e and channel group cg, so each update element is loaded by exactly one
// lane. The block's x tile (TT tokens x S slots x BCG*V channels) is staged in LDS once
// and read by all E event lanes. 1-D grid (slices x chunks).
// ----------------------------------------------------------------------------------
template <typename T, int V, int K, bool CARRIER, bool STORE_D>
__global__ void __launch_bounds__(256) k_wgrad(const T* __restrict__ x, PtrPack z, float* __restrict__ part,
                                               const int32_t* __restrict__ index, int E, Geo g, int tpb,
                                               int nslices, int TT, PtrPack dout, const void* __restrict__ gam,
                                               int gam_f32) {
  // non-temporal loads; the fused triangular backward (3+ updates here) also hints its
  // update-gradient stores (1-2% faster than either alone)
  constexpr int HM = SIHC_TRIB_NTM >= 0 ? SIHC_TRIB_NTM : 3;
  constexpr bool NTL = STORE_D ? (HM & 1) != 0 : true;
  constexpr bool NTS = STORE_D && (HM & 2) != 0;
  constexpr int S = CARRIER ? K * K : 1;
  static_assert(!(STORE_D && CARRIER), "update gradients exist only in workspace mode");
  extern __shared__ float xt[];  // [TT*S rows][BCG*V], lds_w layout
  const int BCG = blockDim.x;
  const int BC = BCG * V;
  const int blk = logical_block<false>();
  int slice, chunk;
  slice_chunk(blk, nslices, slice, chunk);
  const int cs = slice * BC;
  const int cg = threadIdx.x;
  // event lanes past E (padding to whole 4-wave blocks) only help stage the tile
  const int e = min(int(threadIdx.y), E - 1);
  const int c0 = cs + cg * V;
  const bool active = c0 < g.C && int(threadIdx.y) < E;
  const T* __restrict__ ze = static_cast<const T*>(z.p[e]);
  const int tid = threadIdx.y * BCG + threadIdx.x;
  const int nthr = BCG * blockDim.y;
  float acc[S][V];
#pragma unroll
  for (int s = 0; s < S; ++s)
#pragma unroll
    for (int v = 0; v < V; ++v) acc[s][v] = 0.f;
  float gv[V];
  T* __restrict__ de = nullptr;
  if constexpr (STORE_D) {
    de = static_cast<T*>(const_cast<void*>(dout.p[e]));
#pragma unroll
    for (int v = 0; v < V; ++v) {
      const int64_t gi = int64_t(e) * g.C + min(c0 + v, g.C - 1);
      gv[v] = gam_f32 ? static_cast<const float*>(gam)[gi] : to_f32(static_cast<const bf16_t*>(gam)[gi]);
    }
  }
  const int m_begin = chunk * tpb;
  const int m_end = min(m_begin + tpb, g.M);
  for (int t0 = m_begin; t0 < m_end; t0 += TT) {
    // stage the x tile: rows (t, s), BCG vectors per row; 4 vectors per thread are
    // loaded before any is stored so the loads overlap
    const int nvec = TT * S * BCG;
    for (int i0 = tid; i0 < nvec; i0 += 4 * nthr) {
      float v8[4][V];
      int dst[4];
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int i = i0 + q * nthr;
        const int row = min(i, nvec - 1) / BCG;
        const int cgi = min(i, nvec - 1) - row * BCG;
        const int t = row / S;
        const int ss = row - t * S;
        const int m = t0 + t;
        const int ci = cs + cgi * V;
        dst[q] = i < nvec ? row * BCG + cgi : -1;
        if (m < m_end && ci < g.C) {
          int64_t off;
          if constexpr (CARRIER) {
            off = slot_offset<K>(cell_pixel0(m, g, index), ss, g, ci);
          } else {
            off = int64_t(m) * g.C + ci;
          }
          load_vec<T, V, NTL>(x + off, v8[q]);
        } else {
#pragma unroll
          for (int v = 0; v < V; ++v) v8[q][v] = 0.f;
        }
      }
      load_fence();
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        if (dst[q] >= 0) {
          const int row = dst[q] / BCG;
          const int cgi = dst[q] - row * BCG;
#pragma unroll
          for (int v = 0; v < V; ++v) xt[lds_w<V>(row, cgi, v, BCG)] = v8[q][v];
        }
      }
    }
    __syncthreads();
    if (active) {
      const int tn = min(TT, m_end - t0);
      for (int t = 0; t < tn; t += 8) {
        float zv[8][V];
#pragma unroll
        for (int q = 0; q < 8; ++q) {
          const int tq = min(t + q, tn - 1);  // clamp: a repeated token is loaded, not added
          load_vec<T, V, NTL>(ze + int64_t(t0 + tq) * g.C + c0, zv[q]);
        }
        load_fence();
#pragma unroll
        for (int q = 0; q < 8; ++q) {
          if (t + q < tn) {
#pragma unroll
            for (int ss = 0; ss < S; ++ss)
#pragma unroll
              for (int v = 0; v < V; ++v)
                acc[ss][v] = fmaf(xt[lds_w<V>((t + q) * S + ss, cg, v, BCG)], zv[q][v], acc[ss][v]);
            if constexpr (STORE_D) {
              float d[V];
#pragma unroll
              for (int v = 0; v < V; ++v) d[v] = xt[lds_w<V>(t + q, cg, v, BCG)] * gv[v];
              store_vec<T, V, NTS>(de + int64_t(t0 + t + q) * g.C + c0, d);
            }
          }
        }
      }
    }
    __syncthreads();
  }
  if (!active) return;
  float* prow = part + (int64_t(chunk) * E + e) * S * g.C;
#pragma unroll
  for (int ss = 0; ss < S; ++ss) {
#pragma unroll
    for (int v = 0; v < V; ++v) prow[int64_t(ss) * g.C + c0 + v] = acc[ss][v];
  }
}

// ----------------------------------------------------------------------------------
// Fused triangular backward for many updates (workspace mode, whole 16-byte vectors):
//   d_e[m,c] = grad[m,c] * gamma[e,c]    part[chunk][e][c] = sum_{m in chunk} grad * z_e
// One block per (channel slice of 16 lanes x V channels, token chunk). The block stages
// a sub-tile of up to TRIB_TT gradient rows, and the slice of gamma, in LDS as fp32 once;
// then each of its waves takes the updates w, w + NW, ... in turn and streams ONE update
// in and ONE update gradient out at a time. A wave whose loads and stores spread over
// many arrays at once streams markedly slower (a flat 1:1 copy over 24 + 24 arrays:
// 5.3 TB/s when every thread touches all of them, 5.7 when each block touches one; 6.5
// with one array each way), which is what the event-lane kernel k_wgrad does. Each
// lane owns V channels of 4 token rows (16 lanes x 4 rows per wave); the rows of one
// update are loaded as raw words, all before the first use. The 4 rows of a wave are
// added with two fixed-order lane exchanges, so the partial rows are deterministic. ONE:
// the chunk is a single sub-tile (the usual case), so each update's accumulators live
// only while the wave streams it; otherwise they stay in registers across sub-tiles.
// ----------------------------------------------------------------------------------
#define TRIB_TT 64        // most gradient rows per staged sub-tile
#define TRIB_MAXK 8       // most updates per wave (E <= TRIB_MAXK * waves)
#ifndef SIHC_TRIB_RB      // rows of one update loaded per batch by a lane (of TRIB_TT / 4)
#define SIHC_TRIB_RB 8
#endif
#ifndef SIHC_TRIB_MINB    // occupancy hint of k_trib_waves (blocks per CU)
#define SIHC_TRIB_MINB 1
#endif
template <typename T, int V, bool ONE>
__global__ void __launch_bounds__(256, SIHC_TRIB_MINB) k_trib_waves(const T* __restrict__ grad, PtrPack z, float* __restrict__ part,
                                                    int E, Geo g, int tpb, int nslices, PtrPack dout,
                                                    const void* __restrict__ gam, int gam_f32) {
  constexpr int LX = 16, RY = 4, BC = LX * V, RPL = TRIB_TT / RY;  // rows per lane per sub-tile
  constexpr bool NTL = true, NTS = true;
  extern __shared__ float lds[];
  float* gt = lds;                 // [TRIB_TT][BC] gradient rows
  float* gm = lds + TRIB_TT * BC;  // [E][BC] gamma slice
  const int NW = int(blockDim.x) / 64;
  const int blk = int(blockIdx.x);
  int slice, chunk;
  slice_chunk(blk, nslices, slice, chunk);
  const int cs = slice * BC;
  const int tid = int(threadIdx.x), wave = tid / 64, lane = tid % 64;
  const int lx = lane % LX, ly = lane / LX;
  const int c0 = cs + lx * V;
  const bool cok = c0 < g.C;  // the host guarantees C % V == 0: a lane is all in or all out
  const int m_begin = chunk * tpb;
  const int m_end = min(m_begin + tpb, g.M);
  // gamma slice, once per block
  for (int i = tid; i < E * BC; i += blockDim.x) {
    const int e = i / BC, c = cs + (i - e * BC);
    const int64_t gi = int64_t(e) * g.C + min(c, g.C - 1);
    gm[i] = gam_f32 ? static_cast<const float*>(gam)[gi] : to_f32(static_cast<const bf16_t*>(gam)[gi]);
  }
  constexpr int NK = ONE ? 1 : TRIB_MAXK;  // accumulator sets held across sub-tiles
  float acc[NK][V];
#pragma unroll
  for (int k = 0; k < NK; ++k)
#pragma unroll
    for (int v = 0; v < V; ++v) acc[k][v] = 0.f;
  // the 4 token rows of a wave (lanes lx, lx + 16, lx + 32, lx + 48) in fixed order, then
  // the partial row of update e
  auto emit = [&](float (&a)[V], int e) {
#pragma unroll
    for (int v = 0; v < V; ++v) {
      float t = a[v];
      t += __shfl_xor(t, 16);
      t += __shfl_xor(t, 32);
      a[v] = t;
    }
    if (ly == 0 && cok) {
      float* prow = part + (int64_t(chunk) * E + e) * g.C + c0;
#pragma unroll
      for (int v = 0; v < V; ++v) prow[v] = a[v];
    }
  };
  for (int s0 = m_begin; s0 < m_end; s0 += TRIB_TT) {
    const int tn = min(TRIB_TT, m_end - s0);
    // stage the gradient rows of this sub-tile (4 vectors per thread in flight)
    for (int i0 = tid; i0 < tn * LX; i0 += 4 * int(blockDim.x)) {
      float gv[4][V];
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int i = min(i0 + q * int(blockDim.x), tn * LX - 1);
        const int row = i / LX, c = cs + (i - row * LX) * V;
        if (c < g.C) {
          load_vec<T, V, NTL>(grad + int64_t(s0 + row) * g.C + c, gv[q]);
        } else {
#pragma unroll
          for (int v = 0; v < V; ++v) gv[q][v] = 0.f;
        }
      }
      load_fence();
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int i = i0 + q * int(blockDim.x);
        if (i < tn * LX) {
#pragma unroll
          for (int v = 0; v < V; ++v) gt[i * V + v] = gv[q][v];  // row-major [row][BC]
        }
      }
    }
    __syncthreads();
#pragma unroll
    for (int k = 0; k < TRIB_MAXK; ++k) {
      const int e = wave + k * NW;
      float (&ak)[V] = acc[ONE ? 0 : k];
      if (e < E && cok) {
        const T* __restrict__ ze = static_cast<const T*>(z.p[e]);
        T* __restrict__ de = static_cast<T*>(const_cast<void*>(dout.p[e]));
        float gmv[V];
#pragma unroll
        for (int v = 0; v < V; ++v) gmv[v] = gm[e * BC + lx * V + v];
        constexpr int RB = SIHC_TRIB_RB < RPL ? SIHC_TRIB_RB : RPL;
#pragma unroll
        for (int r0 = 0; r0 < RPL; r0 += RB) {
        RawVec<T, V> zr[RB];
#pragma unroll
        for (int rr = 0; rr < RB; ++rr) {
          const int t = min(ly + (r0 + rr) * RY, tn - 1);  // past the sub-tile: a repeated row, loaded not used
          load_raw<T, V, NTL>(ze + int64_t(s0 + t) * g.C + c0, zr[rr]);
        }
        load_fence();
#pragma unroll
        for (int rr = 0; rr < RB; ++rr) {
          const int r = r0 + rr;
          const int t = ly + r * RY;
          if (t < tn) {
            float zv[V], d[V];
            raw_to_f32<T, V>(zr[rr], zv);
            const float* gr = gt + t * BC + lx * V;
#pragma unroll
            for (int v = 0; v < V; ++v) {
              ak[v] = fmaf(gr[v], zv[v], ak[v]);
              d[v] = gr[v] * gmv[v];
            }
            store_vec<T, V, NTS>(de + int64_t(s0 + t) * g.C + c0, d);
          }
        }
        }
      }
      if constexpr (ONE) {  // wave-uniform: every lane exchanges
        if (e < E) {
          emit(ak, e);
#pragma unroll
          for (int v = 0; v < V; ++v) ak[v] = 0.f;
        }
      }
    }
    __syncthreads();
  }
  if constexpr (!ONE) {
#pragma unroll
    for (int k = 0; k < TRIB_MAXK; ++k) {
      const int e = wave + k * NW;
      if (e < E) emit(acc[k], e);
    }
  }
}

// ----------------------------------------------------------------------------------
// Same partial rows as k_wgrad for one or two event lanes, where the shared x tile has
// no reuse to pay for its staging: every lane loads its own x and z_e vectors straight
// from memory, TG tokens per round with all loads issued before the first use, and no
// LDS or barriers. Workspace mode and the 4-slot carrier only (16-slot accumulators
// would not fit the registers beside TG tokens of x).
// ----------------------------------------------------------------------------------
template <typename T, int V, int K, bool CARRIER, bool STORE_D, int HM>
__global__ void __launch_bounds__(256) k_wgrad_direct(const T* __restrict__ x, PtrPack z, float* __restrict__ part,
                                                      const int32_t* __restrict__ index, int E, Geo g, int tpb,
                                                      int nslices, PtrPack dout, const void* __restrict__ gam,
                                                      int gam_f32) {
  // hint mode HM (bit 0 loads, bit 1 stores) applies to the fused triangular backward;
  // the plain weight gradients hint their loads
  constexpr bool NTL = STORE_D ? (HM & 1) != 0 : true;
  constexpr bool NTS = STORE_D && (HM & 2) != 0;
  constexpr int S = CARRIER ? K * K : 1;
  constexpr int TG = CARRIER ? 2 : 4;
  static_assert(!(STORE_D && CARRIER), "update gradients exist only in workspace mode");
  static_assert(S <= 4, "direct path is for the 4-slot carrier and the workspace");
  // plain order: rotated, one event at D = 1152 ran 136.5 -> 139.9 us (1024: 130.9 -> 125.7)
  const int blk = logical_block<false>(), slice = blk % nslices, chunk = blk / nslices;
  const int e = threadIdx.y;
  const int c0 = (slice * blockDim.x + threadIdx.x) * V;
  if (c0 >= g.C) return;  // no barriers below
  const T* __restrict__ ze = static_cast<const T*>(z.p[e]);
  float acc[S][V];
#pragma unroll
  for (int s = 0; s < S; ++s)
#pragma unroll
    for (int v = 0; v < V; ++v) acc[s][v] = 0.f;
  float gv[V];
  T* __restrict__ de = nullptr;
  if constexpr (STORE_D) {
    de = static_cast<T*>(const_cast<void*>(dout.p[e]));
#pragma unroll
    for (int v = 0; v < V; ++v) {
      const int64_t gi = int64_t(e) * g.C + c0 + v;
      gv[v] = gam_f32 ? static_cast<const float*>(gam)[gi] : to_f32(static_cast<const bf16_t*>(gam)[gi]);
    }
  }
  const int m_begin = chunk * tpb;
  const int m_end = min(m_begin + tpb, g.M);
  for (int m0 = m_begin; m0 < m_end; m0 += TG) {
    float xv[TG][S][V], zv[TG][V];
#pragma unroll
    for (int q = 0; q < TG; ++q) {
      const int mq = min(m0 + q, m_end - 1);  // tail: reload a valid token, add nothing
      if constexpr (CARRIER) {
        const int64_t p0 = cell_pixel0(mq, g, index);
#pragma unroll
        for (int s = 0; s < S; ++s) load_vec<T, V, NTL>(x + slot_offset<K>(p0, s, g, c0), xv[q][s]);
      } else {
        load_vec<T, V, NTL>(x + int64_t(mq) * g.C + c0, xv[q][0]);
      }
      load_vec<T, V, NTL>(ze + int64_t(mq) * g.C + c0, zv[q]);
    }
    load_fence();
#pragma unroll
    for (int q = 0; q < TG; ++q) {
      if (m0 + q < m_end) {
#pragma unroll
        for (int s = 0; s < S; ++s)
#pragma unroll
          for (int v = 0; v < V; ++v) acc[s][v] = fmaf(xv[q][s][v], zv[q][v], acc[s][v]);
        if constexpr (STORE_D) {
          float d[V];
#pragma unroll
          for (int v = 0; v < V; ++v) d[v] = xv[q][0][v] * gv[v];
          store_vec<T, V, NTS>(de + int64_t(m0 + q) * g.C + c0, d);
        }
      }
    }
  }
  float* prow = part + (int64_t(chunk) * E + e) * S * g.C;
#pragma unroll
  for (int ss = 0; ss < S; ++ss) {
#pragma unroll
    for (int v = 0; v < V; ++v) prow[int64_t(ss) * g.C + c0 + v] = acc[ss][v];
  }
}

// ----------------------------------------------------------------------------------
// Weight gradient of 16-slot cells (K = 4). k_wgrad's lane (event, channel group)
// would hold 16 x V accumulators and re-read the 16 staged slot values per token for
// every event lane. Here a lane owns ONE channel and a group of C16_EPL events: its
// 16 x C16_EPL accumulators live in registers and every carrier value staged in LDS
// feeds C16_EPL FMAs. Blocks are C16_LANES channel lanes x event groups; the carrier
// tile is staged in LDS once per block, with 16-byte global loads.
// ----------------------------------------------------------------------------------
constexpr int C16_LANES = 64;  // channels per block slice (one per lane of a wave)
constexpr int C16_EPL = 4;     // events per lane
#ifndef SIHC_C16_NQ  // staging loads in flight per thread
#define SIHC_C16_NQ 2
#endif

// LDS carrier tile of 16-slot cells: xt[(t*16 + s)*64 + cl] = x[token t0+t, slot s,
// channel cs+cl], t < tn, raw element copies in VS-element vectors.
template <typename T, int VS>
__device__ __forceinline__ void stage_cells16(T* __restrict__ xt, const T* __restrict__ x, int t0, int tn, int cs,
                                              const Geo& g, const int32_t* __restrict__ index) {
  constexpr int NV = C16_LANES / VS;
  constexpr int NQ = SIHC_C16_NQ;
  using R = typename RawT<VS * int(sizeof(T))>::type;
  const int tid = threadIdx.y * blockDim.x + threadIdx.x;
  const int nthr = blockDim.x * blockDim.y;
  const int total = tn * 16 * NV;
  for (int i0 = tid; i0 < total; i0 += NQ * nthr) {
    R v[NQ];
    int dst[NQ];
#pragma unroll
    for (int q = 0; q < NQ; ++q) {
      const int i = i0 + q * nthr;
      dst[q] = -1;
      if (i < total) {
        const int row = i / NV, j = i - row * NV;
        const int c = cs + j * VS;
        if (c < g.C) {
          const int64_t off = slot_offset<4>(cell_pixel0(t0 + (row >> 4), g, index), row & 15, g, c);
          v[q] = *reinterpret_cast<const R*>(x + off);
          dst[q] = row * C16_LANES + j * VS;
        }
      }
    }
    load_fence();
#pragma unroll
    for (int q = 0; q < NQ; ++q)
      if (dst[q] >= 0) *reinterpret_cast<R*>(xt + dst[q]) = v[q];
  }
}

template <typename T>
__device__ __forceinline__ void stage_cells16_any(int vs, T* xt, const T* x, int t0, int tn, int cs, const Geo& g,
                                                  const int32_t* index) {
  if (vs * int(sizeof(T)) == 16) {
    stage_cells16<T, 16 / int(sizeof(T))>(xt, x, t0, tn, cs, g, index);
  } else if (vs * int(sizeof(T)) == 8) {
    stage_cells16<T, 8 / int(sizeof(T))>(xt, x, t0, tn, cs, g, index);
  } else if (vs * int(sizeof(T)) == 4) {
    stage_cells16<T, 4 / int(sizeof(T))>(xt, x, t0, tn, cs, g, index);
  } else {
    stage_cells16<T, 1>(xt, x, t0, tn, cs, g, index);
  }
}

// weight gradient, 16 slots: lane (channel c, event group eg) accumulates
// part[chunk][e][s][c] = sum_{m in chunk} x[m,s,c] * z_e[m,c] for its 4 events in
// registers, tokens in ascending order (the same partial rows as k_wgrad).
template <typename T>
__global__ void __launch_bounds__(512) k_wgrad16(const T* __restrict__ x, PtrPack z, float* __restrict__ part,
                                                 const int32_t* __restrict__ index, int E, Geo g, int tpb,
                                                 int nslices, int vs) {
  constexpr int S = 16;
  constexpr int TT = 32 / int(sizeof(T));
  __shared__ T xt[TT * S * C16_LANES];
  constexpr int TG = 4;  // tokens whose update loads are issued together
  const int lane = threadIdx.x;
  const int e0 = __builtin_amdgcn_readfirstlane(threadIdx.y) * C16_EPL;
  const int blk = logical_block<false>();
  int slice, chunk;
  slice_chunk(blk, nslices, slice, chunk);
  const int cs = slice * C16_LANES, c = cs + lane;
  const bool cok = c < g.C;
  const T* ze[C16_EPL];
#pragma unroll
  for (int q = 0; q < C16_EPL; ++q) ze[q] = static_cast<const T*>(z.p[min(e0 + q, E - 1)]);
  float acc[C16_EPL][S];
#pragma unroll
  for (int q = 0; q < C16_EPL; ++q)
#pragma unroll
    for (int s = 0; s < S; ++s) acc[q][s] = 0.f;
  const int m_begin = chunk * tpb;
  const int m_end = min(m_begin + tpb, g.M);
  for (int t0 = m_begin; t0 < m_end; t0 += TT) {
    const int tn = min(TT, m_end - t0);
    stage_cells16_any<T>(vs, xt, x, t0, tn, cs, g, index);
    __syncthreads();
    if (cok) {
      for (int t = 0; t < tn; t += TG) {
        float zv[TG][C16_EPL];
#pragma unroll
        for (int u = 0; u < TG; ++u) {
          const int64_t zoff = int64_t(t0 + min(t + u, tn - 1)) * g.C + c;  // clamp: reloaded, not added
#pragma unroll
          for (int q = 0; q < C16_EPL; ++q) zv[u][q] = to_f32(ze[q][zoff]);
        }
        load_fence();
#pragma unroll
        for (int u = 0; u < TG; ++u) {
          if (t + u < tn) {
#pragma unroll
            for (int s = 0; s < S; ++s) {
              const float xs = to_f32(xt[((t + u) * S + s) * C16_LANES + lane]);
#pragma unroll
              for (int q = 0; q < C16_EPL; ++q) acc[q][s] = fmaf(xs, zv[u][q], acc[q][s]);
            }
          }
        }
      }
    }
    __syncthreads();
  }
  if (!cok) return;
#pragma unroll
  for (int q = 0; q < C16_EPL; ++q) {
    if (e0 + q < E) {
      float* prow = part + (int64_t(chunk) * E + e0 + q) * S * g.C + c;
#pragma unroll
      for (int s = 0; s < S; ++s) prow[int64_t(s) * g.C] = acc[q][s];
    }
  }
}

// Pipelined carrier weight gradient (4- and 16-slot cells) for bf16 rows of whole
// 16-byte vectors and up to 32 events. A lane owns ONE channel and EPL events (EPL x S
// accumulators). The update rows join the carrier tile in LDS (16-byte loads: each wave
// stages whole 64-channel rows of its own events, so the update pointer stays
// wave-uniform), and the loads of tile k+1 are issued into registers before tile k is
// reduced, so every tile's HBM latency overlaps the previous tile's arithmetic. Tokens
// are summed in ascending order, as in k_wgrad16 and k_wgrad: for the same chunks the
// partial rows are identical bit for bit.
// NXQ = carrier vectors staged per thread (TT * S * 8 / threads, rounded up); the waves
// and EPL per event count come from measurements (launch_wgrad): 4 or 8 waves where they
// divide the events well (16 slots, E = 24: 6 waves of 4 events 2031 us, 8 waves of 3
// events 1528 us at batch 256, D 1152), else the fastest measured shape.
#ifndef SIHC_WGZ_K2  // 1: 4-slot carriers also use k_wgradz (from 2 events)
#define SIHC_WGZ_K2 1
#endif
#ifndef SIHC_C16Z_MINW  // minimum waves per SIMD k_wgradz is compiled for
#define SIHC_C16Z_MINW 1
#endif
#ifndef SIHC_C16Z_TT
#define SIHC_C16Z_TT 8  // tokens per tile; TT * (64 / 8) must equal one wave (64 lanes)
#endif
template <int K, int NXQ, int EPL>
__global__ void __launch_bounds__(512, SIHC_C16Z_MINW) k_wgradz(const bf16_t* __restrict__ x, PtrPack z,
                                                                float* __restrict__ part,
                                                                const int32_t* __restrict__ index, int E, Geo g,
                                                                int tpb, int nslices) {
  constexpr bool NTL = true;
  constexpr int S = K * K, TT = SIHC_C16Z_TT, VS = 8, NV = C16_LANES / VS;
  constexpr int NXV = TT * S * NV;  // carrier vectors per tile
  constexpr int NZQ = EPL;  // update rows (events) staged per wave: ceil(E / ceil(E / EPL)) <= EPL
  static_assert(TT * NV == C16_LANES, "a wave stages one event's TT update rows");
  using R = u32x4;
  extern __shared__ __align__(16) unsigned char smem16[];
  bf16_t* xt = reinterpret_cast<bf16_t*>(smem16);  // [TT][S][64]
  bf16_t* zt = xt + TT * S * C16_LANES;            // [TT][E][64]
  const int lane = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.y);
  const int nw = blockDim.y, nthr = C16_LANES * nw, tid = wave * C16_LANES + lane;
  const int e0 = wave * EPL;
  const int blk = logical_block<false>();
  int slice, chunk;
  slice_chunk_unless8(blk, nslices, slice, chunk);
  const int cs = slice * C16_LANES, c = cs + lane;
  const bool cok = c < g.C;
  // this lane's update row slot: token zt_t, vector zt_j of the 64-channel row
  const int zt_t = lane / NV, zt_j = lane % NV, zc = cs + zt_j * VS;
  R xb[NXQ], zb[NZQ];
  // Every load is issued, at a clamped in-range address where its vector is not part
  // of the tile (commit skips those): no branches between the loads, so they all stay
  // in flight together. Addresses (and index reads) are formed before the first load.
  auto issue = [&](int t0, int tn) {
    int64_t off[NXQ];
#pragma unroll
    for (int k = 0; k < NXQ; ++k) {
      const int i = min(tid + k * nthr, NXV - 1);
      const int row = i / NV, t = min(row / S, tn - 1), cc = cs + (i % NV) * VS;
      off[k] = slot_offset<K>(cell_pixel0(t0 + t, g, index), row % S, g, cc < g.C ? cc : cs);
    }
    const int64_t zoff = int64_t(t0 + min(zt_t, tn - 1)) * g.C + (zc < g.C ? zc : cs);
#pragma unroll
    for (int k = 0; k < NXQ; ++k) xb[k] = ld<NTL>(reinterpret_cast<const R*>(x + off[k]));
#pragma unroll
    for (int k = 0; k < NZQ; ++k) {
      const int e = min(wave + k * nw, E - 1);
      zb[k] = ld<NTL>(reinterpret_cast<const R*>(static_cast<const bf16_t*>(z.p[e]) + zoff));
    }
  };
  auto commit = [&](int tn) {
#pragma unroll
    for (int k = 0; k < NXQ; ++k) {
      const int i = tid + k * nthr;
      const int row = i / NV, t = row / S, cc = cs + (i % NV) * VS;
      if (i < NXV && t < tn && cc < g.C) *reinterpret_cast<R*>(xt + row * C16_LANES + (i % NV) * VS) = xb[k];
    }
#pragma unroll
    for (int k = 0; k < NZQ; ++k) {
      const int e = wave + k * nw;
      if (e < E && zt_t < tn && zc < g.C)
        *reinterpret_cast<R*>(zt + (zt_t * E + e) * C16_LANES + zt_j * VS) = zb[k];
    }
  };
  int zrow[EPL];  // this lane's event rows within a token's update rows (clamped)
#pragma unroll
  for (int q = 0; q < EPL; ++q) zrow[q] = min(e0 + q, E - 1);
  float acc[EPL][S];
#pragma unroll
  for (int q = 0; q < EPL; ++q)
#pragma unroll
    for (int s = 0; s < S; ++s) acc[q][s] = 0.f;
  const int m_begin = chunk * tpb;
  const int m_end = min(m_begin + tpb, g.M);
  if (m_begin < m_end) issue(m_begin, min(TT, m_end - m_begin));
  for (int t0 = m_begin; t0 < m_end; t0 += TT) {
    const int tn = min(TT, m_end - t0);
    __syncthreads();  // the previous tile is fully reduced
    commit(tn);
    __syncthreads();
    if (t0 + TT < m_end) issue(t0 + TT, min(TT, m_end - t0 - TT));
    load_fence();
    if (cok) {
      for (int t = 0; t < tn; ++t) {
        float zv[EPL];
#pragma unroll
        for (int q = 0; q < EPL; ++q) zv[q] = to_f32(zt[(t * E + zrow[q]) * C16_LANES + lane]);
#pragma unroll
        for (int s = 0; s < S; ++s) {
          const float xs = to_f32(xt[(t * S + s) * C16_LANES + lane]);
#pragma unroll
          for (int q = 0; q < EPL; ++q) acc[q][s] = fmaf(xs, zv[q], acc[q][s]);
        }
      }
    }
  }
  if (!cok) return;
#pragma unroll
  for (int q = 0; q < EPL; ++q) {
    if (e0 + q < E) {
      float* prow = part + (int64_t(chunk) * E + e0 + q) * S * g.C + c;
#pragma unroll
      for (int s = 0; s < S; ++s) prow[int64_t(s) * g.C] = acc[q][s];
    }
  }
}

// ----------------------------------------------------------------------------------
// 16-slot bf16 weight gradient with dot2 over token pairs: dW[e,s,c] partials =
// sum_m z_e[m,c] * x[m,s,c], two tokens per instruction. The block, its event waves and
// the double-buffered staging follow k_wgradz, but the LDS tiles interleave token pairs:
// xt2[((tp * 16 + s) * 64 + cl)] holds x[t0 + 2tp, s, cs + cl] | x[t0 + 2tp + 1, s, cs + cl]
// << 16, zt2[(tp * E + e) * 64 + cl] the same for z_e (a zero high half for the odd last
// token of a tile). A thread stages both tokens of a pair (two 16-byte loads) and packs
// them with pair_lo / pair_hi into two 16-byte LDS writes; a lane then reads one word per
// (pair, slot) and per (pair, event) and issues 16 x EPL dot2 per token pair where
// k_wgradz issues 32 x EPL FMAs plus the bf16 -> fp32 conversions of 2 x (16 + EPL)
// 2-byte LDS reads. Partial rows as k_wgradz (the summation order differs: pairs).
// NPQ: token-pair carrier vectors per thread; EPL: events per wave (lane).
// ----------------------------------------------------------------------------------
template <int NPQ, int EPL>
__global__ void __launch_bounds__(512, SIHC_C16Z_MINW) k_wgradz_d2(const bf16_t* __restrict__ x, PtrPack z,
                                                                   float* __restrict__ part,
                                                                   const int32_t* __restrict__ index, int E, Geo g,
                                                                   int tpb, int nslices) {
  constexpr bool NTL = true;
  constexpr int K = 4, S = 16, TT = SIHC_C16Z_TT, VS = 8, NV = C16_LANES / VS;
  constexpr int TP = TT / 2;           // token pairs per tile
  constexpr int NXP = TP * S * NV;     // carrier vector pairs per tile
  constexpr int NZK = (EPL + 1) / 2;   // update events staged per lane (two lane halves)
  static_assert(TT % 2 == 0 && TP * NV == C16_LANES / 2, "half a wave stages one event's token pairs");
  using R = u32x4;
  extern __shared__ __align__(16) unsigned char smem16[];
  uint32_t* xt = reinterpret_cast<uint32_t*>(smem16);  // [TP][S][64] pair words
  uint32_t* zt = xt + TP * S * C16_LANES;              // [TP][E][64] pair words
  const int lane = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.y);
  const int nw = blockDim.y, nthr = C16_LANES * nw, tid = wave * C16_LANES + lane;
  const int e0 = wave * EPL;
  const int blk = logical_block<false>();
  int slice, chunk;
  slice_chunk(blk, nslices, slice, chunk);
  const int cs = slice * C16_LANES, c = cs + lane;
  const bool cok = c < g.C;
  // this lane's update staging slot: lane half h (events k = h, h + 2, ... of the wave's
  // share wave + k * nw), token pair zp, vector zj of the 64-channel row
  const int zh = lane / (C16_LANES / 2), zp = (lane % (C16_LANES / 2)) / NV, zj = lane % NV;
  const int zc = cs + zj * VS;
  R xb[NPQ][2], zb[NZK][2];
  // every load is issued at a clamped in-range address (commit drops what is not part of
  // the tile), so no branch separates the loads
  auto issue = [&](int t0, int tn) {
    int64_t off[NPQ][2];
#pragma unroll
    for (int k = 0; k < NPQ; ++k) {
      const int i = min(tid + k * nthr, NXP - 1);
      const int row = i / NV, tp = row / S, cc = cs + (i % NV) * VS;
#pragma unroll
      for (int h = 0; h < 2; ++h)
        off[k][h] = slot_offset<K>(cell_pixel0(t0 + min(2 * tp + h, tn - 1), g, index), row % S, g,
                                   cc < g.C ? cc : cs);
    }
    int64_t zoff[2];
#pragma unroll
    for (int h = 0; h < 2; ++h) zoff[h] = int64_t(t0 + min(2 * zp + h, tn - 1)) * g.C + (zc < g.C ? zc : cs);
#pragma unroll
    for (int k = 0; k < NPQ; ++k)
#pragma unroll
      for (int h = 0; h < 2; ++h) xb[k][h] = ld<NTL>(reinterpret_cast<const R*>(x + off[k][h]));
#pragma unroll
    for (int k = 0; k < NZK; ++k) {
      const int e = min(wave + (2 * k + zh) * nw, E - 1);
#pragma unroll
      for (int h = 0; h < 2; ++h)
        zb[k][h] = ld<NTL>(reinterpret_cast<const R*>(static_cast<const bf16_t*>(z.p[e]) + zoff[h]));
    }
  };
  // two 16-byte vectors of 8 channels (tokens 2tp, 2tp + 1) -> 8 pair words in channel order
  auto put_pairs = [](uint32_t* dst, const R& a, const R& b, bool second) {
    // word k of a vector holds channels 2k, 2k + 1: pair words 2k = pair_lo, 2k + 1 =
    // pair_hi; words 0..1 of the vectors give channels 0..3 (lo), words 2..3 channels 4..7
    R lo, hi;
#pragma unroll
    for (int k = 0; k < 2; ++k) {
      const uint32_t bl = second ? b[k] : 0u, bh = second ? b[k + 2] : 0u;
      lo[2 * k] = pair_lo(a[k], bl);
      lo[2 * k + 1] = pair_hi(a[k], bl);
      hi[2 * k] = pair_lo(a[k + 2], bh);
      hi[2 * k + 1] = pair_hi(a[k + 2], bh);
    }
    reinterpret_cast<R*>(dst)[0] = lo;
    reinterpret_cast<R*>(dst)[1] = hi;
  };
  auto commit = [&](int tn) {
#pragma unroll
    for (int k = 0; k < NPQ; ++k) {
      const int i = tid + k * nthr;
      const int row = i / NV, tp = row / S, j = i % NV, cc = cs + j * VS;
      if (i < NXP && 2 * tp < tn && cc < g.C) put_pairs(xt + row * C16_LANES + j * VS, xb[k][0], xb[k][1], 2 * tp + 1 < tn);
    }
#pragma unroll
    for (int k = 0; k < NZK; ++k) {
      const int e = wave + (2 * k + zh) * nw;
      if (2 * k + zh < EPL && e < E && 2 * zp < tn && zc < g.C)
        put_pairs(zt + (zp * E + e) * C16_LANES + zj * VS, zb[k][0], zb[k][1], 2 * zp + 1 < tn);
    }
  };
  int zrow[EPL];  // this lane's event rows within a token pair's update rows (clamped)
#pragma unroll
  for (int q = 0; q < EPL; ++q) zrow[q] = min(e0 + q, E - 1);
  float acc[EPL][S];
#pragma unroll
  for (int q = 0; q < EPL; ++q)
#pragma unroll
    for (int s = 0; s < S; ++s) acc[q][s] = 0.f;
  const int m_begin = chunk * tpb;
  const int m_end = min(m_begin + tpb, g.M);
  if (m_begin < m_end) issue(m_begin, min(TT, m_end - m_begin));
  for (int t0 = m_begin; t0 < m_end; t0 += TT) {
    const int tn = min(TT, m_end - t0);
    __syncthreads();  // the previous tile is fully reduced
    commit(tn);
    __syncthreads();
    if (t0 + TT < m_end) issue(t0 + TT, min(TT, m_end - t0 - TT));
    load_fence();
    if (cok) {
      for (int tp = 0; 2 * tp < tn; ++tp) {
        uint32_t zv[EPL];
#pragma unroll
        for (int q = 0; q < EPL; ++q) zv[q] = zt[(tp * E + zrow[q]) * C16_LANES + lane];
#pragma unroll
        for (int sl = 0; sl < S; ++sl) {
          const uint32_t xs = xt[(tp * S + sl) * C16_LANES + lane];
#pragma unroll
          for (int q = 0; q < EPL; ++q) acc[q][sl] = dot2(xs, zv[q], acc[q][sl]);
        }
      }
    }
  }
  if (!cok) return;
#pragma unroll
  for (int q = 0; q < EPL; ++q) {
    if (e0 + q < E) {
      float* prow = part + (int64_t(chunk) * E + e0 + q) * S * g.C + c;
#pragma unroll
      for (int sl = 0; sl < S; ++sl) prow[int64_t(sl) * g.C] = acc[q][sl];
    }
  }
}

// ----------------------------------------------------------------------------------
// γ gradient partials on 16-byte row lanes (bf16, 3..32 updates, C % 8 == 0, 16-byte
// aligned rows): part[chunk][j][c] = sum over the chunk's tokens m of g[m,c] * u_j[m,c].
// A read-only mix of 1 + A workspace rows. A block is 16 lanes of 8 channels (a 128-channel
// slice) x G update groups x 16 / G token rows (256 threads). Group y takes updates
// y*NA .. y*NA + NA - 1 (past A: the last update again, never written). Every thread
// streams the chunk's tokens r, r + 16 / G, ...: the gradient vector and its NA update
// vectors with 16-byte non-temporal loads, all issued before they are used, summed in fp32
// registers. Nothing is staged in LDS on the way, and there is no barrier in the loop:
// against the LDS-tile kernels (an 8-token tile through registers and LDS, two barriers
// a tile) this ran A = 9 262 -> 229 us, A = 12 324 -> 296, A = 17 453 -> 407, A = 24
// 613 -> 577 at 65,536 rows x 1152 channels. The group's token rows are then summed in
// ascending row order through LDS, one update at a time; each chunk's sum has a fixed
// order, so the result is bitwise repeatable.
// ----------------------------------------------------------------------------------
template <int NA>
__global__ void __launch_bounds__(256) k_gamma_rows(const bf16_t* __restrict__ grad, PtrPack z,
                                                    float* __restrict__ part, int A, int M, int C, int tpb,
                                                    int nslices) {
  __shared__ float red[256 * 8];  // [token row][group][lane][8]
  const int lx = int(threadIdx.x), gy = int(threadIdx.y), r = int(threadIdx.z);
  const int G = int(blockDim.y), TR = int(blockDim.z);
  int slice, chunk;
  slice_chunk(int(blockIdx.x), nslices, slice, chunk);
  const int c0 = slice * 128 + lx * 8;
  const int j0 = gy * NA;
  float acc[NA][8];
#pragma unroll
  for (int q = 0; q < NA; ++q)
#pragma unroll
    for (int k = 0; k < 8; ++k) acc[q][k] = 0.f;
  if (c0 < C) {
    const int m_end = min(chunk * tpb + tpb, M);
    const u32x4* up[NA];
#pragma unroll
    for (int q = 0; q < NA; ++q) up[q] = static_cast<const u32x4*>(z.p[min(j0 + q, A - 1)]);
    const u32x4* gp = reinterpret_cast<const u32x4*>(grad);
    for (int m = chunk * tpb + r; m < m_end; m += TR) {
      const int64_t o = (int64_t(m) * C + c0) >> 3;  // 16-byte vector index
      const u32x4 gv = ld<true>(gp + o);
      u32x4 uv[NA];
#pragma unroll
      for (int q = 0; q < NA; ++q) uv[q] = ld<true>(up[q] + o);
      load_fence();
      // the gradient's 8 values first, then update by update (this order sets the register
      // allocation, and with it the occupancy the group table was measured at: 4 waves per
      // SIMD for 6-8 updates per lane; interleaved per word, 6 took 96 VGPRs and 5 waves, and
      // A = 23 ran 557 -> 587 us)
      float gf[8];
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        gf[2 * k] = __uint_as_float(gv[k] << 16);
        gf[2 * k + 1] = __uint_as_float(gv[k] & 0xffff0000u);
      }
#pragma unroll
      for (int q = 0; q < NA; ++q)
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          acc[q][2 * k] = fmaf(gf[2 * k], __uint_as_float(uv[q][k] << 16), acc[q][2 * k]);
          acc[q][2 * k + 1] = fmaf(gf[2 * k + 1], __uint_as_float(uv[q][k] & 0xffff0000u), acc[q][2 * k + 1]);
        }
    }
  }
  const int tid = (r * G + gy) * 16 + lx;
#pragma unroll
  for (int q = 0; q < NA; ++q) {
#pragma unroll
    for (int k = 0; k < 8; ++k) red[tid * 8 + k] = acc[q][k];
    __syncthreads();
    for (int i = tid; i < G * 128; i += 256) {  // (group, channel of the slice)
      const int gi = i >> 7, cl = i & 127;
      float sum = 0.f;
      for (int rr = 0; rr < TR; ++rr) sum += red[(rr * G + gi) * 128 + cl];
      const int j = gi * NA + q, c = slice * 128 + cl;
      if (j < A && c < C) part[(int64_t(chunk) * A + j) * C + c] = sum;
    }
    __syncthreads();
  }
}

// ----------------------------------------------------------------------------------
// 4-slot carrier weight-gradient partials on the same row lanes (bf16, 16-byte rows):
// part[chunk][e][s][c] = sum over the chunk's tokens m of x[m,s,c] * z_e[m,c]. Lane = 8
// channels of a 128-channel slice; update group y takes events y*NA .. y*NA + NA - 1 (past
// E: the last event again, never written); each thread streams the chunk's tokens r,
// r + 16 / G, ...: the cell's 4 slot vectors (through the state index if any) and its NA
// update vectors, 4 x 8 x NA fp32 sums in registers. Every group loads the cell's slot
// vectors (the other groups' copies come from L2); nothing is staged in LDS. Measured per
// event count against the pipelined kernel at the XL shape (batch 256, D = 1152): E = 5
// 280 -> 249 us, E = 12 414 -> 372, E = 16 525 -> 501, E = 24 734 -> 712, E = 32 1067 ->
// 923; E = 3-4 and 17-18 keep the pipelined kernel (as fast there, or faster).
// ----------------------------------------------------------------------------------
template <int NA>
__global__ void __launch_bounds__(256) k_wgrad_rows(const bf16_t* __restrict__ x, PtrPack z, float* __restrict__ part,
                                                    const int32_t* __restrict__ index, int E, Geo g, int tpb,
                                                    int nslices) {
  constexpr int S = 4;
  __shared__ float red[256 * 8];  // [token row][group][lane][8]
  const int lx = int(threadIdx.x), gy = int(threadIdx.y), r = int(threadIdx.z);
  const int G = int(blockDim.y), TR = int(blockDim.z);
  int slice, chunk;
  slice_chunk(int(blockIdx.x), nslices, slice, chunk);
  const int c0 = slice * 128 + lx * 8;
  const int j0 = gy * NA;
  float acc[NA][S][8];
#pragma unroll
  for (int q = 0; q < NA; ++q)
#pragma unroll
    for (int s = 0; s < S; ++s)
#pragma unroll
      for (int k = 0; k < 8; ++k) acc[q][s][k] = 0.f;
  if (c0 < g.C) {
    const int m_end = min(chunk * tpb + tpb, g.M);
    const u32x4* up[NA];
#pragma unroll
    for (int q = 0; q < NA; ++q) up[q] = static_cast<const u32x4*>(z.p[min(j0 + q, E - 1)]);
    for (int m = chunk * tpb + r; m < m_end; m += TR) {
      const int64_t p0 = cell_pixel0(m, g, index);
      u32x4 xv[S];
#pragma unroll
      for (int s = 0; s < S; ++s) xv[s] = ld<true>(reinterpret_cast<const u32x4*>(x + slot_offset<2>(p0, s, g, c0)));
      const int64_t o = (int64_t(m) * g.C + c0) >> 3;  // 16-byte vector index of the update rows
      u32x4 uv[NA];
#pragma unroll
      for (int q = 0; q < NA; ++q) uv[q] = ld<true>(up[q] + o);
      load_fence();
      float xf[S][8];
#pragma unroll
      for (int s = 0; s < S; ++s)
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          xf[s][2 * k] = __uint_as_float(xv[s][k] << 16);
          xf[s][2 * k + 1] = __uint_as_float(xv[s][k] & 0xffff0000u);
        }
#pragma unroll
      for (int q = 0; q < NA; ++q)
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          const float z0 = __uint_as_float(uv[q][k] << 16), z1 = __uint_as_float(uv[q][k] & 0xffff0000u);
#pragma unroll
          for (int s = 0; s < S; ++s) {
            acc[q][s][2 * k] = fmaf(xf[s][2 * k], z0, acc[q][s][2 * k]);
            acc[q][s][2 * k + 1] = fmaf(xf[s][2 * k + 1], z1, acc[q][s][2 * k + 1]);
          }
        }
    }
  }
  const int tid = (r * G + gy) * 16 + lx;
#pragma unroll
  for (int q = 0; q < NA; ++q)
#pragma unroll
    for (int s = 0; s < S; ++s) {
#pragma unroll
      for (int k = 0; k < 8; ++k) red[tid * 8 + k] = acc[q][s][k];
      __syncthreads();
      for (int i = tid; i < G * 128; i += 256) {  // (group, channel of the slice)
        const int gi = i >> 7, cl = i & 127;
        float sum = 0.f;
        for (int rr = 0; rr < TR; ++rr) sum += red[(rr * G + gi) * 128 + cl];
        const int e = gi * NA + q, c = slice * 128 + cl;
        if (e < E && c < g.C) part[((int64_t(chunk) * E + e) * S + s) * g.C + c] = sum;
      }
      __syncthreads();
    }
}

// ----------------------------------------------------------------------------------
// Fixed-order sum of partial rows. part is [chunks][R][S][C]; row r of the result
// goes to out0 + r*C*S ([R][C][S], `pair` == 0) or, with `pair`, row 0 -> out0 and
// row 1 -> out1 (each [C][S]). Rows whose bit is set in zero_mask are written as
// zeros without reading partials; a NULL destination row is skipped.
// Block: 32 x NV outputs x 8 chunk groups; each group sums its chunks in ascending
// order, then the 8 group sums are added in ascending group order. With NV = 4 a thread
// reads four neighbouring outputs of each partial row as one 16-byte load (the group's
// lanes then read 512 contiguous bytes per row instead of 128); the sums, and so the
// bits, do not depend on NV.
// ----------------------------------------------------------------------------------
// Block of 256 threads (`tid` = flat thread index); `red` holds FINALIZE_LDS floats of LDS.
#ifndef FINALIZE_FO
#define FINALIZE_FO 32  // output lanes of a block (each NV outputs)
#endif
#ifndef FINALIZE_FG
#define FINALIZE_FG 8   // chunk groups of a block (FINALIZE_FO x FINALIZE_FG = 256 threads)
#endif
static_assert(FINALIZE_FO * FINALIZE_FG == 256, "finalize blocks are 256 threads");
#define FINALIZE_LDS(NV) (FINALIZE_FG * FINALIZE_FO * (NV))
template <typename TO, int NV>
__device__ __forceinline__ void finalize_outputs(const float* __restrict__ part, TO* __restrict__ out0,
                                                 TO* __restrict__ out1, int chunks, int R, int S, int C, int pair,
                                                 int zero_mask, int block, float* __restrict__ lds, int tid) {
  constexpr int FO = FINALIZE_FO, FG = FINALIZE_FG;
  float(*red)[FO * NV] = reinterpret_cast<float(*)[FO * NV]>(lds);  // [FG][FO * NV]
  const int64_t n = int64_t(R) * S * C, SC = int64_t(S) * C;  // NV > 1: SC % NV == 0
  const int o = tid % FO, grp = tid / FO;
  const int64_t i = (int64_t(block) * FO + o) * NV;  // this thread's first output
  const bool live = i < n;
  const int r = live ? int(i / SC) : 0;  // the NV outputs share the row r
  const bool zero = (zero_mask >> r) & 1;
  float sum[NV];
#pragma unroll
  for (int j = 0; j < NV; ++j) sum[j] = 0.f;
  if (live && !zero) {
    // 8 independent loads in flight per thread; the sum order stays ascending in k.
    int k = grp;
    for (; k + 7 * FG < chunks; k += 8 * FG) {
      float v[8][NV];
#pragma unroll
      for (int q = 0; q < 8; ++q) load_vec<float, NV>(part + int64_t(k + q * FG) * n + i, v[q]);
#pragma unroll
      for (int q = 0; q < 8; ++q)
#pragma unroll
        for (int j = 0; j < NV; ++j) sum[j] += v[q][j];
    }
    for (; k < chunks; k += FG) {
      float v[NV];
      load_vec<float, NV>(part + int64_t(k) * n + i, v);
#pragma unroll
      for (int j = 0; j < NV; ++j) sum[j] += v[j];
    }
  }
#pragma unroll
  for (int j = 0; j < NV; ++j) red[grp][o * NV + j] = sum[j];
  __syncthreads();
  if (grp != 0 || !live) return;
  TO* dst = pair ? (r == 0 ? out0 : out1) : (out0 ? out0 + int64_t(r) * C * S : nullptr);
  if (!dst) return;
#pragma unroll
  for (int j = 0; j < NV; ++j) {
    float t = 0.f;
#pragma unroll
    for (int q = 0; q < FG; ++q) t += red[q][o * NV + j];
    const int rem = int(i + j - int64_t(r) * SC);
    const int s = rem / C;
    const int c = rem - s * C;
    dst[int64_t(c) * S + s] = from_f32<TO>(zero ? 0.f : t);
  }
}

template <typename TO, int NV>
__global__ void __launch_bounds__(256) k_finalize(const float* __restrict__ part, TO* __restrict__ out0,
                                                  TO* __restrict__ out1, int chunks, int R, int S, int C,
                                                  int pair, int zero_mask) {
  __shared__ float red[FINALIZE_LDS(NV)];
  finalize_outputs<TO, NV>(part, out0, out1, chunks, R, S, C, pair, zero_mask, int(blockIdx.x), red,
                           int(threadIdx.x));
}

// The per-event backward's finalize for up to SIHC_FINALIZE_BATCH deferred events in one
// launch (grid.y = event): the same fixed-order sums as k_finalize, so the same bits.
// Partial rows of the per-event backward are 16-byte aligned with 2 x S x C (S = 4 or 16)
// entries, so every event takes the 4-wide path.
#define SIHC_FINALIZE_BATCH 32
struct FinalizeBatch {
  const float* part[SIHC_FINALIZE_BATCH];
  void* out0[SIHC_FINALIZE_BATCH];
  void* out1[SIHC_FINALIZE_BATCH];
  int chunks[SIHC_FINALIZE_BATCH];
  int zero_mask[SIHC_FINALIZE_BATCH];
};

template <typename TO>
__global__ void __launch_bounds__(256) k_finalize_batch(FinalizeBatch b, int S, int C) {
  const int e = int(blockIdx.y);
  __shared__ float red[FINALIZE_LDS(4)];
  finalize_outputs<TO, 4>(b.part[e], static_cast<TO*>(b.out0[e]), static_cast<TO*>(b.out1[e]), b.chunks[e], 2, S, C,
                          1, b.zero_mask[e], int(blockIdx.x), red, int(threadIdx.x));
}

// The deferred finalize of one earlier per-event backward call, run by the trailing
// blocks of a later per-event backward launch (sihc_event_backward_chain): blocks
// nmain, nmain + 1, ... of that grid are dispatched after every block of the backward
// proper, so they run while its last round of blocks drains. Same fixed-order sums
// (finalize_outputs, 4 outputs per thread) as k_finalize_batch, so the same bits.
struct EvCarry {
  const float* part;  // the earlier call's partial rows [chunks][2][S][C] (NULL: none)
  void* out0;         // its grad_beta [C][S] (NULL: row 0 not stored)
  void* out1;         // its grad_alpha_next [C][S] (NULL: row 1 not stored)
  int chunks;         // its partial-row count
  int zero_mask;      // rows stored as zeros without reading partials
  int nmain;          // blocks of the launch's own backward; blocks from here on finalize
};
#define EV_CARRY_OUTPUTS_PER_BLOCK (FINALIZE_FO * 4)

template <typename T>
__device__ __forceinline__ bool run_carry(const EvCarry& carry, int S, int C, float* lds) {
  if (int(blockIdx.x) < carry.nmain) return false;
  finalize_outputs<T, 4>(carry.part, static_cast<T*>(carry.out0), static_cast<T*>(carry.out1), carry.chunks, 2, S, C,
                         1, carry.zero_mask, int(blockIdx.x) - carry.nmain, lds,
                         int(threadIdx.y * blockDim.x + threadIdx.x));
  return true;
}

template <typename TO>
__global__ void __launch_bounds__(256) k_fill_zero(TO* __restrict__ out, int64_t n) {
  const int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i < n) out[i] = from_f32<TO>(0.f);
}

// ----------------------------------------------------------------------------------
// triangular: out[m,c] = base[m,c] + sum_j gamma[j,c] * upd_j[m,c]
// (active count padded to a multiple of 4 with zero gamma rows, as in k_write)
// ----------------------------------------------------------------------------------
template <typename T, typename TG, int V, int NTM>
__global__ void __launch_bounds__(256) k_triangular(const T* __restrict__ base, PtrPack upd,
                                                    const TG* __restrict__ gamma, T* __restrict__ out,
                                                    int A, int M, int C, int gs, int nchunks, int nslices) {
  constexpr bool NTL = (NTM & 1) != 0, NTS = (NTM & 2) != 0;  // hints: loads, stores
  constexpr int U = SIHC_RW_UNROLL;  // tokens per lane per iteration: each LDS weight feeds U tokens
  extern __shared__ float lds[];
  const int BCG = blockDim.x, TL = blockDim.y;
  const int BC = BCG * V;
  const int blk = logical_block<false>();
  int slice, chunk;
  slice_chunk(blk, nslices, slice, chunk);
  const int cs = slice * BC;
  const int A4 = (A + 3) & ~3;
  const int tid = threadIdx.y * BCG + threadIdx.x;
  for (int i = tid; i < A4 * BC; i += BCG * TL) {
    const int j = i / BC;
    const int cl = i - j * BC;
    const int c = cs + cl;
    const int cg = cl / V;
    lds[lds_w<V>(j, cg, cl - cg * V, BCG)] = (j < A && c < C) ? to_f32(gamma[int64_t(j) * C + c]) : 0.f;
  }
  __syncthreads();
  const int c0 = cs + threadIdx.x * V;
  if (c0 >= C) return;
  // The block's tokens: groups of gs tokens (a multiple of U * TL), group `chunk` and
  // every nchunks-th one after it (the launchers pass gs = the block's whole run).
  for (int64_t m0 = int64_t(chunk) * gs; m0 < M; m0 += int64_t(nchunks) * gs) {
   const int64_t m_end = min(m0 + gs, int64_t(M));
   for (int64_t mi = m0; mi < m_end; mi += U * TL) {
    const int64_t m = mi + threadIdx.y;
    bool ok[U];
    int64_t off[U];
    float acc[U][V];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      ok[u] = m + u * TL < m_end;
      off[u] = (ok[u] ? m + u * TL : mi) * C + c0;
      load_vec<T, V, NTL>(base + off[u], acc[u]);
    }
    for (int j = 0; j < A4; j += 4) {
      float dz[4][U][V];
#pragma unroll
      for (int q = 0; q < 4; ++q)
#pragma unroll
        for (int u = 0; u < U; ++u) load_vec<T, V, NTL>(static_cast<const T*>(upd.p[j + q]) + off[u], dz[q][u]);
      load_fence();
#pragma unroll
      for (int q = 0; q < 4; ++q)
        if (j + q >= A)  // padded update: zero the loaded values (0 * Inf is NaN)
#pragma unroll
          for (int u = 0; u < U; ++u)
#pragma unroll
            for (int v = 0; v < V; ++v) dz[q][u][v] = 0.f;
#pragma unroll
      for (int q = 0; q < 4; ++q)
#pragma unroll
        for (int v = 0; v < V; ++v) {
          const float gm = lds[lds_w<V>(j + q, threadIdx.x, v, BCG)];
#pragma unroll
          for (int u = 0; u < U; ++u) acc[u][v] = fmaf(gm, dz[q][u][v], acc[u][v]);
        }
    }
#pragma unroll
    for (int u = 0; u < U; ++u)
      if (ok[u]) store_vec<T, V, NTS>(out + off[u], acc[u]);
  }
  }
}

// ----------------------------------------------------------------------------------
// per-event fused forward: x_out = x + beta*dz ; z_out = sum_s alpha_next * x_out
// The single event's [C,S] weights of the lane's V channels live in registers.
// ----------------------------------------------------------------------------------
template <typename T, int V, int K>
__device__ __forceinline__ void load_weights(const T* __restrict__ w, int c0, float (&out)[K * K][V]) {
  constexpr int S = K * K;
  float tmp[V * S];
  load_vec_cached<T, V * S>(w + int64_t(c0) * S, tmp);
#pragma unroll
  for (int v = 0; v < V; ++v)
#pragma unroll
    for (int s = 0; s < S; ++s) out[s][v] = tmp[v * S + s];
}

template <typename T, int V, int K, bool HAS_Z, bool NTL, bool NTS>
__global__ void __launch_bounds__(SIHC_EV_FWD_THREADS, SIHC_EV_MINW) k_event_fwd(const T* __restrict__ x, const T* __restrict__ dz,
                                                   const T* __restrict__ beta,
                                                   const T* __restrict__ alpha, T* __restrict__ xo,
                                                   T* __restrict__ zo, const int32_t* __restrict__ index,
                                                   Geo g, int tpb, int nslices) {
  constexpr int S = K * K;
  constexpr int U = SIHC_EV_UNROLL;  // tokens per lane per iteration
  const int BCG = blockDim.x, TL = blockDim.y;
  const int blk = logical_block<K == 4>();
  int slice, chunk;
  slice_chunk(blk, nslices, slice, chunk);
  const int c0 = (slice * BCG + threadIdx.x) * V;
  if (c0 >= g.C) return;
  float bw[S][V], aw[S][V];
  load_weights<T, V, K>(beta, c0, bw);
  if constexpr (HAS_Z) load_weights<T, V, K>(alpha, c0, aw);
  const int m_begin = chunk * tpb;
  const int m_end = min(m_begin + tpb, g.M);
  for (int m = m_begin + threadIdx.y; m < m_end; m += U * TL) {
    int64_t p0[U], zoff[U];
    bool ok[U];
    float d[U][V];
    float xv[U][S][V];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      ok[u] = m + u * TL < m_end;
      const int mu = ok[u] ? m + u * TL : m;  // tail: reload a valid token, store nothing
      p0[u] = cell_pixel0(mu, g, index);
      zoff[u] = int64_t(mu) * g.C + c0;
      load_vec<T, V, NTL>(dz + zoff[u], d[u]);
#pragma unroll
      for (int s = 0; s < S; ++s) load_vec<T, V, NTL>(x + slot_offset<K>(p0[u], s, g, c0), xv[u][s]);
    }
    load_fence();
#pragma unroll
    for (int u = 0; u < U; ++u) {
      float zacc[V];
#pragma unroll
      for (int v = 0; v < V; ++v) zacc[v] = 0.f;
#pragma unroll
      for (int s = 0; s < S; ++s)
#pragma unroll
        for (int v = 0; v < V; ++v) {
          xv[u][s][v] = round_as<T>(fmaf(bw[s][v], d[u][v], xv[u][s][v]));
          if constexpr (HAS_Z) zacc[v] = fmaf(aw[s][v], xv[u][s][v], zacc[v]);
        }
      if (ok[u]) {
#pragma unroll
        for (int s = 0; s < S; ++s) store_vec<T, V, NTS>(xo + slot_offset<K>(p0[u], s, g, c0), xv[u][s]);
        if constexpr (HAS_Z) store_vec<T, V, NTS>(zo + zoff[u], zacc);
      }
    }
  }
}

// ----------------------------------------------------------------------------------
// 16-slot bf16 per-event forward with 2-channel lanes: k_event_fwd's arithmetic (same
// bits), with the carrier rows and the weights kept as bf16 words and each slot widened,
// updated, rounded and stored in turn (k_event_fwd holds 2 x 16 x 2 fp32 carrier values
// and 64 fp32 weights per lane at 16 slots: 145 VGPRs, 3 waves per SIMD).
// ----------------------------------------------------------------------------------
template <bool HAS_Z, bool NTL, bool NTS>
__global__ void __launch_bounds__(SIHC_EV_FWD_THREADS, SIHC_EV_MINW) k_event_fwd16(const bf16_t* __restrict__ x,
                                                     const bf16_t* __restrict__ dz,
                                                     const bf16_t* __restrict__ beta,
                                                     const bf16_t* __restrict__ alpha, bf16_t* __restrict__ xo,
                                                     bf16_t* __restrict__ zo, const int32_t* __restrict__ index,
                                                     Geo g, int tpb, int nslices) {
  constexpr int K = 4, S = 16, V = 2;
  constexpr int U = SIHC_EV_UNROLL;  // tokens per lane per iteration
  const int BCG = blockDim.x, TL = blockDim.y;
  const int blk = logical_block<true>(), slice = blk % nslices, chunk = blk / nslices;
  const int c0 = (slice * BCG + threadIdx.x) * V;
  if (c0 >= g.C) return;
  uint32_t bw[16], aw[16];  // word v * 8 + p: channel c0 + v, slots 2p, 2p + 1
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const u32x4 r = reinterpret_cast<const u32x4*>(beta + int64_t(c0) * S)[q];
#pragma unroll
    for (int k = 0; k < 4; ++k) bw[4 * q + k] = r[k];
  }
  if constexpr (HAS_Z) {
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const u32x4 r = reinterpret_cast<const u32x4*>(alpha + int64_t(c0) * S)[q];
#pragma unroll
      for (int k = 0; k < 4; ++k) aw[4 * q + k] = r[k];
    }
  }
  auto wget = [](const uint32_t (&w)[16], int sl, int v) {
    const uint32_t u = w[v * 8 + (sl >> 1)];
    return __uint_as_float((sl & 1) ? (u & 0xffff0000u) : (u << 16));
  };
  const int64_t row_w = int64_t(g.GK) * (g.C >> 1);  // words per carrier row (C even here)
  const int pix_w = g.C >> 1;
  const uint32_t* xw = reinterpret_cast<const uint32_t*>(x);
  uint32_t* xow = reinterpret_cast<uint32_t*>(xo);
  const int m_begin = chunk * tpb;
  const int m_end = min(m_begin + tpb, g.M);
  for (int m = m_begin + threadIdx.y; m < m_end; m += U * TL) {
    int64_t b0[U], zw[U];
    bool ok[U];
    uint32_t dr[U], xr[U][S];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      ok[u] = m + u * TL < m_end;
      const int mu = ok[u] ? m + u * TL : m;  // tail: reload a valid token, store nothing
      b0[u] = (cell_pixel0(mu, g, index) * g.C + c0) >> 1;
      zw[u] = (int64_t(mu) * g.C + c0) >> 1;
      dr[u] = ld<NTL>(reinterpret_cast<const uint32_t*>(dz) + zw[u]);
#pragma unroll
      for (int uy = 0; uy < K; ++uy)
#pragma unroll
        for (int ux = 0; ux < K; ++ux) xr[u][uy * K + ux] = ld<NTL>(xw + b0[u] + uy * row_w + ux * pix_w);
    }
    load_fence();
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const float d[V] = {__uint_as_float(dr[u] << 16), __uint_as_float(dr[u] & 0xffff0000u)};
      float zacc[V] = {0.f, 0.f};
#pragma unroll
      for (int sl = 0; sl < S; ++sl) {
        float xv[V] = {__uint_as_float(xr[u][sl] << 16), __uint_as_float(xr[u][sl] & 0xffff0000u)};
#pragma unroll
        for (int v = 0; v < V; ++v) {
          xv[v] = round_as<bf16_t>(fmaf(wget(bw, sl, v), d[v], xv[v]));
          if constexpr (HAS_Z) zacc[v] = fmaf(wget(aw, sl, v), xv[v], zacc[v]);
        }
        if (ok[u])
          store_vec<bf16_t, V, NTS>(reinterpret_cast<bf16_t*>(xow + b0[u] + (sl / K) * row_w + (sl % K) * pix_w), xv);
      }
      if constexpr (HAS_Z) {
        if (ok[u]) store_vec<bf16_t, V, NTS>(zo + 2 * zw[u], zacc);
      }
    }
  }
}

// ----------------------------------------------------------------------------------
// 4-slot per-event forward over whole channel rows: block (C / V, TR) holds TR tokens,
// each thread one 16-byte lane (V channels) of one token, so a wave's loads and stores
// are whole contiguous runs of a carrier pixel row (2 x C elements per slot pair) and of
// the dz / z_out rows. k_event_fwd's arithmetic per element (same bits); one-shot, no
// loop: token blockIdx.x * TR + threadIdx.y.
// ----------------------------------------------------------------------------------
template <typename T, int V, bool HAS_Z, bool NTL, bool NTS>
__global__ void __launch_bounds__(1024) k_event_fwd_rows(const T* __restrict__ x, const T* __restrict__ dz,
                                                         const T* __restrict__ beta, const T* __restrict__ alpha,
                                                         T* __restrict__ xo, T* __restrict__ zo,
                                                         const int32_t* __restrict__ index, Geo g) {
  constexpr int K = 2, S = 4;
  const int m = int(blockIdx.x) * int(blockDim.y) + int(threadIdx.y);
  const int c0 = int(threadIdx.x) * V;
  if (m >= g.M) return;
  float bw[S][V], aw[S][V];
  load_weights<T, V, K>(beta, c0, bw);
  if constexpr (HAS_Z) load_weights<T, V, K>(alpha, c0, aw);
  // The weights (L2-resident, shared by the block's rows) arrive before any carrier load
  // is issued: left to the scheduler, the carrier loads go out between the weight loads
  // and the forward ran 11% slower (271 against 243 us per event at batch 256, C 1152).
  __builtin_amdgcn_s_waitcnt(0);
  __builtin_amdgcn_sched_barrier(0);
  const int64_t p0 = cell_pixel0(m, g, index);
  const int64_t zoff = int64_t(m) * g.C + c0;
  float d[V], xv[S][V];
  load_vec<T, V, NTL>(dz + zoff, d);
#pragma unroll
  for (int s = 0; s < S; ++s) load_vec<T, V, NTL>(x + slot_offset<K>(p0, s, g, c0), xv[s]);
  load_fence();
  float zacc[V];
#pragma unroll
  for (int v = 0; v < V; ++v) zacc[v] = 0.f;
#pragma unroll
  for (int s = 0; s < S; ++s)
#pragma unroll
    for (int v = 0; v < V; ++v) {
      xv[s][v] = round_as<T>(fmaf(bw[s][v], d[v], xv[s][v]));
      if constexpr (HAS_Z) zacc[v] = fmaf(aw[s][v], xv[s][v], zacc[v]);
    }
#pragma unroll
  for (int s = 0; s < S; ++s) store_vec<T, V, NTS>(xo + slot_offset<K>(p0, s, g, c0), xv[s]);
  if constexpr (HAS_Z) store_vec<T, V, NTS>(zo + zoff, zacc);
}

// ----------------------------------------------------------------------------------
// per-event fused backward (see sihc_event_backward in sihc_hip.h)
//   HAS_H: grad_x_out given      HAS_G: read part (grad_z_out, x_out, alpha_next)
//   HAS_W: write part (dz, beta)  STORE_T: store t as grad_x (else the caller aliases)
// part[chunk][0][s][c] = partial grad_beta, part[chunk][1][s][c] = partial grad_alpha_next
// ----------------------------------------------------------------------------------
template <typename T, int V, int K, bool HAS_H, bool HAS_G, bool HAS_W, bool STORE_T, bool NTL, bool NTS>
__global__ void __launch_bounds__(256, SIHC_EV_MINW) k_event_bwd(const T* __restrict__ gxo, const T* __restrict__ gzo,
                                                   const T* __restrict__ xo, const T* __restrict__ dz,
                                                   const T* __restrict__ beta,
                                                   const T* __restrict__ alpha, T* __restrict__ gx,
                                                   T* __restrict__ gdz, float* __restrict__ part,
                                                   const int32_t* __restrict__ index, Geo g, int gs, int nchunks,
                                                   int nslices, EvCarry carry) {
  constexpr int S = K * K;
  constexpr int U = SIHC_EV_UNROLL;  // tokens per lane per iteration
  extern __shared__ float red[];  // TL x BCG x S x V floats (>= FINALIZE_LDS(4): 256 x 4)
  if (run_carry<T>(carry, S, g.C, red)) return;
  const int BCG = blockDim.x, TL = blockDim.y;
  const int BC = BCG * V;
  const int blk = logical_block_of<K == 4>(carry.nmain);
  int slice, chunk;
  slice_chunk(blk, nslices, slice, chunk);
  const int c0 = slice * BC + threadIdx.x * V;
  float db[S][V], da[S][V];
#pragma unroll
  for (int s = 0; s < S; ++s)
#pragma unroll
    for (int v = 0; v < V; ++v) {
      db[s][v] = 0.f;
      da[s][v] = 0.f;
    }
  if (c0 < g.C) {
    float bw[S][V], aw[S][V];
    if constexpr (HAS_W) load_weights<T, V, K>(beta, c0, bw);
    if constexpr (HAS_G) load_weights<T, V, K>(alpha, c0, aw);
    // weights in registers before the first carrier load goes out (0.6% at batch 256)
    __builtin_amdgcn_s_waitcnt(0);
    __builtin_amdgcn_sched_barrier(0);
    // The chunk's tokens: groups of gs tokens (a multiple of U * TL), group `chunk`
    // and every nchunks-th one after it, so the blocks resident at one time work on
    // neighbouring groups and the device streams through a narrow window of each array.
    const int64_t M = g.M;
    // one token's compute and stores (tail tokens: zero every loaded value so it adds
    // exactly nothing -- a zero factor alone would turn an Inf in the repeated token
    // into NaN -- and store nothing)
    auto consume = [&](float (&gz)[V], float (&d)[V], float (&t)[S][V], float (&xv)[S][V], int64_t p0,
                       int64_t zoff, bool ok) {
      if (!ok) {
#pragma unroll
        for (int v = 0; v < V; ++v) {
          gz[v] = 0.f;
          d[v] = 0.f;
        }
#pragma unroll
        for (int ss = 0; ss < S; ++ss)
#pragma unroll
          for (int v = 0; v < V; ++v) {
            t[ss][v] = 0.f;
            xv[ss][v] = 0.f;
          }
      }
      float gd[V];
#pragma unroll
      for (int v = 0; v < V; ++v) gd[v] = 0.f;
#pragma unroll
      for (int s = 0; s < S; ++s)
#pragma unroll
        for (int v = 0; v < V; ++v) {
          if constexpr (HAS_G) {
            da[s][v] = fmaf(xv[s][v], gz[v], da[s][v]);
            t[s][v] = fmaf(aw[s][v], gz[v], t[s][v]);
          }
          if constexpr (HAS_W) {
            gd[v] = fmaf(bw[s][v], t[s][v], gd[v]);
            db[s][v] = fmaf(d[v], t[s][v], db[s][v]);
          }
        }
      if (ok) {
        if constexpr (STORE_T) {
#pragma unroll
          for (int s = 0; s < S; ++s) store_vec<T, V, NTS>(gx + slot_offset<K>(p0, s, g, c0), t[s]);
        }
        if constexpr (HAS_W) store_vec<T, V, NTS>(gdz + zoff, gd);
      }
    };
    // With a state index, the cells of an iteration's tokens are loaded one iteration
    // ahead, so its carrier addresses do not wait on an index load (an unhidden dependent
    // load per iteration cost the indexed backward 8% at 2 waves per SIMD).
    const int64_t gstride = int64_t(nchunks) * gs;
    uint32_t cell_next[U];
#pragma unroll
    for (int u = 0; u < U; ++u) cell_next[u] = 0u;
    auto fetch_cells = [&](int64_t mi, int64_t m_end) {
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int64_t mt = mi + threadIdx.y + u * TL;
        cell_next[u] = index_cell(int(mt < m_end ? mt : mi), g, index);
      }
    };
    if (index && int64_t(chunk) * gs < M) fetch_cells(int64_t(chunk) * gs, min(int64_t(chunk) * gs + gs, M));
    for (int64_t m0 = int64_t(chunk) * gs; m0 < M; m0 += gstride) {
      const int64_t m_end = min(m0 + gs, M);
      for (int64_t mi = m0; mi < m_end; mi += U * TL) {
        int64_t p0[U], zoff[U];
        bool ok[U];
        float gz[U][V], d[U][V], t[U][S][V], xv[U][S][V];
        uint32_t cell[U];
#pragma unroll
        for (int u = 0; u < U; ++u) cell[u] = cell_next[u];
        if (index) {  // the next iteration: this group's next rows, or the chunk's next group
          const bool same = mi + U * TL < m_end;
          const int64_t mn = same ? mi + U * TL : m0 + gstride;
          if (mn < M) fetch_cells(mn, same ? m_end : min(mn + gs, M));
        }
        // loads (tail tokens reload the iteration's first token, which is valid)
#pragma unroll
        for (int u = 0; u < U; ++u) {
          const int64_t mt = mi + threadIdx.y + u * TL;
          ok[u] = mt < m_end;
          const int mu = int(ok[u] ? mt : mi);
          p0[u] = cell_pixel0_at(mu, cell[u], index != nullptr, g);
          zoff[u] = int64_t(mu) * g.C + c0;
          if constexpr (HAS_G) load_vec<T, V, NTL>(gzo + zoff[u], gz[u]);
          if constexpr (HAS_W) load_vec<T, V, NTL>(dz + zoff[u], d[u]);
#pragma unroll
          for (int s = 0; s < S; ++s) {
            const int64_t off = slot_offset<K>(p0[u], s, g, c0);
            if constexpr (HAS_H) {
              load_vec<T, V, NTL>(gxo + off, t[u][s]);
            } else {
#pragma unroll
              for (int v = 0; v < V; ++v) t[u][s][v] = 0.f;
            }
            if constexpr (HAS_G) load_vec<T, V, NTL>(xo + off, xv[u][s]);
          }
        }
        load_fence();
#pragma unroll
        for (int u = 0; u < U; ++u) consume(gz[u], d[u], t[u], xv[u], p0[u], zoff[u], ok[u]);
      }
    }
  }
  // Block reduction of the [S][V] accumulators; partial rows are [2][S][C].
  float* prow = part + int64_t(chunk) * 2 * S * g.C;
  const int cs = slice * BC;
#pragma unroll
  for (int w = 0; w < 2; ++w) {
    if ((w == 0 && !HAS_W) || (w == 1 && !HAS_G)) continue;
    float flat[S * V];
#pragma unroll
    for (int s = 0; s < S; ++s)
#pragma unroll
      for (int v = 0; v < V; ++v) flat[s * V + v] = w == 0 ? db[s][v] : da[s][v];
    // lane-major layout in `red`: [ty][lane][s][v]; remap to [s][c] on emit.
    block_reduce_rows<S * V>(flat, red, [&](int i, float sum) {
      const int lane = i / (S * V);
      const int r = i - lane * S * V;
      const int s = r / V;
      const int v = r - s * V;
      const int c = cs + lane * V + v;
      if (c < g.C) prow[(int64_t(w) * S + s) * g.C + c] = sum;
    });
  }
}

// ----------------------------------------------------------------------------------
// 16-slot bf16 per-event backward with 2-channel lanes: k_event_bwd's arithmetic in the
// same order (so the same bits), one token per lane per iteration, and the weights and
// loaded rows kept as bf16 words, widened where they are used. A lane's 16-slot cell
// otherwise holds 68 loaded values per token beside 64 accumulators and 64 weights:
// k_event_bwd at 16 slots needs 334 VGPRs with two tokens per lane (one wave per SIMD).
// A lane reads its channel pair's 16-slot weight rows ([C][16] bf16: 8 words per channel,
// word p = slots 2p, 2p + 1) with four 16-byte loads. The token order per thread equals
// k_event_bwd's (tokens ty, ty + TL, ... of each group), so the partial rows are the same.
// ----------------------------------------------------------------------------------
template <bool HAS_H, bool HAS_G, bool HAS_W, bool STORE_T, bool NTL, bool NTS>
__global__ void __launch_bounds__(256, SIHC_EV16_MINW) k_event_bwd16(const bf16_t* __restrict__ gxo,
                                                     const bf16_t* __restrict__ gzo,
                                                     const bf16_t* __restrict__ xo, const bf16_t* __restrict__ dz,
                                                     const bf16_t* __restrict__ beta,
                                                     const bf16_t* __restrict__ alpha, bf16_t* __restrict__ gx,
                                                     bf16_t* __restrict__ gdz, float* __restrict__ part,
                                                     const int32_t* __restrict__ index, Geo g, int gs, int nchunks,
                                                     int nslices, EvCarry carry) {
  constexpr int K = 4, S = 16, V = 2;
  extern __shared__ float red[];  // TL x BCG x S x V floats (>= FINALIZE_LDS(4))
  if (run_carry<bf16_t>(carry, S, g.C, red)) return;
  const int BCG = blockDim.x, TL = blockDim.y;
  const int BC = BCG * V;
  const int blk = logical_block_of<true>(carry.nmain), slice = blk % nslices, chunk = blk / nslices;
  const int c0 = slice * BC + threadIdx.x * V;
  float db[S][V], da[S][V];
#pragma unroll
  for (int sl = 0; sl < S; ++sl)
#pragma unroll
    for (int v = 0; v < V; ++v) db[sl][v] = da[sl][v] = 0.f;
  // word w of a weight row pair: channel w / 8, slots 2 (w % 8), 2 (w % 8) + 1
  auto wget = [](const uint32_t (&w)[16], int sl, int v) {
    const uint32_t u = w[v * 8 + (sl >> 1)];
    return __uint_as_float((sl & 1) ? (u & 0xffff0000u) : (u << 16));
  };
  auto lo_f = [](uint32_t u) { return __uint_as_float(u << 16); };
  auto hi_f = [](uint32_t u) { return __uint_as_float(u & 0xffff0000u); };
  if (c0 < g.C) {
    uint32_t bw[16], aw[16];
    if constexpr (HAS_W) {
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const u32x4 r = reinterpret_cast<const u32x4*>(beta + int64_t(c0) * S)[q];
#pragma unroll
        for (int k = 0; k < 4; ++k) bw[4 * q + k] = r[k];
      }
    }
    if constexpr (HAS_G) {
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const u32x4 r = reinterpret_cast<const u32x4*>(alpha + int64_t(c0) * S)[q];
#pragma unroll
        for (int k = 0; k < 4; ++k) aw[4 * q + k] = r[k];
      }
    }
    const int64_t M = g.M;
    const int64_t row_w = int64_t(g.GK) * (g.C >> 1);  // words per carrier row (C even here)
    const int pix_w = g.C >> 1;
    const uint32_t* gxw = reinterpret_cast<const uint32_t*>(gxo);
    const uint32_t* xow = reinterpret_cast<const uint32_t*>(xo);
    uint32_t* gxo_w = reinterpret_cast<uint32_t*>(gx);
    for (int64_t m0 = int64_t(chunk) * gs; m0 < M; m0 += int64_t(nchunks) * gs) {
      const int64_t m_end = min(m0 + gs, M);
      for (int64_t mi = m0; mi < m_end; mi += TL) {
        const int64_t mt = mi + threadIdx.y;
        const bool ok = mt < m_end;
        const int mu = int(ok ? mt : mi);  // tail: reload the iteration's first token
        const int64_t b0 = (cell_pixel0(mu, g, index) * g.C + c0) >> 1;
        const int64_t zw = (int64_t(mu) * g.C + c0) >> 1;
        uint32_t gzr = 0u, dr = 0u, tr[S], xr[S];
        if constexpr (HAS_G) gzr = ld<NTL>(reinterpret_cast<const uint32_t*>(gzo) + zw);
        if constexpr (HAS_W) dr = ld<NTL>(reinterpret_cast<const uint32_t*>(dz) + zw);
#pragma unroll
        for (int uy = 0; uy < K; ++uy)
#pragma unroll
          for (int ux = 0; ux < K; ++ux) {
            const int64_t o = b0 + uy * row_w + ux * pix_w;
            tr[uy * K + ux] = HAS_H ? ld<NTL>(gxw + o) : 0u;
            if constexpr (HAS_G) xr[uy * K + ux] = ld<NTL>(xow + o);
          }
        load_fence();
        // a tail token adds exactly nothing: every loaded value is zeroed (a zero factor
        // alone would turn an Inf in the repeated token into NaN), and nothing is stored
        if (!ok) {
          gzr = dr = 0u;
#pragma unroll
          for (int sl = 0; sl < S; ++sl) tr[sl] = xr[sl] = 0u;
        }
        const float gz[V] = {lo_f(gzr), hi_f(gzr)}, d[V] = {lo_f(dr), hi_f(dr)};
        float gd[V] = {0.f, 0.f};
#pragma unroll
        for (int sl = 0; sl < S; ++sl) {
          float t[V] = {lo_f(tr[sl]), hi_f(tr[sl])};
#pragma unroll
          for (int v = 0; v < V; ++v) {
            if constexpr (HAS_G) {
              const float xv = v ? hi_f(xr[sl]) : lo_f(xr[sl]);
              da[sl][v] = fmaf(xv, gz[v], da[sl][v]);
              t[v] = fmaf(wget(aw, sl, v), gz[v], t[v]);
            }
            if constexpr (HAS_W) {
              gd[v] = fmaf(wget(bw, sl, v), t[v], gd[v]);
              db[sl][v] = fmaf(d[v], t[v], db[sl][v]);
            }
          }
          if constexpr (STORE_T) {
            if (ok) {
              const int uy = sl / K, ux = sl % K;
              store_vec<bf16_t, V, NTS>(reinterpret_cast<bf16_t*>(gxo_w + b0 + uy * row_w + ux * pix_w), t);
            }
          }
        }
        if constexpr (HAS_W) {
          if (ok) store_vec<bf16_t, V, NTS>(gdz + (int64_t(mu) * g.C + c0), gd);
        }
      }
    }
  }
  // Block reduction of the [S][V] accumulators, as k_event_bwd: partial rows [2][S][C].
  float* prow = part + int64_t(chunk) * 2 * S * g.C;
  const int cs = slice * BC;
#pragma unroll
  for (int w = 0; w < 2; ++w) {
    if ((w == 0 && !HAS_W) || (w == 1 && !HAS_G)) continue;
    float flat[S * V];
#pragma unroll
    for (int sl = 0; sl < S; ++sl)
#pragma unroll
      for (int v = 0; v < V; ++v) flat[sl * V + v] = w == 0 ? db[sl][v] : da[sl][v];
    block_reduce_rows<S * V>(flat, red, [&](int i, float sum) {
      const int lane = i / (S * V);
      const int r = i - lane * S * V;
      const int sl = r / V;
      const int v = r - sl * V;
      const int c = cs + lane * V + v;
      if (c < g.C) prow[(int64_t(w) * S + sl) * g.C + c] = sum;
    });
  }
}

// ----------------------------------------------------------------------------------
// gather / scatter of whole cells (bit-exact copies of CH-byte chunks)
// cells[m][s][:] <-> x[pixel(index(m), s)][:]
// ----------------------------------------------------------------------------------
template <typename R, int K, bool GATHER>
__global__ void __launch_bounds__(256) k_cells(const R* __restrict__ src, R* __restrict__ dst,
                                               const int32_t* __restrict__ index, Geo g, int row_chunks) {
  constexpr int S = K * K;
  const int64_t row = int64_t(blockIdx.x) * blockDim.y + threadIdx.y;  // m*S + s
  if (row >= int64_t(g.M) * S) return;
  const int m = int(row / S);
  const int s = int(row - int64_t(m) * S);
  const int64_t pix = cell_pixel0(m, g, index) + int64_t(s / K) * g.GK + (s % K);
  const int64_t xrow = pix * row_chunks;
  const int64_t crow = row * row_chunks;
  for (int i = threadIdx.x; i < row_chunks; i += blockDim.x) {
    constexpr bool NTL = (SIHC_CELLS_NTM & 1) != 0, NTS = (SIHC_CELLS_NTM & 2) != 0;
    if constexpr (GATHER) {
      st<NTS>(dst + crow + i, ld<NTL>(src + xrow + i));
    } else {
      st<NTS>(dst + xrow + i, ld<NTL>(src + crow + i));
    }
  }
}

// ----------------------------------------------------------------------------------
// adjoint of the gather for any in-range index (repeats allowed): the cell n of batch b
// receives the fp32 sum, over the tokens t of row b with index[b,t] == n in ascending t,
// of cells[b,t]; cells that no token selects receive zeros. One block per destination
// cell: the batch row of the index is staged in LDS and every thread scans it in order
// (a block-uniform test, so no divergence). No atomics: deterministic. The sum starts
// from -0.0 (the identity of fp32 addition), so a cell with one contributor receives its
// value bit for bit, as the scatter copy would. Out-of-range indices (only possible when
// the host-side validation is skipped) are clamped as the gather clamps them (to the last
// cell), so the adjoint returns every gathered row's gradient to the cell it was read
// from. Each block scans its batch row's GG indices per output vector: O(GG^2) work per
// batch row, negligible at the benchmark grid (GG = 256) and bounded by GG <= 16384.
// ----------------------------------------------------------------------------------
template <typename T, int V, int K>
__global__ void __launch_bounds__(256) k_cells_add(const T* __restrict__ cells, T* __restrict__ x,
                                                   const int32_t* __restrict__ index, Geo g) {
  constexpr int S = K * K;
  extern __shared__ int32_t sidx[];
  const int64_t m = blockIdx.x;  // destination cell b * GG + n
  const int b = int(m / g.GG), n = int(m - int64_t(b) * g.GG);
  for (int t = threadIdx.x; t < g.GG; t += blockDim.x)
    sidx[t] = int32_t(min(uint32_t(index[int64_t(b) * g.GG + t]), uint32_t(g.GG) - 1u));
  __syncthreads();
  const int64_t pix0 = cell_pixel0(int(m), g, nullptr);
  const int nvec = S * g.C / V;
  for (int i = threadIdx.x; i < nvec; i += blockDim.x) {
    const int e = i * V;
    const int s = e / g.C;
    const int c = e - s * g.C;
    float acc[V];
#pragma unroll
    for (int v = 0; v < V; ++v) acc[v] = -0.f;
    int hits = 0;
    for (int t = 0; t < g.GG; ++t) {
      if (sidx[t] != n) continue;
      float val[V];
      load_vec<T, V>(cells + ((int64_t(b) * g.GG + t) * S + s) * g.C + c, val);
#pragma unroll
      for (int v = 0; v < V; ++v) acc[v] += val[v];
      ++hits;
    }
    if (hits == 0) {
#pragma unroll
      for (int v = 0; v < V; ++v) acc[v] = 0.f;
    }
    store_vec<T, V>(x + slot_offset<K>(pix0, s, g, c), acc);
  }
}

__global__ void __launch_bounds__(256) k_copy16(const u32x4* __restrict__ src, u32x4* __restrict__ dst, int64_t n) {
  const int64_t stride = int64_t(gridDim.x) * blockDim.x;
  constexpr bool NTL = (SIHC_COPY_NTM & 1) != 0, NTS = (SIHC_COPY_NTM & 2) != 0;
  for (int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += stride)
    st<NTS>(dst + i, ld<NTL>(src + i));
}

// Streaming calibration, in the access pattern that measured fastest on this memory
// system for mixed traffic: one-shot blocks (each block moves one 4 KB unit of every
// array and exits, so the device sweeps memory in block order), 16-byte vectors,
// non-temporal loads and stores, all loads of a thread issued before its first store.
// The first R4 sources and the first W4 destinations are carrier-shaped (4 vectors per
// unit and thread: the 4 slots of a 4-slot cell), the others workspace-shaped (1). Each
// output is the XOR of the inputs (an index pattern when there are none), so no load
// can be skipped.
template <int NR, int NW, int R4, int W4>
__global__ void __launch_bounds__(256) k_stream(PtrPack src, PtrPack dst, int64_t units) {
  const int64_t u = blockIdx.x;
  if (u >= units) return;
  const int t = int(threadIdx.x);
  constexpr int NV = 4 * R4 + (NR - R4) > 0 ? 4 * R4 + (NR - R4) : 1;
  u32x4 v[NV];
  int k = 0;
#pragma unroll
  for (int r = 0; r < NR; ++r) {
    const u32x4* a = static_cast<const u32x4*>(src.p[r]);
    if (r < R4) {
#pragma unroll
      for (int q = 0; q < 4; ++q) v[k++] = ld<true>(a + u * 1024 + q * 256 + t);
    } else {
      v[k++] = ld<true>(a + u * 256 + t);
    }
  }
  load_fence();
  u32x4 acc = {uint32_t(u), uint32_t(t), 0u, 0u};
#pragma unroll
  for (int i = 0; i < 4 * R4 + (NR - R4); ++i) acc ^= v[i];
#pragma unroll
  for (int w = 0; w < NW; ++w) {
    u32x4* b = static_cast<u32x4*>(const_cast<void*>(dst.p[w]));
    if (w < W4) {
#pragma unroll
      for (int q = 0; q < 4; ++q) st<true>(b + u * 1024 + q * 256 + t, acc ^ uint32_t(w * 4 + q));
    } else {
      st<true>(b + u * 256 + t, acc ^ uint32_t(w));
    }
  }
}

// The same one-shot stream over any op's own array mix: sources and destinations in any
// number up to 32, the first ncs sources and the first ncd destinations carrier-shaped
// (`slots` 4 KB units of each per block: a cell's slots), the others workspace-shaped (one
// unit). Loads go out eight at a time before they are combined. Destination w gets the
// XOR of every source vector of the thread ^ (w * slots + q) for slot q of a carrier-shaped
// one, ^ w otherwise. With no destination (a read-only mix, as a weight gradient's) each
// wave stores the XOR of its lanes' values to sink[u * 4 + wave], 1/256 of the bytes read.
__global__ void __launch_bounds__(256) k_stream_mix(PtrPack src, int nsrc, int ncs, PtrPack dst, int ndst, int ncd,
                                                    int slots, int64_t units, u32x4* __restrict__ sink) {
  const int64_t u = blockIdx.x;
  if (u >= units) return;
  const int t = int(threadIdx.x);
  u32x4 acc = {uint32_t(u), uint32_t(t), 0u, 0u};
  const int ncv = ncs * slots;           // carrier source vectors
  const int nv = ncv + (nsrc - ncs);     // all source vectors of the thread
  for (int i0 = 0; i0 < nv; i0 += 8) {   // i0 is uniform: the source and slot are scalars
    u32x4 v[8];
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const int i = min(i0 + k, nv - 1);  // past the end: the last vector again, not combined
      const bool car = i < ncv;
      const int r = car ? i / slots : ncs + (i - ncv);
      const int64_t off = car ? (u * slots + (i - (i / slots) * slots)) * 256 + t : u * 256 + t;
      v[k] = ld<true>(static_cast<const u32x4*>(src.p[r]) + off);
    }
    load_fence();
#pragma unroll
    for (int k = 0; k < 8; ++k)
      if (i0 + k < nv) acc ^= v[k];
  }
  for (int w = 0; w < ndst; ++w) {
    u32x4* b = static_cast<u32x4*>(const_cast<void*>(dst.p[w]));
    if (w < ncd) {
      for (int q = 0; q < slots; ++q) st<true>(b + (u * slots + q) * 256 + t, acc ^ uint32_t(w * slots + q));
    } else {
      st<true>(b + u * 256 + t, acc ^ uint32_t(w));
    }
  }
  if (ndst == 0) {
#pragma unroll
    for (int m = 1; m < 64; m <<= 1)
#pragma unroll
      for (int k = 0; k < 4; ++k) acc[k] ^= uint32_t(__shfl_xor(int(acc[k]), m, 64));
    if (t % 64 == 0) sink[u * 4 + t / 64] = acc;
  }
}

// Vector-ALU calibration: CH independent accumulation chains per thread, 4 steps of each
// per iteration, one sum per thread stored so no chain can be dropped. FORM 0: fp32 fma
// with register operands (v_fma_f32, the form the kernels' products take); FORM 1: the
// multiplier and addend as literal constants (v_fmamk_f32); FORM 2: v_dot2c_f32_bf16 of
// two bf16 pairs (2 lane-FMAs a step); FORM 3: the chain value as the addend, a = fma(mul,
// add, a) (v_fmac_f32, the form of the kernels' accumulations). No packed fp32: the
// library's flags keep it out.
template <int CH, int FORM>
__global__ void __launch_bounds__(256) k_fma_chains(float* __restrict__ out, int iters, float mul, float add,
                                                    uint32_t pa, uint32_t pb) {
  float a[CH];
#pragma unroll
  for (int k = 0; k < CH; ++k) a[k] = float(threadIdx.x) * 1e-3f + float(k);
  for (int i = 0; i < iters; ++i) {
#pragma unroll
    for (int u = 0; u < 4; ++u)
#pragma unroll
      for (int k = 0; k < CH; ++k) {
        if constexpr (FORM == 0) a[k] = fmaf(a[k], mul, add);
        else if constexpr (FORM == 1) a[k] = fmaf(a[k], 1.0000001f, 1e-7f);
        else if constexpr (FORM == 2) a[k] = dot2(pa, pb, a[k]);
        else a[k] = fmaf(mul, add, a[k]);
      }
  }
  float s = 0.f;
#pragma unroll
  for (int k = 0; k < CH; ++k) s += a[k];
  out[int64_t(blockIdx.x) * 256 + threadIdx.x] = s;
}

__global__ void k_copy1(const uint8_t* __restrict__ src, uint8_t* __restrict__ dst, int64_t n) {
  const int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i < n) dst[i] = src[i];
}

// ==================================================================================
// host side
// ==================================================================================
thread_local std::string g_last_error;

int fail(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_last_error = buf;
  return code;
}

int check_launch(const char* what) {
  hipError_t err = hipGetLastError();
  if (err != hipSuccess) return fail(SIHC_ERR_HIP, "%s: launch failed: %s", what, hipGetErrorString(err));
  return SIHC_OK;
}

int elem_size(int dtype) { return dtype == SIHC_DTYPE_F32 ? 4 : 2; }
bool valid_dtype(int dtype) { return dtype == SIHC_DTYPE_F32 || dtype == SIHC_DTYPE_BF16; }

bool aligned(const void* p, int bytes) { return (reinterpret_cast<uintptr_t>(p) % uintptr_t(bytes)) == 0; }

// Largest V in {8, 4, 2, 1} with V <= max_v and V*elem <= 16 such that C % V == 0 and
// every pointer is aligned to V*elem bytes. `elem` is the widest element size.
int pick_vec(int C, int elem, int max_v, const void* const* ptrs, int n) {
  for (int v : {8, 4, 2}) {
    if (v > max_v || v * elem > 16 || C % v) continue;
    bool ok = true;
    for (int i = 0; i < n && ok; ++i) ok = ptrs[i] == nullptr || aligned(ptrs[i], v * elem);
    if (ok) return v;
  }
  return 1;
}

struct Shape2D {
  int bcg, tl, slices;
};

// Channel groups per block: `bcg0` lanes of V channels, fewer when C is small or the
// weight slice would not fit `lds_cap` bytes.
Shape2D shape_for(int C, int V, int bcg0, int lds_per_channel, int lds_cap = 64 * 1024) {
  const int CG = (C + V - 1) / V;
  int bcg = bcg0;
  while (bcg > 1 && bcg / 2 >= CG) bcg /= 2;
  while (bcg > 1 && int64_t(lds_per_channel) * bcg * V > lds_cap) bcg /= 2;
  Shape2D sh;
  sh.bcg = bcg;
  sh.tl = 256 / bcg;
  sh.slices = (CG + bcg - 1) / bcg;
  return sh;
}

// Tokens per lane of k_read / k_write. Each block first stages its E x S weight slice
// into LDS; with 16-slot cells that staging is large enough that blocks must cover more
// tokens as E grows (measured at batch 256, D 1152: E = 24 read 1872 -> 1624 us with
// 64 tokens per lane, while E = 1 is fastest with 8).
int rw_tokens_per_lane(int cell, int events, bool read = false, bool dot2_read = false) {
  // 4-slot reads: 32-token blocks (64 with one event) stream through a narrower window
  // than 128-token ones (E = 2..16: 6-7% faster)
  // 4-slot writes: 4 tokens per lane from 4 events (XL shape: E = 8 426 -> 417 us, E = 16
  // 655 -> 647, E = 24 889 -> 883; fewer events measured the same as with 8)
  if (cell == 2) return read ? (events == 1 ? 4 : 2) : (events >= 4 ? 4 : SIHC_RW_TPT);
  // 16-slot bf16 reads on k_read_d2 (packed weights, cheap to stage): short blocks past 12
  // events (XL shape: E = 16 957 -> 929 us with 8 tokens, E = 24 1251 -> 1206 us with 16,
  // E = 32 2210 -> 2078; 3-12 events do not care)
  if (dot2_read && events > 12) return events <= 16 ? 8 : 16;
  // 16 slots: the weight slice staged per block grows with E, so blocks grow too; with
  // hinted loads and stores reads with 3-12 events and writes with 9-12 gain from twice
  // the tokens again (read E = 8: 794 -> 745 us), 1-2 and 13+ events do not
  if (read && events >= 3 && events <= 12) return events <= 4 ? 16 : 32;
  if (!read && events > 8 && events <= 12) return 32;
  return events <= 4 ? SIHC_RW_TPT : events <= 16 ? 16 : 64;
}

int chunk_count(int64_t M, int tokens_per_chunk, int max_chunks) {
  int64_t n = (M + tokens_per_chunk - 1) / tokens_per_chunk;
  if (n < 1) n = 1;
  if (n > max_chunks) n = max_chunks;
  return int(n);
}
// Token chunks of the reductions: functions of sizes only, so that the workspace
// size queries and the launches agree.
// Block shape of the weight-gradient reduction: `bcg` channel-group lanes x `events`
// event lanes (<= 256 threads), `slices` blocks across the channels.
void wgrad_block(int C, int V, int events, int* bcg_out, int* slices_out) {
  const int CG = (C + V - 1) / V;
  int bcg = SIHC_WG_BCG;
  while (bcg > 1 && bcg * events > 256) bcg /= 2;
  while (bcg > 1 && bcg / 2 >= CG) bcg /= 2;
  *bcg_out = bcg;
  *slices_out = (CG + bcg - 1) / bcg;
}

// Token chunks (one partial row set each) of the weight-gradient reduction: one per
// SIHC_WG_CHUNK tokens up to 128, raised until the grid holds about 16 waves per CU
// (few events give small blocks), with at least 32 tokens per chunk. A function of the
// sizes only (the block shape is taken at the widest vector), so the workspace size is
// known before the pointers are.
int wgrad_chunks(int64_t M, int events, int C, int cell = 2) {
  int bcg, slices;
  wgrad_block(C, 8, std::max(events, 1), &bcg, &slices);
  const int64_t waves_per_chunk = int64_t(slices) * ((bcg * std::max(events, 1) + 63) / 64);
  const int64_t want = (4096 + waves_per_chunk - 1) / waves_per_chunk;
  const int base = chunk_count(M, cell == 4 ? SIHC_WG_CHUNK_K4 : SIHC_WG_CHUNK, 128);
  const int64_t cap = std::max<int64_t>(1, std::min<int64_t>(M / 32, 2048));
  return int(std::max<int64_t>(base, std::min(want, cap)));
}
// Reduction chunks of the per-event backward: 4-slot cells one per SIHC_EV_CHUNK tokens up
// to SIHC_EV_MAXCHUNKS; 16-slot cells, whose partial rows are 4x larger per chunk, one per
// SIHC_EV_CHUNK_K4 tokens up to SIHC_EV_MAXCHUNKS_K4. At the benchmark shape (65,536 tokens,
// 4 slots) 1,024 chunks of 64 tokens: blocks of ~20 us whose ragged last round costs less
// than the 128-token chunks' (380 vs 383 us per event with the chained finalize).
int event_bwd_chunks(int64_t M, int cell) {
  return cell == 2 ? chunk_count(M, SIHC_EV_CHUNK, SIHC_EV_MAXCHUNKS)
                   : chunk_count(M, SIHC_EV_CHUNK_K4, SIHC_EV_MAXCHUNKS_K4);
}
// Token chunks of the fused triangular backward (which also stores the update
// gradients): one per SIHC_TRIB_CHUNK tokens up to 1024, at least the weight-gradient
// count. Shorter runs per block stream through a narrower window of each array (A = 3:
// 269 -> 234 us, A = 11: 731 -> 682 us at the XL shape); the read-only gradients keep
// their longer chunks, which shorter ones slow down (fewer tokens per partial row).
int trib_chunks(int64_t M, int events, int C) {
  return std::max(wgrad_chunks(M, events, C), chunk_count(M, SIHC_TRIB_CHUNK, 1024));
}

// Tokens per interleaved group of a reduction chunk (chunk c takes groups c, c + chunks,
// ...): `want` rounded up to a multiple of `step` (the tokens of one loop iteration or
// tile); want = 0 gives each chunk one contiguous run.
int group_tokens(int want, int64_t M, int chunks, int step) {
  const int64_t w = want > 0 ? want : (M + chunks - 1) / std::max(chunks, 1);
  return int((std::max<int64_t>(w, 1) + step - 1) / step * step);
}

// Compute units of the current device (cached per device; 0 if unknown).
int device_cus() {
  static std::atomic<int> cus[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 0;
  int n = cus[dev].load(std::memory_order_relaxed);
  if (n == 0 && hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess)
    cus[dev].store(n, std::memory_order_relaxed);
  return n;
}

// Blocks of `kernel` (at this block size and dynamic LDS) resident on the whole device
// at once; 0 if the runtime cannot tell. Cached per (kernel, block size, LDS).
int resident_blocks(const void* kernel, int threads, size_t lds) {
  struct Key {
    const void* k;
    int threads;
    size_t lds;
    bool operator<(const Key& o) const {
      return std::tie(k, threads, lds) < std::tie(o.k, o.threads, o.lds);
    }
  };
  static std::mutex mu;
  static std::map<Key, int> cache;
  const Key key{kernel, threads, lds};
  {
    std::lock_guard<std::mutex> lock(mu);
    auto it = cache.find(key);
    if (it != cache.end()) return it->second * device_cus();
  }
  int per_cu = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kernel, threads, lds) != hipSuccess) {
    (void)hipGetLastError();
    return 0;
  }
  std::lock_guard<std::mutex> lock(mu);
  cache[key] = per_cu;
  return per_cu * device_cus();
}

// Chunk count <= max_chunks for which slices x chunks blocks form a whole number of
// rounds of `resident` blocks, so no round runs part-empty (a grid of 4.5 rounds
// leaves half the device idle for its last tenth). max_chunks when unknown or when the
// grid is under one round.
int whole_rounds(int slices, int max_chunks, int resident) {
  if (resident <= 0) return max_chunks;
  const int64_t rounds = int64_t(slices) * max_chunks / resident;
  if (rounds < 1) return max_chunks;
  return int(std::max<int64_t>(1, rounds * resident / slices));
}

int check_geometry(const char* what, int64_t batch, int grid, int cell, int channels, Geo* g) {
  if (batch < 0 || grid <= 0 || channels <= 0) return fail(SIHC_ERR_INVALID, "%s: bad sizes", what);
  if (cell != 2 && cell != 4) return fail(SIHC_ERR_INVALID, "%s: cell must be 2 or 4 (4 or 16 slots)", what);
  const int64_t M = batch * int64_t(grid) * grid;
  const int64_t carrier = M * cell * cell * int64_t(channels);
  if (M >= SIHC_MAX_TOKENS || carrier >= (int64_t(1) << 47))
    return fail(SIHC_ERR_INVALID, "%s: tensor too large", what);
  g->M = int(M);
  g->GG = grid * grid;
  g->G = grid;
  g->K = cell;
  g->GK = grid * cell;
  g->C = channels;
  set_divisors(*g);
  return SIHC_OK;
}

int check_count(const char* what, int events) {
  if (events < 1 || events > SIHC_MAX_EVENTS)
    return fail(SIHC_ERR_INVALID, "%s: events must be in 1..%d, got %d", what, SIHC_MAX_EVENTS, events);
  return SIHC_OK;
}

int check_events(const char* what, int events, const void* const* ptrs) {
  if (events < 1 || events > SIHC_MAX_EVENTS)
    return fail(SIHC_ERR_INVALID, "%s: events must be in 1..%d, got %d", what, SIHC_MAX_EVENTS, events);
  if (!ptrs) return fail(SIHC_ERR_INVALID, "%s: null pointer array", what);
  for (int i = 0; i < events; ++i)
    if (!ptrs[i]) return fail(SIHC_ERR_INVALID, "%s: null tensor pointer %d", what, i);
  return SIHC_OK;
}

// Kernel-argument pointer pack; slots past n repeat the last pointer so that padded
// event groups always load valid memory (their weights are zero or their sums unused).
PtrPack pack(const void* const* ptrs, int n) {
  PtrPack p;
  for (int i = 0; i < SIHC_MAX_EVENTS; ++i) p.p[i] = ptrs[i < n ? i : n - 1];
  return p;
}

template <typename F>
int with_dtype(int dtype, F&& f) {
  if (dtype == SIHC_DTYPE_F32) return f(float{});
  return f(bf16_t{});
}
template <typename F>
int with_vec(int v, F&& f) {
  if (v == 8) return f(IC<8>{});
  if (v == 4) return f(IC<4>{});
  if (v == 2) return f(IC<2>{});
  return f(IC<1>{});
}
template <typename F>
int with_cell(int k, F&& f) {
  if (k == 2) return f(IC<2>{});
  return f(IC<4>{});
}
// Compile-time lane counts of the 16-slot read / write (0: runtime value). Measured: a
// known lane count saves the per-row LDS address adds at 16 slots (write E=24 3.6 -> 3.2
// ms); at 4 slots it raises register use and occupancy drops, so those stay runtime.
template <int K, typename F>
int with_bcg(int bcg, F&& f) {
  if constexpr (K == 4) {
    if (bcg == 32) return f(IC<32>{});
    if (bcg == 16) return f(IC<16>{});
  }
  return f(IC<0>{});
}

template <typename F>
int with_bool(bool b, F&& f) {
  if (b) return f(std::true_type{});
  return f(std::false_type{});
}

// Non-temporal hint mode of a stage kernel: bit 0 loads, bit 1 stores. A compile-time
// FORCED >= 0 instantiates that mode only.
template <int FORCED, typename F>
int with_hints(int mode, F&& f) {
  if constexpr (FORCED >= 0) {
    (void)mode;
    return f(IC<FORCED>{});
  } else {
    switch (mode) {
      case 1: return f(IC<1>{});
      case 2: return f(IC<2>{});
      case 3: return f(IC<3>{});
      default: return f(IC<0>{});
    }
  }
}

// Hint modes of the stage kernels, measured per launch shape at batch 256, D 1152, bf16
// (all modes give identical results). Slices narrower than a 128-byte line take no hint
// (16-slot cells with 16+ events: loads or stores hinted run 7-60% slower).
int read_hints(bool whole_line, int cell, int events) {
  if (!whole_line) return 0;
  if (events == 1) return 1;                       // read-dominated (S rows in, 1 out)
  if (cell == 4 || events <= 8) return 3;          // 2-5% faster than loads only / none
  return 2;                                        // write-dominated: stores only (0-1.5%)
}
int write_hints(bool whole_line, int events) {
  if (!whole_line) return 0;
  return events <= 2 ? 2 : 3;  // E <= 2: stores only (4-5%); more events: both (3-7%)
}
int triangular_hints(int active) {
  // stores only for 1-2 updates, then loads and stores (XL shape: A = 9 296 -> 270 us,
  // A = 23 652 -> 603 against loads only; 3-6 updates equal)
  return active <= 2 ? 2 : 3;
}

// 1-D grid of slices x chunks (slices fastest: concurrently resident blocks cover whole
// channel rows of a token range).
unsigned blocks1d(int slices, int64_t chunks) { return unsigned(int64_t(slices) * chunks); }

template <typename TO>
int launch_fill_zero(void* out, int64_t n, hipStream_t st, const char* what) {
  if (n <= 0) return SIHC_OK;
  hipLaunchKernelGGL((k_fill_zero<TO>), dim3(unsigned((n + 255) / 256)), dim3(256), 0, st, static_cast<TO*>(out), n);
  return check_launch(what);
}
int fill_zero(int dtype, void* out, int64_t n, hipStream_t st, const char* what) {
  return dtype == SIHC_DTYPE_F32 ? launch_fill_zero<float>(out, n, st, what)
                                 : launch_fill_zero<bf16_t>(out, n, st, what);
}

int launch_finalize(const char* what, const float* part, void* out0, void* out1, int chunks, int R, int S, int C,
                    bool pair, int zero_mask, int out_dtype, hipStream_t st) {
  const int64_t n = int64_t(R) * S * C;
  // 4 outputs per thread when they never straddle a row and the rows are 16-byte aligned
  const bool wide = (int64_t(S) * C) % 4 == 0 && aligned(part, 16);
  auto go = [&](auto nv) {
    constexpr int NV = decltype(nv)::value;
    const unsigned blocks = unsigned((n + FINALIZE_FO * NV - 1) / (FINALIZE_FO * NV));
    if (out_dtype == SIHC_DTYPE_F32) {
      hipLaunchKernelGGL((k_finalize<float, NV>), dim3(blocks), dim3(256), 0, st, part, static_cast<float*>(out0),
                         static_cast<float*>(out1), chunks, R, S, C, pair ? 1 : 0, zero_mask);
    } else {
      hipLaunchKernelGGL((k_finalize<bf16_t, NV>), dim3(blocks), dim3(256), 0, st, part,
                         static_cast<bf16_t*>(out0), static_cast<bf16_t*>(out1), chunks, R, S, C, pair ? 1 : 0,
                         zero_mask);
    }
  };
  if (wide) {
    go(std::integral_constant<int, 4>{});
  } else {
    go(std::integral_constant<int, 1>{});
  }
  return check_launch(what);
}

int cells_copy(const char* what, bool gather, const void* src, const int32_t* index, void* dst, int64_t batch,
               int grid, int cell, int channels, int dtype, void* stream) {
  Geo g;
  if (int rc = check_geometry(what, batch, grid, cell, channels, &g)) return rc;
  if (!valid_dtype(dtype)) return fail(SIHC_ERR_INVALID, "%s: bad dtype %d", what, dtype);
  if (g.M == 0) return SIHC_OK;  // empty tensors may carry NULL data pointers
  if (!src || !dst) return fail(SIHC_ERR_INVALID, "%s: null pointer", what);
  const int64_t row_bytes = int64_t(channels) * elem_size(dtype);
  const int S = cell * cell;
  const int64_t rows = int64_t(g.M) * S;
  hipStream_t st = static_cast<hipStream_t>(stream);
  auto go = [&](auto r) {
    using R = decltype(r);
    const int row_chunks = int(row_bytes / int64_t(sizeof(R)));
    int bx = 64;
    while (bx > 1 && bx / 2 >= row_chunks) bx /= 2;
    const int by = 256 / bx;
    const int64_t gx = (rows + by - 1) / by;
    if (gx > 0x7fffffff) return fail(SIHC_ERR_INVALID, "%s: too many rows", what);
    auto launch = [&](auto kk) {
      constexpr int KK = decltype(kk)::value;
      if (gather) {
        hipLaunchKernelGGL((k_cells<R, KK, true>), dim3(unsigned(gx)), dim3(bx, by), 0, st,
                           static_cast<const R*>(src), static_cast<R*>(dst), index, g, row_chunks);
      } else {
        hipLaunchKernelGGL((k_cells<R, KK, false>), dim3(unsigned(gx)), dim3(bx, by), 0, st,
                           static_cast<const R*>(src), static_cast<R*>(dst), index, g, row_chunks);
      }
      return check_launch(what);
    };
    return with_cell(cell, launch);
  };
  if (row_bytes % 16 == 0 && aligned(src, 16) && aligned(dst, 16)) return go(u32x4{});
  if (row_bytes % 4 == 0 && aligned(src, 4) && aligned(dst, 4)) return go(uint32_t{});
  return go(uint16_t{});
}

// Adjoint of the gather (k_cells_add): one block per destination cell.
int cells_add(const char* what, const void* cells, const int32_t* index, void* x, int64_t batch, int grid, int cell,
              int channels, int dtype, void* stream) {
  Geo g;
  if (int rc = check_geometry(what, batch, grid, cell, channels, &g)) return rc;
  if (!valid_dtype(dtype)) return fail(SIHC_ERR_INVALID, "%s: bad dtype %d", what, dtype);
  if (g.M == 0) return SIHC_OK;  // empty tensors may carry NULL data pointers
  if (!cells || !x) return fail(SIHC_ERR_INVALID, "%s: null pointer", what);
  if (!index) return cells_copy(what, false, cells, nullptr, x, batch, grid, cell, channels, dtype, stream);
  if (g.GG > 16384) return fail(SIHC_ERR_INVALID, "%s: grid of %d cells exceeds 16384", what, g.GG);
  const void* ptrs[] = {cells, x};
  const int V = pick_vec(channels, elem_size(dtype), 8, ptrs, 2);
  const size_t lds = size_t(g.GG) * sizeof(int32_t);
  hipStream_t st = static_cast<hipStream_t>(stream);
  return with_dtype(dtype, [&](auto t) {
    using T = decltype(t);
    return with_vec(V, [&](auto vv) {
      constexpr int VV = decltype(vv)::value;
      if constexpr (VV * sizeof(T) > 16) {
        return fail(SIHC_ERR_INVALID, "%s: internal vector width", what);
      } else {
        return with_cell(cell, [&](auto kk) {
          constexpr int KK = decltype(kk)::value;
          hipLaunchKernelGGL((k_cells_add<T, VV, KK>), dim3(unsigned(g.M)), dim3(256), lds, st,
                             static_cast<const T*>(cells), static_cast<T*>(x), index, g);
          return check_launch(what);
        });
      }
    });
  });
}

// Shared launcher of the atomics-free weight-gradient reduction + finalize. With
// `dout` (workspace mode), the update gradients dout[e] = x * gamma[e] are written in
// the same pass.
int launch_wgrad(const char* what, const void* x, const void* const* z, void* out, int events, const Geo& g,
                 int S, bool carrier, const int32_t* index, int dtype, int out_dtype, void* workspace,
                 size_t workspace_bytes, hipStream_t st, void* const* dout = nullptr, const void* gamma = nullptr,
                 int gamma_dtype = SIHC_DTYPE_F32) {
  const int max_chunks = dout ? trib_chunks(g.M, events, g.C) : wgrad_chunks(g.M, events, g.C, carrier ? g.K : 2);
  int chunks = max_chunks;  // k_wgradz may use fewer (whole rounds of resident blocks)
  const size_t need = size_t(max_chunks) * events * S * g.C * sizeof(float);
  if (!workspace || workspace_bytes < need)
    return fail(SIHC_ERR_INVALID, "%s: workspace of %zu bytes required, got %zu", what, need, workspace_bytes);
  if (!aligned(workspace, 16)) return fail(SIHC_ERR_INVALID, "%s: workspace must be 16-byte aligned", what);
  const int es = elem_size(dtype);
  const void* ptrs[2 * SIHC_MAX_EVENTS + 1];
  int nptr = 0;
  for (int i = 0; i < events; ++i) ptrs[nptr++] = z[i];
  if (dout)
    for (int i = 0; i < events; ++i) ptrs[nptr++] = dout[i];
  ptrs[nptr++] = x;
  const int V = pick_vec(g.C, es, 8, ptrs, nptr);
  int bcg, slices;
  wgrad_block(g.C, V, events, &bcg, &slices);
  const int tpb = int((int64_t(g.M) + chunks - 1) / chunks);
  // Only chunks that hold tokens are launched and finalized: with tpb rounded up, the last
  // chunks of max_chunks can lie wholly past the last token (70,000 rows in 1,024 chunks:
  // 69 rows each, 1,015 chunks), and their partial rows would be read but never written.
  // (A zero-row branch for them inside k_trib_waves cost that kernel 7%.)
  if (g.M > 0) chunks = int((int64_t(g.M) + tpb - 1) / tpb);
  // x tile of TT tokens: at most 32 KB of LDS. With 16 or fewer event lanes on the
  // carrier, 8-token tiles keep one round of update loads per tile (measured: E=16
  // 828 -> 766 us at the XL shape; more events or the workspace mode prefer up to 64:
  // fused triangular backward A = 11 682 -> 667 us against 32). The tile size does not
  // change the summation order.
  int tt = 32768 / (S * bcg * V * int(sizeof(float)));
  tt = std::max(1, std::min(tt, carrier && events <= 16 ? 8 : SIHC_WG_TT));
  const size_t lds = size_t(tt) * S * bcg * V * sizeof(float);
  // event lanes of k_wgrad: padded so the block is a whole number of 4-wave groups (the
  // 4 SIMDs of a CU then hold equal shares) where that costs at most SIHC_WG_PAD lanes
  int lanes = events;
  if (SIHC_WG_PAD > 0) {
    int pad = events;
    while ((bcg * pad) % 256 != 0 && bcg * pad < 256) ++pad;
    if ((bcg * pad) % 256 == 0 && pad - events <= SIHC_WG_PAD) lanes = pad;
  }
  const PtrPack pk = pack(z, events);
  const PtrPack dk = dout ? pack(const_cast<const void* const*>(dout), events) : PtrPack{};
  // 16-slot carrier: k_wgrad16 (one channel per lane); only x is loaded as vectors
  const int slices16 = (g.C + C16_LANES - 1) / C16_LANES;
  const int vs16 = pick_vec(g.C, es, 8, &x, 1);
  // pipelined k_wgradz: bf16, up to 32 events, every row of x and the updates in whole
  // 16-byte vectors (C % 8 == 0, 16-byte aligned pointers)
  const bool usez = SIHC_C16Z && dtype == SIHC_DTYPE_BF16 && events <= 32 && !dout &&
                    pick_vec(g.C, es, 8, ptrs, nptr) == 8;
  const int slicesz = (g.C + C16_LANES - 1) / C16_LANES;
  float* part = static_cast<float*>(workspace);
  const int gf32 = gamma_dtype == SIHC_DTYPE_F32;
  int rc = with_dtype(dtype, [&](auto t) {
    using T = decltype(t);
    return with_vec(V, [&](auto vv) {
      constexpr int VV = decltype(vv)::value;
      if constexpr (VV * sizeof(T) > 16) {
        return fail(SIHC_ERR_INVALID, "%s: internal vector width", what);
      } else {
        auto go = [&](auto kk, auto car, auto sd) {
          constexpr int KK = decltype(kk)::value;
          constexpr bool CAR = decltype(car)::value;
          constexpr bool SD = decltype(sd)::value;
          // pipelined k_wgradz<KZ, NQ, EP> with nw event waves
          auto goz = [&](auto kz, auto nq, auto ep, int nw) {
            constexpr int KZ = decltype(kz)::value;
            constexpr int NQ = decltype(nq)::value;
            constexpr int EP = decltype(ep)::value;
            const size_t ldsz = size_t(SIHC_C16Z_TT) * (KZ * KZ + events) * C16_LANES * sizeof(bf16_t);
            // 16 slots: token pairs summed by dot2 (the same LDS bytes, NQ / 2 vector pairs
            // per thread)
            constexpr int NPQ = (NQ + 1) / 2;
            constexpr bool D2 = SIHC_K4_DOT2 && KZ == 4;
            const void* kfn;
            if constexpr (D2) {
              kfn = reinterpret_cast<const void*>(&k_wgradz_d2<NPQ, EP>);
            } else {
              kfn = reinterpret_cast<const void*>(&k_wgradz<KZ, NQ, EP>);
            }
            // whole rounds of resident blocks, so the last round is not part-empty
            chunks = whole_rounds(slicesz, max_chunks, resident_blocks(kfn, C16_LANES * nw, ldsz));
            const int tpbz = int((int64_t(g.M) + chunks - 1) / chunks);
            if (tpbz > 0) chunks = int((int64_t(g.M) + tpbz - 1) / tpbz);  // no chunk past the last token
            if constexpr (D2) {
              hipLaunchKernelGGL((k_wgradz_d2<NPQ, EP>), dim3(blocks1d(slicesz, chunks)), dim3(C16_LANES, nw), ldsz,
                                 st, reinterpret_cast<const bf16_t*>(x), pk, part, index, events, g, tpbz, slicesz);
            } else {
              hipLaunchKernelGGL((k_wgradz<KZ, NQ, EP>), dim3(blocks1d(slicesz, chunks)), dim3(C16_LANES, nw), ldsz,
                                 st, reinterpret_cast<const bf16_t*>(x), pk, part, index, events, g, tpbz, slicesz);
            }
          };
          const bool bf = std::is_same<T, bf16_t>::value && usez;
          // Shapes of the pipelined kernel (waves x events per lane), measured per event count
          // at the XL shape (batch 256, D 1152). Every shape stages every event row (waves x
          // events per lane >= E) and covers the carrier tile (64 x waves x vectors per
          // thread >= 256 vectors at 4 slots, 1024 at 16).
          if constexpr (CAR && KK == 4) {
            if (bf) {
              // 16 slots: E = 9 3 x 3 730 us (2 x 5 of 4: 907), E = 17-21 8 x 3 1095-1142 us
              // (5-6 x 4: 1320-1429), E = 28 / 32 8 x 4 1405 / 1421 us (k_wgrad16: 2290 / 2089)
              if (events <= 4) goz(IC<4>{}, IC<4>{}, IC<1>{}, 4);        // idle waves only stage
              else if (events <= 8) goz(IC<4>{}, IC<8>{}, IC<4>{}, 2);
              else if (events == 9) goz(IC<4>{}, IC<6>{}, IC<3>{}, 3);
              else if (events <= 12) goz(IC<4>{}, IC<4>{}, IC<3>{}, 4);
              else if (events <= 16) goz(IC<4>{}, IC<4>{}, IC<4>{}, 4);
              else if (events <= 24) goz(IC<4>{}, IC<2>{}, IC<3>{}, 8);
              else goz(IC<4>{}, IC<2>{}, IC<4>{}, 8);
            } else {
              const int nw = (events + C16_EPL - 1) / C16_EPL;
              hipLaunchKernelGGL((k_wgrad16<T>), dim3(blocks1d(slices16, chunks)), dim3(C16_LANES, nw), 0, st,
                                 static_cast<const T*>(x), pk, part, index, events, g, tpb, slices16, vs16);
            }
          } else if (CAR && KK == 2 && bf && (events == 2 || (events >= 5 && events <= 16) ||
                                               (events >= 19 && events <= 32))) {
            // 4 slots on row lanes (k_wgrad_rows), update groups per block measured per event
            // count at the XL shape: 2 for E = 2 and 5-6, 4 for 7-16, 8 for 19-32
            const int G = events <= 6 ? 2 : events <= 16 ? 4 : 8;
            const int slr = (g.C + 127) / 128;
            auto gorows = [&](auto na) {
              constexpr int NA = decltype(na)::value;
              chunks = whole_rounds(slr, max_chunks,
                                    resident_blocks(reinterpret_cast<const void*>(&k_wgrad_rows<NA>), 256, 0));
              const int tpr = int((int64_t(g.M) + chunks - 1) / chunks);
              if (tpr > 0) chunks = int((int64_t(g.M) + tpr - 1) / tpr);  // no chunk past the last token
              hipLaunchKernelGGL((k_wgrad_rows<NA>), dim3(blocks1d(slr, chunks)), dim3(16, G, 16 / G), 0, st,
                                 reinterpret_cast<const bf16_t*>(x), pk, part, index, events, g, tpr, slr);
            };
            switch ((events + G - 1) / G) {
              case 1: gorows(IC<1>{}); break;
              case 2: gorows(IC<2>{}); break;
              case 3: gorows(IC<3>{}); break;
              case 4: gorows(IC<4>{}); break;
              default: return fail(SIHC_ERR_INVALID, "%s: internal weight-gradient shape", what);
            }
          } else if (CAR && KK == 2 && bf && SIHC_WGZ_K2 && events >= 2) {
            // 4 slots, 3-4 and 17-18 events (one event keeps its direct kernel): E = 3 4 x 1
            // 201 us (k_wgrad: 504), E = 17-18 6 x 3 558-573 us (k_wgrad: 933-941; row lanes
            // 579-592)
            if (events <= 4) goz(IC<2>{}, IC<1>{}, IC<1>{}, 4);  // idle waves only stage
            else goz(IC<2>{}, IC<1>{}, IC<3>{}, (events + 2) / 3);
          } else if (!CAR && !SD && bf && events == 2) {
            // gamma gradient of 2 updates: the pipelined kernel on one-slot rows (1 wave x 2
            // updates: 77 us at 65,536 rows x 1152 channels; row lanes 81)
            goz(IC<1>{}, IC<1>{}, IC<2>{}, 1);
          } else if (!CAR && !SD && bf && events >= 3) {
            // gamma gradient of 3..32 updates on row lanes (k_gamma_rows), update groups per
            // block measured per update count at 65,536 rows x 1152 channels: A = 3-4 in 4
            // groups (A = 4 124 -> 117 us), 5-10 in one (A = 9 262 -> 229), 11-22 in two (A =
            // 17 453 -> 407), 23-32 in four (A = 32 798 -> 767); against the previous kernels
            const int G = events <= 4 ? 4 : events <= 10 ? 1 : events <= 22 ? 2 : 4;
            const int slr = (g.C + 127) / 128;
            auto gorows = [&](auto na) {
              constexpr int NA = decltype(na)::value;
              chunks = whole_rounds(slr, max_chunks,
                                    resident_blocks(reinterpret_cast<const void*>(&k_gamma_rows<NA>), 256, 0));
              const int tpr = int((int64_t(g.M) + chunks - 1) / chunks);
              if (tpr > 0) chunks = int((int64_t(g.M) + tpr - 1) / tpr);  // no chunk past the last token
              hipLaunchKernelGGL((k_gamma_rows<NA>), dim3(blocks1d(slr, chunks)), dim3(16, G, 16 / G), 0, st,
                                 reinterpret_cast<const bf16_t*>(x), pk, part, events, int(g.M), g.C, tpr, slr);
            };
            switch ((events + G - 1) / G) {
              case 1: gorows(IC<1>{}); break;
              case 5: gorows(IC<5>{}); break;
              case 6: gorows(IC<6>{}); break;
              case 7: gorows(IC<7>{}); break;
              case 8: gorows(IC<8>{}); break;
              case 9: gorows(IC<9>{}); break;
              case 10: gorows(IC<10>{}); break;
              case 11: gorows(IC<11>{}); break;
              default: return fail(SIHC_ERR_INVALID, "%s: internal gamma-gradient shape", what);
            }
          } else {
            if (events <= 2) {
              // fused triangular backward: 1 update hints loads only, 2 updates stores
              // only (11% faster than loads only at the XL shape)
              auto direct = [&](auto h) {
                constexpr int HM = decltype(h)::value;
                hipLaunchKernelGGL((k_wgrad_direct<T, VV, KK, CAR, SD, HM>), dim3(blocks1d(slices, chunks)),
                                   dim3(bcg, events), 0, st, static_cast<const T*>(x), pk, part, index, events, g,
                                   tpb, slices, dk, gamma, gf32);
              };
              if constexpr (SIHC_TRIB_NTM >= 0) {
                direct(IC<SIHC_TRIB_NTM>{});
              } else if (SD && events == 2) {
                direct(IC<2>{});
              } else {
                direct(IC<1>{});
              }
            } else {
              bool waves = false;
              if constexpr (SD && VV * sizeof(T) == 16) {
                // many updates: each wave streams one update at a time (k_trib_waves)
                waves = SIHC_TRIB_WAVES > 0 && events >= SIHC_TRIB_WAVES && g.C % VV == 0;
                if (waves) {
                  const int slicesw = (g.C + 16 * VV - 1) / (16 * VV);
                  const size_t ldsw = size_t(TRIB_TT + events) * 16 * VV * sizeof(float);
                  if (tpb <= TRIB_TT)
                    hipLaunchKernelGGL((k_trib_waves<T, VV, true>), dim3(blocks1d(slicesw, chunks)), dim3(256), ldsw,
                                       st, static_cast<const T*>(x), pk, part, events, g, tpb, slicesw, dk, gamma, gf32);
                  else
                    hipLaunchKernelGGL((k_trib_waves<T, VV, false>), dim3(blocks1d(slicesw, chunks)), dim3(256), ldsw,
                                       st, static_cast<const T*>(x), pk, part, events, g, tpb, slicesw, dk, gamma, gf32);
                }
              }
              if (!waves)
                hipLaunchKernelGGL((k_wgrad<T, VV, KK, CAR, SD>), dim3(blocks1d(slices, chunks)), dim3(bcg, lanes),
                                   lds, st, static_cast<const T*>(x), pk, part, index, events, g, tpb, slices, tt, dk,
                                   gamma, gf32);
            }
          }
          return check_launch(what);
        };
        if (!carrier && dout) return go(IC<2>{}, std::false_type{}, std::true_type{});
        if (!carrier) return go(IC<2>{}, std::false_type{}, std::false_type{});
        if (g.K == 2) return go(IC<2>{}, std::true_type{}, std::false_type{});
        return go(IC<4>{}, std::true_type{}, std::false_type{});
      }
    });
  });
  if (rc) return rc;
  return launch_finalize(what, part, out, nullptr, chunks, events, S, g.C, false, 0, out_dtype, st);
}

// Vector width of the per-event kernels: registers hold up to 2*S*V weights and 2*S*V
// accumulators, so wide vectors are used only for the 4-slot cell.
int event_vec(int C, int es, int cell, const void* const* ptrs, int n) {
  return pick_vec(C, es, cell == 2 ? SIHC_EV_VEC : 2, ptrs, n);
}

}  // namespace

// ----------------------------------------------------------------------------------
// Scratch of the allocation-free per-event backward (sihc_event_backward_noalloc): the
// fp32 partial rows of its weight-gradient reduction. Every GPU the library runs on
// holds its own copy of this array, at its own address, until the process ends. In host
// code `scratch` names a host-side stand-in, never device memory: host code uses only
// the per-device address that scratch_address() obtains from the runtime.
// ----------------------------------------------------------------------------------
static __device__ __align__(256) float scratch[SIHC_SCRATCH_BYTES / sizeof(float)];

namespace {

// Device address of `scratch` on the current device, looked up once per device (with
// that device current) and kept; SIHC_ERR_HIP if the runtime cannot resolve it.
int scratch_address(const char* what, void** out) {
  static std::mutex mu;
  static void* addr[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) {
    (void)hipGetLastError();
    return fail(SIHC_ERR_HIP, "%s: no current HIP device", what);
  }
  std::lock_guard<std::mutex> lock(mu);
  if (!addr[dev]) {
    void* p = nullptr;
    const hipError_t err = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (err != hipSuccess || !p) {
      (void)hipGetLastError();
      return fail(SIHC_ERR_HIP, "%s: cannot resolve the scratch array on device %d: %s", what, dev,
                  hipGetErrorString(err));
    }
    addr[dev] = p;
  }
  *out = addr[dev];
  return SIHC_OK;
}

}  // namespace

// ==================================================================================
// C ABI
// ==================================================================================
extern "C" {

const char* sihc_last_error(void) { return g_last_error.c_str(); }
int sihc_abi_version(void) { return SIHC_ABI_VERSION; }

int sihc_read(const void* x, const void* alpha, void* const* out, int events, int64_t batch, int grid,
              int cell, int channels, const int32_t* index, int dtype, void* stream) {
  const char* what = "sihc_read";
  Geo g;
  if (int rc = check_geometry(what, batch, grid, cell, channels, &g)) return rc;
  if (!valid_dtype(dtype)) return fail(SIHC_ERR_INVALID, "%s: bad dtype %d", what, dtype);
  if (int rc = check_count(what, events)) return rc;
  if (g.M == 0) return SIHC_OK;  // empty tensors may carry NULL data pointers
  if (!x || !alpha) return fail(SIHC_ERR_INVALID, "%s: null input", what);
  if (int rc = check_events(what, events, const_cast<const void* const*>(out))) return rc;
  const int es = elem_size(dtype);
  const void* ptrs[SIHC_MAX_EVENTS + 1];
  for (int i = 0; i < events; ++i) ptrs[i] = out[i];
  ptrs[events] = x;
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int V = pick_vec(channels, es, cell == 2 ? 8 : SIHC_RW_VEC_K4, ptrs, events + 1);
  const int S = cell * cell;
  // 16 slots, bf16 weights, 2-channel lanes: weights packed as bf16 in LDS (half the
  // bytes, so twice the channels per block within the LDS budget)
  const bool wb = dtype == SIHC_DTYPE_BF16 &&
                  ((SIHC_K4_BF16W && cell == 4 && V == 2) || (SIHC_K2_BF16W && cell == 2 && V == 8));
  const int wbytes = wb ? 2 : 4;
  // 16 slots, bf16, 2-channel lanes, word-aligned weights: slot pairs summed by dot2 (the
  // weights' pair words staged in the same LDS bytes as the packed bf16 weights)
  const bool d2 = SIHC_K4_DOT2 && wb && cell == 4 && aligned(alpha, 4);
  // 4 slots, bf16, 16-byte lanes, many events: one output array per wave at a time
  if (SIHC_RDW_MINE > 0 && cell == 2 && dtype == SIHC_DTYPE_BF16 && V == 8 && events >= SIHC_RDW_MINE &&
      aligned(alpha, 4)) {
    const int slicesw = (channels + 127) / 128;
    const int64_t chunksw = (int64_t(g.M) + RDW_TT - 1) / RDW_TT;
    const size_t ldsw = size_t(RDW_TT + events) * 2 * 128 * sizeof(uint32_t);
    const PtrPack pkw = pack(ptrs, events);
    return with_hints<SIHC_RD_NTM>(read_hints(true, cell, events), [&](auto nt) {
      constexpr int NT = decltype(nt)::value;
      hipLaunchKernelGGL((k_read_w<NT>), dim3(blocks1d(slicesw, chunksw)), dim3(256), ldsw, st,
                         static_cast<const bf16_t*>(x), static_cast<const bf16_t*>(alpha), pkw, index, events, g,
                         slicesw);
      return check_launch(what);
    });
  }
  const Shape2D sh = cell == 2 ? shape_for(channels, V, SIHC_RW_BCG, events * S * wbytes)
                               : shape_for(channels, V, events <= 8 ? 64 : SIHC_RW_BCG_K4, events * S * wbytes,
                                           SIHC_RW_LDS_K4);  // 64 lanes to 8 events: E = 4 569 -> 542 us
  const int tpb = sh.tl * rw_tokens_per_lane(cell, events, true, d2 && V == 2);
  const int64_t chunks = (int64_t(g.M) + tpb - 1) / tpb;
  const int gs = tpb;  // one contiguous run per block (interleaved groups measured no faster)
  const size_t lds = size_t(events) * S * sh.bcg * V * wbytes;
  const PtrPack pk = pack(ptrs, events);
  return with_dtype(dtype, [&](auto t) {
    using T = decltype(t);
    return with_vec(V, [&](auto vv) {
      constexpr int VV = decltype(vv)::value;
      if constexpr (VV * sizeof(T) > 16) {
        return fail(SIHC_ERR_INVALID, "%s: internal vector width", what);
      } else {
        return with_cell(cell, [&](auto kk) {
          constexpr int KK = decltype(kk)::value;
          if constexpr (KK == 4 && VV > SIHC_RW_VEC_K4) {
            return fail(SIHC_ERR_INVALID, "%s: internal vector width", what);
          } else {
            // non-temporal carrier loads: for 1-2 events (4 slots) or up to 12 (16 slots),
            // and only with slice rows of whole 128-byte lines
            const int hints = read_hints(sh.bcg * VV * int(sizeof(T)) >= 128, cell, events);
            return with_bcg<KK>(sh.bcg, [&](auto bb) {
              constexpr int BB = decltype(bb)::value;
              return with_hints<SIHC_RD_NTM>(hints, [&](auto nt) {
                constexpr int NT = decltype(nt)::value;
                auto go = [&](auto w) {
                  constexpr bool WB = decltype(w)::value;
                  hipLaunchKernelGGL((k_read<T, VV, KK, BB, NT, WB>), dim3(blocks1d(sh.slices, chunks)),
                                     dim3(sh.bcg, sh.tl), lds, st, static_cast<const T*>(x),
                                     static_cast<const T*>(alpha), pk, index, events, g, gs, int(chunks), sh.slices);
                  return check_launch(what);
                };
                if constexpr (KK == 4 && VV == 2 && std::is_same_v<T, bf16_t>) {
                  if (d2) {
                    hipLaunchKernelGGL((k_read_d2<SIHC_RD2_U, BB, NT>), dim3(blocks1d(sh.slices, chunks)),
                                       dim3(sh.bcg, sh.tl), lds, st, static_cast<const T*>(x),
                                       static_cast<const T*>(alpha), pk, index, events, g, gs, int(chunks),
                                       sh.slices);
                    return check_launch(what);
                  }
                }
                if constexpr (((KK == 4 && VV == 2) || (KK == 2 && VV == 8)) && std::is_same_v<T, bf16_t>) {
                  if (wb) return go(std::true_type{});
                }
                return go(std::false_type{});
              });
            });
          }
        });
      }
    });
  });
}

int sihc_write(const void* x, const void* const* updates, const void* beta, void* out, int events,
               int64_t batch, int grid, int cell, int channels, int add_x, const int32_t* index, int x_dtype,
               int w_dtype, void* stream) {
  const char* what = "sihc_write";
  Geo g;
  if (int rc = check_geometry(what, batch, grid, cell, channels, &g)) return rc;
  if (!valid_dtype(x_dtype) || !valid_dtype(w_dtype)) return fail(SIHC_ERR_INVALID, "%s: bad dtype", what);
  if (x_dtype == SIHC_DTYPE_BF16 && w_dtype == SIHC_DTYPE_F32)
    return fail(SIHC_ERR_INVALID, "%s: fp32 updates with a bf16 carrier are not supported", what);
  if (int rc = check_count(what, events)) return rc;
  if (g.M == 0) return SIHC_OK;  // empty tensors may carry NULL data pointers
  if ((add_x && !x) || !beta || !out) return fail(SIHC_ERR_INVALID, "%s: null input", what);
  if (int rc = check_events(what, events, updates)) return rc;
  const void* ptrs[SIHC_MAX_EVENTS + 2];
  for (int i = 0; i < events; ++i) ptrs[i] = updates[i];
  ptrs[events] = add_x ? x : nullptr;
  ptrs[events + 1] = out;
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int es = std::max(elem_size(x_dtype), elem_size(w_dtype));
  const int V = pick_vec(channels, es, cell == 2 ? 8 : SIHC_RW_VEC_K4, ptrs, events + 2);
  const int S = cell * cell;
  const int E4 = (events + 3) & ~3;
  // 16 slots, bf16 weights, 2-channel lanes: weights packed as bf16 in LDS (as sihc_read)
  const bool wb = w_dtype == SIHC_DTYPE_BF16 &&
                  ((SIHC_K4_BF16W && cell == 4 && V == 2) || (SIHC_K2_BF16W && cell == 2 && V == 8));
  const int wbytes = wb ? 2 : 4;
  // 16 slots, bf16 carrier, updates and weights, 2-channel lanes: event pairs summed by
  // dot2 (pair words staged in no more LDS than the packed bf16 weights)
  const bool d2 = SIHC_K4_DOT2 && wb && cell == 4 && x_dtype == SIHC_DTYPE_BF16;
  const Shape2D sh = cell == 2 ? shape_for(channels, V, SIHC_RW_BCG, E4 * S * wbytes)
                               : shape_for(channels, V, E4 <= 8 ? 64 : SIHC_RW_BCG_K4, E4 * S * wbytes,
                                           SIHC_RW_LDS_K4);  // 64 lanes to 8 events: E = 4 1010 -> 964 us
  const int tpb = sh.tl * rw_tokens_per_lane(cell, E4);
  const int64_t chunks = (int64_t(g.M) + tpb - 1) / tpb;
  const int gs = tpb;  // one contiguous run per block (interleaved groups measured no faster)
  const size_t lds = size_t(E4) * S * sh.bcg * V * wbytes;
  const PtrPack pk = pack(updates, events);
  auto launch = [&](auto tx, auto tw) {
    using TX = decltype(tx);
    using TW = decltype(tw);
    return with_vec(V, [&](auto vv) {
      constexpr int VV = decltype(vv)::value;
      if constexpr (VV * sizeof(TX) > 16) {
        return fail(SIHC_ERR_INVALID, "%s: internal vector width", what);
      } else {
        return with_cell(cell, [&](auto kk) {
          constexpr int KK = decltype(kk)::value;
          if constexpr (KK == 4 && VV > SIHC_RW_VEC_K4) {
            return fail(SIHC_ERR_INVALID, "%s: internal vector width", what);
          } else {
            // non-temporal loads with 8+ events and slice rows of whole 128-byte lines
            const int hints = write_hints(sh.bcg * VV * int(sizeof(TX)) >= 128, events);
            return with_bool(add_x != 0, [&](auto ax) {
              constexpr bool AX = decltype(ax)::value;
              return with_bcg<KK>(sh.bcg, [&](auto bb) {
                constexpr int BB = decltype(bb)::value;
                return with_hints<SIHC_WR_NTM>(hints, [&](auto nt) {
                  constexpr int NT = decltype(nt)::value;
                  auto go = [&](auto w) {
                    constexpr bool WB = decltype(w)::value;
                    hipLaunchKernelGGL((k_write<TX, TW, VV, KK, AX, BB, NT, WB>), dim3(blocks1d(sh.slices, chunks)),
                                       dim3(sh.bcg, sh.tl), lds, st, static_cast<const TX*>(x), pk,
                                       static_cast<const TW*>(beta), static_cast<TX*>(out), index, events, g, gs,
                                       int(chunks), sh.slices);
                    return check_launch(what);
                  };
                  if constexpr (KK == 4 && VV == 2 && std::is_same_v<TX, bf16_t> && std::is_same_v<TW, bf16_t>) {
                    if (d2) {
                      hipLaunchKernelGGL((k_write_d2<SIHC_WR2_U, AX, BB, NT>), dim3(blocks1d(sh.slices, chunks)),
                                         dim3(sh.bcg, sh.tl), lds, st, static_cast<const TX*>(x), pk,
                                         static_cast<const TW*>(beta), static_cast<TX*>(out), index, events, g, gs,
                                         int(chunks), sh.slices);
                      return check_launch(what);
                    }
                  }
                  if constexpr (((KK == 4 && VV == 2) || (KK == 2 && VV == 8)) && std::is_same_v<TW, bf16_t>) {
                    if (wb) return go(std::true_type{});
                  }
                  return go(std::false_type{});
                });
              });
            });
          }
        });
      }
    });
  };
  if (x_dtype == SIHC_DTYPE_F32 && w_dtype == SIHC_DTYPE_F32) return launch(float{}, float{});
  if (x_dtype == SIHC_DTYPE_F32) return launch(float{}, bf16_t{});
  return launch(bf16_t{}, bf16_t{});
}

size_t sihc_weight_grad_workspace_size(int events, int64_t batch, int grid, int cell, int channels) {
  if (events < 1 || batch < 0 || grid <= 0 || cell <= 0 || channels <= 0) return 0;
  const int64_t M = batch * int64_t(grid) * grid;
  return size_t(wgrad_chunks(M, events, channels, cell)) * events * cell * cell * channels * sizeof(float);
}

int sihc_weight_grad(const void* x, const void* const* z, void* out, int events, int64_t batch, int grid, int cell,
                     int channels, const int32_t* index, int dtype, int out_dtype, void* workspace,
                     size_t workspace_bytes, void* stream) {
  const char* what = "sihc_weight_grad";
  Geo g;
  if (int rc = check_geometry(what, batch, grid, cell, channels, &g)) return rc;
  if (!valid_dtype(dtype) || !valid_dtype(out_dtype)) return fail(SIHC_ERR_INVALID, "%s: bad dtype", what);
  if (int rc = check_count(what, events)) return rc;
  if (!out) return fail(SIHC_ERR_INVALID, "%s: null output", what);
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (g.M == 0)  // empty reduction: zero gradient (inputs may carry NULL pointers)
    return fill_zero(out_dtype, out, int64_t(events) * cell * cell * channels, st, what);
  if (!x) return fail(SIHC_ERR_INVALID, "%s: null input", what);
  if (int rc = check_events(what, events, z)) return rc;
  return launch_wgrad(what, x, z, out, events, g, cell * cell, true, index, dtype, out_dtype, workspace,
                      workspace_bytes, st);
}

int sihc_triangular(const void* base, const void* const* updates, const void* gamma, void* out, int active,
                    int64_t rows, int channels, int dtype, int gamma_dtype, void* stream) {
  const char* what = "sihc_triangular";
  if (rows < 0 || rows >= SIHC_MAX_TOKENS || channels <= 0) return fail(SIHC_ERR_INVALID, "%s: bad sizes", what);
  if (!valid_dtype(dtype) || !valid_dtype(gamma_dtype)) return fail(SIHC_ERR_INVALID, "%s: bad dtype", what);
  if (int rc = check_count(what, active)) return rc;
  if (rows == 0) return SIHC_OK;  // empty tensors may carry NULL data pointers
  if (!base || !gamma || !out) return fail(SIHC_ERR_INVALID, "%s: null input", what);
  if (int rc = check_events(what, active, updates)) return rc;
  const int es = elem_size(dtype);
  const void* ptrs[SIHC_MAX_EVENTS + 2];
  for (int i = 0; i < active; ++i) ptrs[i] = updates[i];
  ptrs[active] = base;
  ptrs[active + 1] = out;
  const int V = pick_vec(channels, es, 8, ptrs, active + 2);
  const int A4 = (active + 3) & ~3;
  const Shape2D sh = shape_for(channels, V, SIHC_RW_BCG, A4 * 4);
  // 32-token blocks (64 with one update): 3-5% faster than 128-token ones
  const int tpb = sh.tl * (active == 1 ? 4 : 2);
  const int64_t chunks = (rows + tpb - 1) / tpb;
  const int gs = tpb;  // one contiguous run per block
  const size_t lds = size_t(A4) * sh.bcg * V * 4;
  const PtrPack pk = pack(updates, active);
  hipStream_t st = static_cast<hipStream_t>(stream);
  return with_dtype(dtype, [&](auto t) {
    using T = decltype(t);
    return with_dtype(gamma_dtype, [&](auto tg) {
      using TG = decltype(tg);
      return with_vec(V, [&](auto vv) {
        constexpr int VV = decltype(vv)::value;
        if constexpr (VV * sizeof(T) > 16) {
          return fail(SIHC_ERR_INVALID, "%s: internal vector width", what);
        } else {
          return with_hints<SIHC_TRI_NTM>(triangular_hints(active), [&](auto nt) {
            constexpr int NT = decltype(nt)::value;
            hipLaunchKernelGGL((k_triangular<T, TG, VV, NT>), dim3(blocks1d(sh.slices, chunks)), dim3(sh.bcg, sh.tl),
                               lds, st, static_cast<const T*>(base), pk, static_cast<const TG*>(gamma),
                               static_cast<T*>(out), active, int(rows), channels, gs, int(chunks), sh.slices);
            return check_launch(what);
          });
        }
      });
    });
  });
}

size_t sihc_triangular_gamma_grad_workspace_size(int active, int64_t rows, int channels) {
  if (active < 1 || rows < 0 || channels <= 0) return 0;
  // covers both users: the gamma gradient and the fused triangular backward (more chunks)
  return size_t(trib_chunks(rows, active, channels)) * active * channels * sizeof(float);
}

int sihc_triangular_gamma_grad(const void* grad, const void* const* updates, void* out, int active, int64_t rows,
                               int channels, int dtype, int out_dtype, void* workspace, size_t workspace_bytes,
                               void* stream) {
  const char* what = "sihc_triangular_gamma_grad";
  if (rows < 0 || rows >= SIHC_MAX_TOKENS || channels <= 0) return fail(SIHC_ERR_INVALID, "%s: bad sizes", what);
  if (!valid_dtype(dtype) || !valid_dtype(out_dtype)) return fail(SIHC_ERR_INVALID, "%s: bad dtype", what);
  if (int rc = check_count(what, active)) return rc;
  if (!out) return fail(SIHC_ERR_INVALID, "%s: null output", what);
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (rows == 0) return fill_zero(out_dtype, out, int64_t(active) * channels, st, what);
  if (!grad) return fail(SIHC_ERR_INVALID, "%s: null input", what);
  if (int rc = check_events(what, active, updates)) return rc;
  Geo g;
  g.M = int(rows);
  g.GG = 1;
  g.G = 1;
  g.K = 1;
  g.GK = 1;
  g.C = channels;
  set_divisors(g);
  return launch_wgrad(what, grad, updates, out, active, g, 1, false, nullptr, dtype, out_dtype, workspace,
                      workspace_bytes, st);
}

int sihc_triangular_backward(const void* grad, const void* const* updates, const void* gamma,
                             void* const* grad_updates, void* grad_gamma, int active, int64_t rows, int channels,
                             int dtype, int gamma_dtype, int out_dtype, void* workspace, size_t workspace_bytes,
                             void* stream) {
  const char* what = "sihc_triangular_backward";
  if (rows < 0 || rows >= SIHC_MAX_TOKENS || channels <= 0) return fail(SIHC_ERR_INVALID, "%s: bad sizes", what);
  if (!valid_dtype(dtype) || !valid_dtype(gamma_dtype) || !valid_dtype(out_dtype))
    return fail(SIHC_ERR_INVALID, "%s: bad dtype", what);
  if (int rc = check_count(what, active)) return rc;
  if (!grad_gamma || !grad_updates) return fail(SIHC_ERR_INVALID, "%s: null output", what);
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (rows == 0) return fill_zero(out_dtype, grad_gamma, int64_t(active) * channels, st, what);
  if (!grad || !gamma) return fail(SIHC_ERR_INVALID, "%s: null input", what);
  if (int rc = check_events(what, active, updates)) return rc;
  if (int rc = check_events(what, active, const_cast<const void* const*>(grad_updates))) return rc;
  Geo g;
  g.M = int(rows);
  g.GG = 1;
  g.G = 1;
  g.K = 1;
  g.GK = 1;
  g.C = channels;
  set_divisors(g);
  return launch_wgrad(what, grad, updates, grad_gamma, active, g, 1, false, nullptr, dtype, out_dtype, workspace,
                      workspace_bytes, st, grad_updates, gamma, gamma_dtype);
}

int sihc_event_forward(const void* x, const void* dz, const void* beta, const void* alpha_next, void* x_out,
                       void* z_out, int64_t batch, int grid, int cell, int channels, const int32_t* index, int dtype,
                       void* stream) {
  const char* what = "sihc_event_forward";
  Geo g;
  if (int rc = check_geometry(what, batch, grid, cell, channels, &g)) return rc;
  if (!valid_dtype(dtype)) return fail(SIHC_ERR_INVALID, "%s: bad dtype", what);
  if (g.M == 0) return SIHC_OK;  // empty tensors may carry NULL data pointers
  if (!x || !dz || !beta || !x_out) return fail(SIHC_ERR_INVALID, "%s: null input", what);
  if ((alpha_next == nullptr) != (z_out == nullptr))
    return fail(SIHC_ERR_INVALID, "%s: alpha_next and z_out must both be given or both be NULL", what);
  const int es = elem_size(dtype);
  const int S = cell * cell;
  if (!aligned(beta, std::min(16, S * es)) || (alpha_next && !aligned(alpha_next, std::min(16, S * es))))
    return fail(SIHC_ERR_INVALID, "%s: weights must be aligned to %d bytes", what, std::min(16, S * es));
  const void* ptrs[] = {x, dz, x_out, z_out};
  int V = event_vec(channels, es, cell, ptrs, 4);
  // Weight rows are loaded as V*S contiguous elements: need min(16, V*S*es) alignment.
  while (V > 1 && (!aligned(beta, std::min(16, V * S * es)) ||
                   (alpha_next && !aligned(alpha_next, std::min(16, V * S * es)))))
    V /= 2;
  Shape2D sh = shape_for(channels, V, SIHC_EV_BCG, 0);
  sh.tl = SIHC_EV_FWD_THREADS / sh.bcg;  // one-shot blocks of SIHC_EV_FWD_THREADS threads
  const int tpb = sh.tl * SIHC_EV_TPT;
  const int64_t chunks = (int64_t(g.M) + tpb - 1) / tpb;
  hipStream_t st = static_cast<hipStream_t>(stream);
  return with_dtype(dtype, [&](auto t) {
    using T = decltype(t);
    return with_vec(V, [&](auto vv) {
      constexpr int VV = decltype(vv)::value;
      return with_cell(cell, [&](auto kk) {
        constexpr int KK = decltype(kk)::value;
        if constexpr (VV * sizeof(T) > 16 || (KK == 4 && VV > 2) || VV > SIHC_EV_VEC) {
          return fail(SIHC_ERR_INVALID, "%s: internal vector width", what);
        } else {
          return with_bool(alpha_next != nullptr, [&](auto hz) {
            constexpr bool HZ = decltype(hz)::value;
            constexpr bool NTL = (SIHC_EV_FWD_NT & 1) != 0, NTS = (SIHC_EV_FWD_NT & 2) != 0;
            if constexpr (SIHC_EV_FWD_ROWS && KK == 2 && HZ && std::is_same_v<T, bf16_t>) {
              // whole rows of 16-byte lanes: every carrier, dz and z_out row and both weight
              // arrays 16-byte aligned, C / 8 lanes of one token within one block. With a read
              // part only: the write-only forward (no alpha_next) ran 3% slower on whole rows
              // than on the general kernel (224 against 217 us at batch 256, C 1152).
              constexpr int VR = 8;
              const int lanes = channels / VR;
              if (channels % VR == 0 && lanes <= 1024 && aligned(x, 16) && aligned(dz, 16) && aligned(x_out, 16) &&
                  aligned(z_out, 16) && aligned(beta, 16) && aligned(alpha_next, 16)) {
                const int tr = std::max(1, SIHC_EV_ROW_THREADS / lanes);
                const int64_t blocks = (int64_t(g.M) + tr - 1) / tr;
                hipLaunchKernelGGL((k_event_fwd_rows<T, VR, HZ, NTL, NTS>), dim3(unsigned(blocks)), dim3(lanes, tr), 0,
                                   st, static_cast<const T*>(x), static_cast<const T*>(dz),
                                   static_cast<const T*>(beta), static_cast<const T*>(alpha_next),
                                   static_cast<T*>(x_out), static_cast<T*>(z_out), index, g);
                return check_launch(what);
              }
            }
            if constexpr (SIHC_EV_FWD16 && KK == 4 && VV == 2 && std::is_same_v<T, bf16_t>) {
              hipLaunchKernelGGL((k_event_fwd16<HZ, NTL, NTS>), dim3(blocks1d(sh.slices, chunks)), dim3(sh.bcg, sh.tl),
                                 0, st, static_cast<const T*>(x), static_cast<const T*>(dz),
                                 static_cast<const T*>(beta), static_cast<const T*>(alpha_next),
                                 static_cast<T*>(x_out), static_cast<T*>(z_out), index, g, tpb, sh.slices);
              return check_launch(what);
            }
            hipLaunchKernelGGL((k_event_fwd<T, VV, KK, HZ, NTL, NTS>), dim3(blocks1d(sh.slices, chunks)), dim3(sh.bcg, sh.tl), 0,
                               st, static_cast<const T*>(x), static_cast<const T*>(dz), static_cast<const T*>(beta),
                               static_cast<const T*>(alpha_next), static_cast<T*>(x_out), static_cast<T*>(z_out),
                               index, g, tpb, sh.slices);
            return check_launch(what);
          });
        }
      });
    });
  });
}

size_t sihc_event_backward_workspace_size(int64_t batch, int grid, int cell, int channels) {
  if (batch < 0 || grid <= 0 || cell <= 0 || channels <= 0) return 0;
  const int64_t M = batch * int64_t(grid) * grid;
  return size_t(event_bwd_chunks(M, cell)) * 2 * cell * cell * channels * sizeof(float);
}

// sihc_event_backward and its allocation-free variant (errors name the entry point)
static int event_backward_impl(const char* what, const void* grad_x_out, const void* grad_z_out, const void* x_out,
                               const void* dz, const void* beta, const void* alpha_next, void* grad_x, void* grad_dz,
                               void* grad_beta, void* grad_alpha_next, int64_t batch, int grid, int cell,
                               int channels, const int32_t* index, int dtype, int w_dtype, void* workspace,
                               size_t workspace_bytes, void* stream, int* defer = nullptr,
                               const EvCarry* prev = nullptr) {
  Geo g;
  if (int rc = check_geometry(what, batch, grid, cell, channels, &g)) return rc;
  if (!valid_dtype(dtype) || !valid_dtype(w_dtype)) return fail(SIHC_ERR_INVALID, "%s: bad dtype", what);
  // beta / alpha_next are read as `dtype`, and their gradients share their dtype
  if (w_dtype != dtype)
    return fail(SIHC_ERR_INVALID, "%s: weights must share the carrier dtype (w_dtype %d, dtype %d)", what, w_dtype,
                dtype);
  const int S = cell * cell;
  const int64_t wn = int64_t(S) * channels;
  hipStream_t st = static_cast<hipStream_t>(stream);
  // an earlier deferred call's finalize, run by this launch's trailing blocks
  const bool carry = prev && prev->part;
  const unsigned carry_blocks =
      carry ? unsigned((int64_t(2) * S * channels + EV_CARRY_OUTPUTS_PER_BLOCK - 1) / EV_CARRY_OUTPUTS_PER_BLOCK) : 0u;
  if (g.M == 0) {  // no tokens: zero weight gradients (token tensors may carry NULL pointers)
    if (defer) defer[0] = defer[1] = 0;  // nothing left for the finalize
    if (carry) {  // no launch of the backward to carry it: a finalize launch of its own
      FinalizeBatch b{};
      b.part[0] = prev->part;
      b.out0[0] = prev->out0;
      b.out1[0] = prev->out1;
      b.chunks[0] = prev->chunks;
      b.zero_mask[0] = prev->zero_mask;
      if (w_dtype == SIHC_DTYPE_F32)
        hipLaunchKernelGGL((k_finalize_batch<float>), dim3(carry_blocks, 1), dim3(256), 0, st, b, S, channels);
      else
        hipLaunchKernelGGL((k_finalize_batch<bf16_t>), dim3(carry_blocks, 1), dim3(256), 0, st, b, S, channels);
      if (int rc = check_launch(what)) return rc;
    }
    if (beta && grad_beta)
      if (int rc = fill_zero(w_dtype, grad_beta, wn, st, what)) return rc;
    if (grad_alpha_next) return fill_zero(w_dtype, grad_alpha_next, wn, st, what);
    return SIHC_OK;
  }
  const bool has_w = beta != nullptr;
  const bool has_g = grad_z_out != nullptr;
  const bool has_h = grad_x_out != nullptr;
  if (has_w != (dz != nullptr) || has_w != (grad_dz != nullptr) || has_w != (grad_beta != nullptr))
    return fail(SIHC_ERR_INVALID, "%s: beta, dz, grad_dz and grad_beta must all be given or all be NULL", what);
  if (has_g && (!alpha_next || !x_out || !grad_alpha_next))
    return fail(SIHC_ERR_INVALID, "%s: grad_z_out needs alpha_next, x_out and grad_alpha_next", what);
  if (!has_w && !has_g) return fail(SIHC_ERR_INVALID, "%s: neither a write nor a read part", what);
  if (!grad_x && has_g)
    return fail(SIHC_ERR_INVALID, "%s: grad_x may be NULL only without grad_z_out (it equals grad_x_out)", what);
  const int max_chunks = event_bwd_chunks(g.M, cell);
  const size_t need = size_t(max_chunks) * 2 * S * channels * sizeof(float);
  if (!workspace || workspace_bytes < need)
    return fail(SIHC_ERR_INVALID, "%s: workspace of %zu bytes required, got %zu", what, need, workspace_bytes);
  int chunks = max_chunks;
  if (!aligned(workspace, 16)) return fail(SIHC_ERR_INVALID, "%s: workspace must be 16-byte aligned", what);
  const int es = elem_size(dtype);
  if ((beta && !aligned(beta, std::min(16, S * es))) || (alpha_next && !aligned(alpha_next, std::min(16, S * es))))
    return fail(SIHC_ERR_INVALID, "%s: weights must be aligned to %d bytes", what, std::min(16, S * es));
  const void* ptrs[] = {grad_x_out, grad_z_out, x_out, dz, grad_x, grad_dz};
  int V = event_vec(channels, es, cell, ptrs, 6);
  while (V > 1 && ((beta && !aligned(beta, std::min(16, V * S * es))) ||
                   (has_g && !aligned(alpha_next, std::min(16, V * S * es)))))
    V /= 2;
  const Shape2D sh = shape_for(channels, V, SIHC_EV_BCG, 0);
  const size_t lds = size_t(sh.tl) * sh.bcg * S * V * sizeof(float);  // TL x (BCG*S*V) floats
  if (carry && (sh.tl * sh.bcg != 256 || lds < FINALIZE_LDS(4) * sizeof(float)))
    return fail(SIHC_ERR_INVALID, "%s: internal block shape of the carried finalize", what);
  float* part = static_cast<float*>(workspace);
  const bool store_t = grad_x != nullptr;
  // Valid part combinations: read part present (t stored), or write part only.
  const int mode = has_g ? (has_w ? 0 : 1) : (store_t ? 2 : 3);
  int rc = with_dtype(dtype, [&](auto t) {
    using T = decltype(t);
    return with_vec(V, [&](auto vv) {
      constexpr int VV = decltype(vv)::value;
      return with_cell(cell, [&](auto kk) {
        constexpr int KK = decltype(kk)::value;
        if constexpr (VV * sizeof(T) > 16 || (KK == 4 && VV > 2) || VV > SIHC_EV_VEC) {
          return fail(SIHC_ERR_INVALID, "%s: internal vector width", what);
        } else {
          return with_bool(has_h, [&](auto hh) {
            constexpr bool HH = decltype(hh)::value;
            auto go = [&](auto hg, auto hw, auto stt) {
              constexpr bool HG = decltype(hg)::value, HW = decltype(hw)::value, STT = decltype(stt)::value;
              constexpr bool NTL = (SIHC_EV_BWD_NT & 1) != 0, NTS = (SIHC_EV_BWD_NT & 2) != 0;
              // 16-slot bf16 cells with 2-channel lanes: the register-lean kernel
              constexpr bool B16 = SIHC_EV_BWD16 && KK == 4 && VV == 2 && std::is_same_v<T, bf16_t>;
              const void* kfn;
              if constexpr (B16) {
                kfn = reinterpret_cast<const void*>(&k_event_bwd16<HH, HG, HW, STT, NTL, NTS>);
              } else {
                kfn = reinterpret_cast<const void*>(&k_event_bwd<T, VV, KK, HH, HG, HW, STT, NTL, NTS>);
              }
              chunks = whole_rounds(sh.slices, max_chunks, resident_blocks(kfn, sh.bcg * sh.tl, lds));
              // token groups: a multiple of one loop iteration (SIHC_EV_UNROLL x TL tokens);
              // group 0 means one contiguous run of tokens per chunk
              const int gs = group_tokens(KK == 2 ? SIHC_EV_GROUP : SIHC_EV_GROUP_K4, g.M, chunks,
                                          SIHC_EV_UNROLL * sh.tl);
              EvCarry cy{};
              if (carry) cy = *prev;
              cy.nmain = int(blocks1d(sh.slices, chunks));
              const dim3 grid_blocks(blocks1d(sh.slices, chunks) + carry_blocks);
              if constexpr (B16) {
                hipLaunchKernelGGL((k_event_bwd16<HH, HG, HW, STT, NTL, NTS>), grid_blocks, dim3(sh.bcg, sh.tl), lds,
                                   st, static_cast<const T*>(grad_x_out), static_cast<const T*>(grad_z_out),
                                   static_cast<const T*>(x_out), static_cast<const T*>(dz),
                                   static_cast<const T*>(beta), static_cast<const T*>(alpha_next),
                                   static_cast<T*>(grad_x), static_cast<T*>(grad_dz), part, index, g, gs, chunks,
                                   sh.slices, cy);
                return check_launch(what);
              }
              hipLaunchKernelGGL((k_event_bwd<T, VV, KK, HH, HG, HW, STT, NTL, NTS>), grid_blocks, dim3(sh.bcg, sh.tl),
                                 lds, st, static_cast<const T*>(grad_x_out), static_cast<const T*>(grad_z_out),
                                 static_cast<const T*>(x_out), static_cast<const T*>(dz),
                                 static_cast<const T*>(beta), static_cast<const T*>(alpha_next),
                                 static_cast<T*>(grad_x), static_cast<T*>(grad_dz), part, index, g, gs, chunks,
                                 sh.slices, cy);
              return check_launch(what);
            };
            switch (mode) {
              case 0: return go(std::true_type{}, std::true_type{}, std::true_type{});
              case 1: return go(std::true_type{}, std::false_type{}, std::true_type{});
              case 2: return go(std::false_type{}, std::true_type{}, std::true_type{});
              default: return go(std::false_type{}, std::true_type{}, std::false_type{});
            }
          });
        }
      });
    });
  });
  if (rc) return rc;
  if (defer) {  // the caller runs the finalize later (sihc_event_finalize)
    defer[0] = chunks;
    defer[1] = (has_w ? 1 : 0) | (has_g ? 2 : 0);
    if (!has_g && grad_alpha_next) return fill_zero(w_dtype, grad_alpha_next, wn, st, what);
    return SIHC_OK;
  }
  // Partial rows are [chunks][2][S][C]: row 0 -> grad_beta, row 1 -> grad_alpha_next
  // (written as zeros when there is no read part). A part the kernel did not run has no
  // partial rows, so the finalize does not read them.
  return launch_finalize(what, part, has_w ? grad_beta : nullptr, grad_alpha_next, chunks, 2, S, channels, true,
                         (has_w ? 0 : 1) | (has_g ? 0 : 2), w_dtype, st);
}

int sihc_event_backward(const void* grad_x_out, const void* grad_z_out, const void* x_out, const void* dz,
                        const void* beta, const void* alpha_next, void* grad_x, void* grad_dz, void* grad_beta,
                        void* grad_alpha_next, int64_t batch, int grid, int cell, int channels,
                        const int32_t* index, int dtype, int w_dtype, void* workspace, size_t workspace_bytes,
                        void* stream) {
  return event_backward_impl("sihc_event_backward", grad_x_out, grad_z_out, x_out, dz, beta, alpha_next, grad_x,
                             grad_dz, grad_beta, grad_alpha_next, batch, grid, cell, channels, index, dtype, w_dtype,
                             workspace, workspace_bytes, stream);
}

int sihc_event_backward_partial(const void* grad_x_out, const void* grad_z_out, const void* x_out, const void* dz,
                                const void* beta, const void* alpha_next, void* grad_x, void* grad_dz,
                                void* grad_beta, void* grad_alpha_next, int64_t batch, int grid, int cell,
                                int channels, const int32_t* index, int dtype, int w_dtype, void* workspace,
                                size_t workspace_bytes, int* info, void* stream) {
  const char* what = "sihc_event_backward_partial";
  if (!info) return fail(SIHC_ERR_INVALID, "%s: null info", what);
  return event_backward_impl(what, grad_x_out, grad_z_out, x_out, dz, beta, alpha_next, grad_x, grad_dz, grad_beta,
                             grad_alpha_next, batch, grid, cell, channels, index, dtype, w_dtype, workspace,
                             workspace_bytes, stream, info);
}

// [a, a + na) and [b, b + nb) share a byte
static bool overlaps(const void* a, size_t na, const void* b, size_t nb) {
  const uintptr_t x = reinterpret_cast<uintptr_t>(a), y = reinterpret_cast<uintptr_t>(b);
  return na && nb && x < y + nb && y < x + na;
}

int sihc_event_backward_chain(const void* grad_x_out, const void* grad_z_out, const void* x_out, const void* dz,
                              const void* beta, const void* alpha_next, void* grad_x, void* grad_dz, void* grad_beta,
                              void* grad_alpha_next, int64_t batch, int grid, int cell, int channels,
                              const int32_t* index, int dtype, int w_dtype, void* workspace, size_t workspace_bytes,
                              int* info, const void* prev_workspace, size_t prev_workspace_bytes,
                              const int* prev_info, void* prev_grad_beta, void* prev_grad_alpha_next,
                              void* stream) {
  const char* what = "sihc_event_backward_chain";
  if (!info) return fail(SIHC_ERR_INVALID, "%s: null info", what);
  if (!prev_workspace)  // nothing carried: sihc_event_backward_partial
    return event_backward_impl(what, grad_x_out, grad_z_out, x_out, dz, beta, alpha_next, grad_x, grad_dz,
                               grad_beta, grad_alpha_next, batch, grid, cell, channels, index, dtype, w_dtype,
                               workspace, workspace_bytes, stream, info);
  if (!prev_info) return fail(SIHC_ERR_INVALID, "%s: null prev_info", what);
  if (cell != 2 && cell != 4) return fail(SIHC_ERR_INVALID, "%s: cell must be 2 or 4 (4 or 16 slots)", what);
  if (channels <= 0) return fail(SIHC_ERR_INVALID, "%s: bad sizes", what);
  const int chunks = prev_info[0], rows = prev_info[1];
  if (chunks < 0 || rows < 0 || rows > 3) return fail(SIHC_ERR_INVALID, "%s: bad prev_info", what);
  const int S = cell * cell;
  const size_t wbytes = size_t(S) * channels * elem_size(w_dtype);
  const size_t prev_bytes = size_t(chunks) * 2 * S * channels * sizeof(float);
  EvCarry cy{};
  if (chunks > 0 && rows > 0) {
    if (((rows & 1) && !prev_grad_beta) || ((rows & 2) && !prev_grad_alpha_next))
      return fail(SIHC_ERR_INVALID, "%s: null gradient of the carried call", what);
    if (prev_workspace_bytes < prev_bytes)
      return fail(SIHC_ERR_INVALID, "%s: prev_workspace holds %zu bytes, its %d partial rows need %zu", what,
                  prev_workspace_bytes, chunks, prev_bytes);
    if (!aligned(prev_workspace, 16)) return fail(SIHC_ERR_INVALID, "%s: prev_workspace must be 16-byte aligned", what);
    // the trailing blocks read prev_workspace and write the carried gradients while the
    // backward proper writes its own partial rows and gradients
    if (overlaps(prev_workspace, prev_bytes, workspace, workspace_bytes))
      return fail(SIHC_ERR_INVALID, "%s: prev_workspace overlaps this call's workspace", what);
    const void* mine[] = {grad_beta, grad_alpha_next};
    const void* theirs[] = {(rows & 1) ? prev_grad_beta : nullptr, (rows & 2) ? prev_grad_alpha_next : nullptr};
    for (const void* a : mine)
      for (const void* b : theirs)
        if (a && b && overlaps(a, wbytes, b, wbytes))
          return fail(SIHC_ERR_INVALID, "%s: the carried call's gradients overlap this call's", what);
    for (const void* b : theirs)
      if (b && overlaps(b, wbytes, workspace, workspace_bytes))
        return fail(SIHC_ERR_INVALID, "%s: the carried call's gradients overlap this call's workspace", what);
    cy.part = static_cast<const float*>(prev_workspace);
    cy.out0 = theirs[0] ? prev_grad_beta : nullptr;
    cy.out1 = theirs[1] ? prev_grad_alpha_next : nullptr;
    cy.chunks = chunks;
    cy.zero_mask = ((rows & 1) ? 0 : 1) | ((rows & 2) ? 0 : 2);  // rows without partials: not read
  }
  return event_backward_impl(what, grad_x_out, grad_z_out, x_out, dz, beta, alpha_next, grad_x, grad_dz, grad_beta,
                             grad_alpha_next, batch, grid, cell, channels, index, dtype, w_dtype, workspace,
                             workspace_bytes, stream, info, cy.part ? &cy : nullptr);
}

int sihc_event_finalize(int n, const void* const* workspaces, const size_t* workspace_bytes, const int* info,
                        void* const* grad_beta, void* const* grad_alpha_next, int cell, int channels, int w_dtype,
                        void* stream) {
  const char* what = "sihc_event_finalize";
  if (n < 0 || channels <= 0) return fail(SIHC_ERR_INVALID, "%s: bad sizes", what);
  if (cell != 2 && cell != 4) return fail(SIHC_ERR_INVALID, "%s: cell must be 2 or 4 (4 or 16 slots)", what);
  if (!valid_dtype(w_dtype)) return fail(SIHC_ERR_INVALID, "%s: bad dtype %d", what, w_dtype);
  if (n == 0) return SIHC_OK;
  if (!workspaces || !workspace_bytes || !info || !grad_beta || !grad_alpha_next)
    return fail(SIHC_ERR_INVALID, "%s: null array", what);
  const int S = cell * cell;
  // validate everything before the first launch
  for (int i = 0; i < n; ++i) {
    const int chunks = info[2 * i], rows = info[2 * i + 1];
    if (chunks < 0 || rows < 0 || rows > 3) return fail(SIHC_ERR_INVALID, "%s: bad info of event %d", what, i);
    if (chunks == 0 || rows == 0) continue;
    if (!workspaces[i]) return fail(SIHC_ERR_INVALID, "%s: null workspace of event %d", what, i);
    const size_t need = size_t(chunks) * 2 * S * size_t(channels) * sizeof(float);
    if (workspace_bytes[i] < need)
      return fail(SIHC_ERR_INVALID, "%s: workspace of event %d holds %zu bytes, its %d partial rows need %zu", what,
                  i, workspace_bytes[i], chunks, need);
    if (!aligned(workspaces[i], 16)) return fail(SIHC_ERR_INVALID, "%s: workspace of event %d misaligned", what, i);
    if (((rows & 1) && !grad_beta[i]) || ((rows & 2) && !grad_alpha_next[i]))
      return fail(SIHC_ERR_INVALID, "%s: null gradient of event %d", what, i);
  }
  hipStream_t st = static_cast<hipStream_t>(stream);
  const unsigned bx = unsigned((int64_t(2) * S * channels + EV_CARRY_OUTPUTS_PER_BLOCK - 1) /
                               EV_CARRY_OUTPUTS_PER_BLOCK);  // FINALIZE_FO x 4 outputs per block
  for (int i0 = 0; i0 < n; i0 += SIHC_FINALIZE_BATCH) {
    FinalizeBatch b{};
    int nb = 0;
    for (int i = i0; i < std::min(n, i0 + SIHC_FINALIZE_BATCH); ++i) {
      const int chunks = info[2 * i], rows = info[2 * i + 1];
      if (chunks == 0 || rows == 0) continue;
      b.part[nb] = static_cast<const float*>(workspaces[i]);
      b.out0[nb] = (rows & 1) ? grad_beta[i] : nullptr;
      b.out1[nb] = (rows & 2) ? grad_alpha_next[i] : nullptr;
      b.chunks[nb] = chunks;
      b.zero_mask[nb] = ((rows & 1) ? 0 : 1) | ((rows & 2) ? 0 : 2);  // rows without partials: not read
      ++nb;
    }
    if (nb == 0) continue;
    if (w_dtype == SIHC_DTYPE_F32) {
      hipLaunchKernelGGL((k_finalize_batch<float>), dim3(bx, unsigned(nb)), dim3(256), 0, st, b, S, channels);
    } else {
      hipLaunchKernelGGL((k_finalize_batch<bf16_t>), dim3(bx, unsigned(nb)), dim3(256), 0, st, b, S, channels);
    }
    if (int rc = check_launch(what)) return rc;
  }
  return SIHC_OK;
}

int sihc_event_backward_noalloc(const void* grad_x_out, const void* grad_z_out, const void* x_out, const void* dz,
                                const void* beta, const void* alpha_next, void* grad_x, void* grad_dz,
                                void* grad_beta, void* grad_alpha_next, int64_t batch, int grid, int cell,
                                int channels, const int32_t* index, int dtype, int w_dtype, void* stream) {
  const char* what = "sihc_event_backward_noalloc";
  Geo g;
  if (int rc = check_geometry(what, batch, grid, cell, channels, &g)) return rc;
  // the partial rows the launch may use (its chunk count never exceeds this one)
  const size_t need = size_t(event_bwd_chunks(g.M, cell)) * 2 * cell * cell * size_t(channels) * sizeof(float);
  if (need > size_t(SIHC_SCRATCH_BYTES))
    return fail(SIHC_ERR_INVALID,
                "%s: these sizes need %zu bytes of reduction scratch, more than the %zu-byte array this entry point "
                "holds per GPU; use sihc_event_backward with a workspace",
                what, need, size_t(SIHC_SCRATCH_BYTES));
  void* ptr = nullptr;
  if (g.M > 0)
    if (int rc = scratch_address(what, &ptr)) return rc;
  // same checks, kernels and reduction order as sihc_event_backward, with the scratch
  // array as its workspace
  return event_backward_impl(what, grad_x_out, grad_z_out, x_out, dz, beta, alpha_next, grad_x, grad_dz, grad_beta,
                             grad_alpha_next, batch, grid, cell, channels, index, dtype, w_dtype, ptr,
                             size_t(SIHC_SCRATCH_BYTES), stream);
}

int sihc_gather_cells(const void* x, const int32_t* index, void* cells, int64_t batch, int grid, int cell,
                      int channels, int dtype, void* stream) {
  return cells_copy("sihc_gather_cells", true, x, index, cells, batch, grid, cell, channels, dtype, stream);
}

int sihc_scatter_cells(const void* cells, const int32_t* index, void* x, int64_t batch, int grid, int cell,
                       int channels, int dtype, void* stream) {
  return cells_copy("sihc_scatter_cells", false, cells, index, x, batch, grid, cell, channels, dtype, stream);
}

int sihc_scatter_add_cells(const void* cells, const int32_t* index, void* x, int64_t batch, int grid, int cell,
                           int channels, int dtype, void* stream) {
  return cells_add("sihc_scatter_add_cells", cells, index, x, batch, grid, cell, channels, dtype, stream);
}

int sihc_stream(const void* const* src, int nsrc, void* const* dst, int ndst, size_t bytes, int shape,
                void* stream) {
  const char* what = "sihc_stream";
  if (bytes == 0) return SIHC_OK;
  if ((nsrc > 0 && !src) || !dst) return fail(SIHC_ERR_INVALID, "%s: null array", what);
  if (bytes % 4096) return fail(SIHC_ERR_INVALID, "%s: bytes must be a multiple of 4096", what);
  if (shape < 0 || shape > 2) return fail(SIHC_ERR_INVALID, "%s: shape must be 0, 1 or 2", what);
  if (shape == 0 && !((nsrc == 0 && ndst == 1) || (nsrc == 1 && ndst == 1) || (nsrc == 2 && ndst == 1) ||
                      (nsrc == 2 && ndst == 2) || (nsrc == 4 && ndst == 2)))
    return fail(SIHC_ERR_INVALID, "%s: unsupported mix %d:%d (0:1, 1:1, 2:1, 2:2, 4:2)", what, nsrc, ndst);
  if (shape == 1 && !(nsrc == 2 && ndst == 2))
    return fail(SIHC_ERR_INVALID, "%s: shape 1 takes 2 sources and 2 destinations", what);
  if (shape == 2 && !(nsrc == 4 && ndst == 2))
    return fail(SIHC_ERR_INVALID, "%s: shape 2 takes 4 sources and 2 destinations", what);
  for (int i = 0; i < nsrc; ++i)
    if (!src[i] || !aligned(src[i], 16)) return fail(SIHC_ERR_INVALID, "%s: source %d null or misaligned", what, i);
  for (int i = 0; i < ndst; ++i)
    if (!dst[i] || !aligned(dst[i], 16)) return fail(SIHC_ERR_INVALID, "%s: destination %d null or misaligned", what, i);
  PtrPack ps{}, pd{};
  for (int i = 0; i < nsrc; ++i) ps.p[i] = src[i];
  for (int i = 0; i < ndst; ++i) pd.p[i] = dst[i];
  const int64_t units = int64_t(bytes / 4096);
  if (units > 0x7fffffff) return fail(SIHC_ERR_INVALID, "%s: too many units", what);
  hipStream_t st = static_cast<hipStream_t>(stream);
  auto go = [&](auto kern) {
    hipLaunchKernelGGL(kern, dim3(unsigned(units)), dim3(256), 0, st, ps, pd, units);
    return check_launch(what);
  };
  if (shape == 1) return go(k_stream<2, 2, 1, 1>);  // x, dz -> x_out, z_out
  if (shape == 2) return go(k_stream<4, 2, 2, 1>);  // grad x_out, x_out, grad z_out, dz -> grad x, grad dz
  if (nsrc == 1 && ndst == 1) return go(k_stream<1, 1, 0, 0>);
  if (nsrc == 2 && ndst == 1) return go(k_stream<2, 1, 0, 0>);
  if (nsrc == 2 && ndst == 2) return go(k_stream<2, 2, 0, 0>);
  if (nsrc == 4 && ndst == 2) return go(k_stream<4, 2, 0, 0>);
  return go(k_stream<0, 1, 0, 0>);
}

int sihc_fma_rate(void* out, int chains, int form, int blocks, int iters, void* stream) {
  const char* what = "sihc_fma_rate";
  if (chains != 4 && chains != 8 && chains != 16) return fail(SIHC_ERR_INVALID, "%s: chains must be 4, 8 or 16", what);
  if (form < 0 || form > 3) return fail(SIHC_ERR_INVALID, "%s: form must be 0..3", what);
  if (blocks < 1 || iters < 1) return fail(SIHC_ERR_INVALID, "%s: blocks and iters must be positive", what);
  if (!out || !aligned(out, 4)) return fail(SIHC_ERR_INVALID, "%s: null or misaligned output", what);
  hipStream_t st = static_cast<hipStream_t>(stream);
  float* o = static_cast<float*>(out);
  // bf16 pairs (0.5, 0.25) . (0.5, 0.5): each dot2 step adds exactly 0.375
  const uint32_t pa = 0x3e803f00u, pb = 0x3f003f00u;
  auto go = [&](auto ch) {
    constexpr int CH = decltype(ch)::value;
    if (form == 0)
      hipLaunchKernelGGL((k_fma_chains<CH, 0>), dim3(blocks), dim3(256), 0, st, o, iters, 1.0000001f, 1e-7f, pa, pb);
    else if (form == 1)
      hipLaunchKernelGGL((k_fma_chains<CH, 1>), dim3(blocks), dim3(256), 0, st, o, iters, 1.0000001f, 1e-7f, pa, pb);
    else if (form == 2)
      hipLaunchKernelGGL((k_fma_chains<CH, 2>), dim3(blocks), dim3(256), 0, st, o, iters, 1.0000001f, 1e-7f, pa, pb);
    else
      hipLaunchKernelGGL((k_fma_chains<CH, 3>), dim3(blocks), dim3(256), 0, st, o, iters, 1.0000001f, 1e-7f, pa, pb);
  };
  if (chains == 4) go(IC<4>{});
  else if (chains == 8) go(IC<8>{});
  else go(IC<16>{});
  return check_launch(what);
}

int sihc_stream_mix(const void* const* src, int nsrc, int ncar_src, void* const* dst, int ndst, int ncar_dst,
                    int slots, size_t bytes, void* sink, void* stream) {
  const char* what = "sihc_stream_mix";
  if (bytes == 0) return SIHC_OK;
  if (nsrc < 0 || nsrc > SIHC_MAX_EVENTS || ndst < 0 || ndst > SIHC_MAX_EVENTS || nsrc + ndst == 0)
    return fail(SIHC_ERR_INVALID, "%s: %d sources and %d destinations (0..%d each, not both 0)", what, nsrc, ndst,
                SIHC_MAX_EVENTS);
  if (ncar_src < 0 || ncar_src > nsrc || ncar_dst < 0 || ncar_dst > ndst)
    return fail(SIHC_ERR_INVALID, "%s: carrier-shaped counts %d / %d exceed the array counts", what, ncar_src,
                ncar_dst);
  if (slots != 1 && slots != 4 && slots != 16) return fail(SIHC_ERR_INVALID, "%s: slots must be 1, 4 or 16", what);
  if (bytes % 4096) return fail(SIHC_ERR_INVALID, "%s: bytes must be a multiple of 4096", what);
  if ((nsrc > 0 && !src) || (ndst > 0 && !dst)) return fail(SIHC_ERR_INVALID, "%s: null array", what);
  for (int i = 0; i < nsrc; ++i)
    if (!src[i] || !aligned(src[i], 16)) return fail(SIHC_ERR_INVALID, "%s: source %d null or misaligned", what, i);
  for (int i = 0; i < ndst; ++i)
    if (!dst[i] || !aligned(dst[i], 16)) return fail(SIHC_ERR_INVALID, "%s: destination %d null or misaligned", what, i);
  if (ndst == 0 && (!sink || !aligned(sink, 16)))
    return fail(SIHC_ERR_INVALID, "%s: a read-only mix needs a 16-byte aligned sink", what);
  const int64_t units = int64_t(bytes / 4096);
  if (units > 0x7fffffff) return fail(SIHC_ERR_INVALID, "%s: too many units", what);
  PtrPack ps{}, pd{};
  for (int i = 0; i < nsrc; ++i) ps.p[i] = src[i];
  for (int i = 0; i < ndst; ++i) pd.p[i] = dst[i];
  hipLaunchKernelGGL(k_stream_mix, dim3(unsigned(units)), dim3(256), 0, static_cast<hipStream_t>(stream), ps, nsrc,
                     ncar_src, pd, ndst, ncar_dst, slots, units, static_cast<u32x4*>(ndst == 0 ? sink : nullptr));
  return check_launch(what);
}

int sihc_copy(const void* src, void* dst, size_t bytes, void* stream) {
  const char* what = "sihc_copy";
  if (bytes == 0) return SIHC_OK;
  if (!src || !dst) return fail(SIHC_ERR_INVALID, "%s: null pointer", what);
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (aligned(src, 16) && aligned(dst, 16) && bytes % 16 == 0) {
    const int64_t n = int64_t(bytes / 16);
    int64_t blocks = (n + 255) / 256;
    if (blocks > 256 * 64) blocks = 256 * 64;
    hipLaunchKernelGGL(k_copy16, dim3(unsigned(blocks)), dim3(256), 0, st, static_cast<const u32x4*>(src),
                       static_cast<u32x4*>(dst), n);
  } else {
    const int64_t n = int64_t(bytes);
    hipLaunchKernelGGL(k_copy1, dim3(unsigned((n + 255) / 256)), dim3(256), 0, st, static_cast<const uint8_t*>(src),
                       static_cast<uint8_t*>(dst), n);
  }
  return check_launch(what);
}

}  // extern "C"
