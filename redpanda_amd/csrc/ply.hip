// Host boundary of one lockstep rollout ply, on the device side: what the
// reference moves to the host row by row (engine/mars_search.py:262, the
// continuation row of every rollout; :475, the logits of a rollout's legal
// moves; :446 / :556, the rollout values) is reduced and packed here, so one
// copy per ply carries it.
//
//   ply_topk:   per rollout row, the k largest logits with their token ids
//               (descending; equal values by ascending id) and the value;
//   ply_gather: per rollout, the logits of a padded list of token ids.
//
// ply_topk: one wave per row.  Lane l reads elements l, l + 64, ... (every
// load coalesced) and keeps its own k largest as sorted 64-bit keys
//     key = (order-preserving bits of the fp32 logit) << 32 | ~id,
// so a larger key is a larger logit, or the smaller id of equal logits.  The
// first block fills the lists with a sorting network; after it, a wave-wide
// lower bound on the row's k-th logit (from a sort of the lane maxima across
// the wave) lets most elements skip the insert after one float compare.  The lanes' lists are then merged: k rounds of a wave max
// over the lanes' heads, the winning lane shifting its list.  V logits are
// read once per row.

#include <type_traits>

#include "rp_device.h"
#include "rp_launch.h"

namespace rp {

namespace {

// fp32 bits -> uint32 whose unsigned order is numpy's order of the floats,
// which the reference's argpartition / argsort apply: -inf < ... < +inf <
// NaN, with -0 equal to +0 and every NaN above +inf whatever its sign.  The
// key is that of the canonical value (+0 for -0, the NaN with its sign bit
// cleared), so equal values tie and fall to the id order; key_value gives
// the canonical value back.
__device__ __forceinline__ uint32_t order_key(float v) {
  uint32_t b = __float_as_uint(v);
  if ((b & 0x7fffffffu) > 0x7f800000u) b &= 0x7fffffffu;  // NaN of either sign
  if (b == 0x80000000u) b = 0u;                           // -0
  return b ^ ((b & 0x80000000u) ? 0xffffffffu : 0x80000000u);
}
__device__ __forceinline__ float key_value(uint32_t k) {
  return __uint_as_float(k ^ ((k & 0x80000000u) ? 0x80000000u : 0xffffffffu));
}

// Exchanges of a 64-bit value across lanes by DPP, within rows of 16 lanes.
template <int kCtrl>
__device__ __forceinline__ uint64_t dpp_u64(uint64_t v) {
  const uint32_t lo = __builtin_amdgcn_mov_dpp((int)(uint32_t)v, kCtrl, 0xf, 0xf, false);
  const uint32_t hi = __builtin_amdgcn_mov_dpp((int)(uint32_t)(v >> 32), kCtrl, 0xf, 0xf, false);
  return ((uint64_t)hi << 32) | lo;
}
__device__ __forceinline__ uint64_t max_u64(uint64_t a, uint64_t b) { return a > b ? a : b; }

// The wave's largest value, the same in every lane: within each row of 16
// lanes, lane i meets lane i ^ 1, i ^ 2 (quad permutes), 7 - i within its 8
// and 15 - i within its 16 (mirrors); then the four rows' maxima are read
// into scalars.  No LDS round trip, unlike a shuffle.
__device__ __forceinline__ uint64_t wave_max_u64(uint64_t w) {
  w = max_u64(w, dpp_u64<0xb1>(w));   // quad_perm [1, 0, 3, 2]
  w = max_u64(w, dpp_u64<0x4e>(w));   // quad_perm [2, 3, 0, 1]
  w = max_u64(w, dpp_u64<0x141>(w));  // row_half_mirror
  w = max_u64(w, dpp_u64<0x140>(w));  // row_mirror
  uint64_t m = 0;
#pragma unroll
  for (int r = 0; r < kWave; r += 16) {
    const uint32_t lo = __builtin_amdgcn_readlane((int)(uint32_t)w, r);
    const uint32_t hi = __builtin_amdgcn_readlane((int)(uint32_t)(w >> 32), r);
    m = max_u64(m, ((uint64_t)hi << 32) | lo);
  }
  return m;
}

// A logit as fp32, the storage dtype fixed at compile time (a run-time
// dtype branch per load would serialise the loads in flight).
template <int DT>
__device__ __forceinline__ float load_logit(const void* p, int64_t i) {
  if constexpr (DT == RP_F32) {
    return static_cast<const float*>(p)[i];
  } else if constexpr (DT == RP_BF16) {
    return __uint_as_float((uint32_t)static_cast<const uint16_t*>(p)[i] << 16);
  } else {
    return static_cast<float>(static_cast<const _Float16*>(p)[i]);
  }
}

}  // namespace

// KL: list length (k <= KL); each lane holds its KL largest keys, l[0] first.
// Key 0 is below every element's key (an element's id part ~id is nonzero).
constexpr int kPlyUnroll = 16;

template <int KL, int DT>
__global__ __launch_bounds__(kThreads) void ply_topk_kernel(PlyTopkParams p) {
  const int lane = threadIdx.x % kWave;
  const int64_t row = (int64_t)blockIdx.x * kWaves + threadIdx.x / kWave;
  if (row >= p.R) return;
  uint64_t l[KL];
#pragma unroll
  for (int j = 0; j < KL; ++j) l[j] = 0;
  const int64_t base = row * p.lsr;
  // thr: the KL-th largest logit among the lanes' largest keys.  KL
  // distinct elements (those lane maxima) have that logit or a larger one,
  // so no element with a smaller logit is among the row's k <= KL largest.  thr_f, its logit, filters elements
  // with one float compare: one below it can be skipped (a NaN or a logit
  // equal to it takes the exact 64-bit test).
  uint64_t thr = 0;
  float thr_f = -__builtin_inff();
  constexpr int kBlock = kWave * kPlyUnroll;
  // full blocks: unconditional loads at one address plus immediate offsets;
  // the last, partial block: loads masked by the row length (0 beyond it)
  auto load_full = [&](int i0, float (&v)[kPlyUnroll]) {
#pragma unroll
    for (int u = 0; u < kPlyUnroll; ++u) v[u] = load_logit<DT>(p.logits, base + i0 + lane + u * kWave);
  };
  auto load_part = [&](int i0, float (&v)[kPlyUnroll]) {
#pragma unroll
    for (int u = 0; u < kPlyUnroll; ++u) {
      const int i = i0 + u * kWave + lane;
      v[u] = i < p.V ? load_logit<DT>(p.logits, base + i) : 0.f;
    }
  };
  int nb = 0;  // blocks taken
  auto take_block = [&](auto full, auto first, int i0, const float (&v)[kPlyUnroll]) {
    constexpr bool kFull = decltype(full)::value;
    // ~id of the block's slot u is idb - 64 u.  The empty asm makes idb
    // opaque, so the compiler rebuilds each slot's id with one subtract
    // instead of keeping 16 per-slot 64-bit constants live across the loop.
    uint32_t idb = ~(uint32_t)(i0 + lane);
    asm volatile("" : "+v"(idb));
    if constexpr (decltype(first)::value) {
      // the first block fills the (empty) lists: its keys sorted, largest
      // first, by a bitonic network in registers (elements past V: key 0)
      static_assert(KL <= kPlyUnroll, "the first block fills the list");
      uint64_t x[kPlyUnroll];
#pragma unroll
      for (int u = 0; u < kPlyUnroll; ++u) {
        const int i = i0 + u * kWave + lane;
        x[u] = (kFull || i < p.V) ? ((uint64_t)order_key(v[u]) << 32) | (idb - (uint32_t)(u * kWave)) : 0;
      }
#pragma unroll
      for (int kk = 2; kk <= kPlyUnroll; kk <<= 1) {
#pragma unroll
        for (int j = kk >> 1; j > 0; j >>= 1) {
#pragma unroll
          for (int a = 0; a < kPlyUnroll; ++a) {
            const int b = a ^ j;
            if (b <= a) continue;
            // descending runs where a & kk == 0, ascending elsewhere, so
            // the last merge leaves the whole array descending
            const bool desc = (a & kk) == 0;
            const uint64_t lo = x[a] < x[b] ? x[a] : x[b];
            const uint64_t hi = x[a] < x[b] ? x[b] : x[a];
            x[a] = desc ? hi : lo;
            x[b] = desc ? lo : hi;
          }
        }
      }
#pragma unroll
      for (int j = 0; j < KL; ++j) l[j] = x[j];
    } else {
#pragma unroll
      for (int u = 0; u < kPlyUnroll; ++u) {
        const int i = i0 + u * kWave + lane;
        if (!kFull && i >= p.V) break;
        if (v[u] < thr_f) continue;
        uint64_t x = ((uint64_t)order_key(v[u]) << 32) | (idb - (uint32_t)(u * kWave));
        if (x > l[KL - 1] && x > thr) {
          // sorted insert: the larger of (slot, carry) stays, the smaller moves on
#pragma unroll
          for (int j = 0; j < KL; ++j) {
            const uint64_t hi = x > l[j] ? x : l[j];
            x = x > l[j] ? l[j] : x;
            l[j] = hi;
          }
        }
      }
    }
    // the bound is refreshed after blocks 1, 2, 4, 8, ...: it tightens
    // fastest early, and each refresh is a 21-stage exchange across the wave.
    // None after the row's last block: only the merge follows.
    const bool refresh = (nb & (nb + 1)) == 0 && i0 + kBlock < p.V;
    ++nb;
    if (!refresh) return;
    // bitonic sort of the lane maxima's logit keys (the upper halves; ids do
    // not matter for a bound) across the wave, ascending by lane; the KL-th
    // largest is lane 64 - KL's.  thr keeps every element with that logit
    // or a larger one (its id half is zero, below any element's)
    uint32_t w = (uint32_t)(l[0] >> 32);
#pragma unroll
    for (int kk = 2; kk <= kWave; kk <<= 1) {
#pragma unroll
      for (int j = kk >> 1; j > 0; j >>= 1) {
        const uint32_t o = __shfl_xor(w, j);
        const bool keep_min = ((lane & j) == 0) == ((lane & kk) == 0);
        w = keep_min ? min(o, w) : max(o, w);
      }
    }
    const uint32_t thi = __shfl(w, kWave - KL);
    thr = (uint64_t)thi << 32;
    if (thi != 0) thr_f = key_value(thi);
  };
  // A row is one wave's serial walk, so its memory latency is covered by
  // loads in flight: kPlyUnroll per lane, and the next block's loads issued
  // before the current block is taken (two register buffers, alternating).
  // The full blocks' loads carry no per-lane condition, so the loads of one
  // block stay in flight while the other block is taken.
  const std::integral_constant<bool, true> full, first;
  const std::integral_constant<bool, false> part, rest;
  const int nfull = p.V / kBlock;
  float va[kPlyUnroll], vb[kPlyUnroll];
  int b = 0;
  if (nfull > 0) {
    // the first block, taken out of the loop (the sorting network is the
    // largest code path; the loop holds only the filtered inserts)
    load_full(0, va);
    if (nfull > 1) load_full(kBlock, vb);
    take_block(full, first, 0, va);
    // block b is in vb on entry to each iteration
    for (b = 1; b + 1 < nfull; b += 2) {
      load_full((b + 1) * kBlock, va);
      take_block(full, rest, b * kBlock, vb);
      if (b + 2 < nfull) load_full((b + 2) * kBlock, vb);
      take_block(full, rest, (b + 1) * kBlock, va);
    }
    if (b < nfull) take_block(full, rest, (b++) * kBlock, vb);
  }
  if (b * kBlock < p.V) {
    load_part(b * kBlock, va);
    if (b == 0)
      take_block(part, first, 0, va);
    else
      take_block(part, rest, b * kBlock, va);
  }
  // merge: k rounds, each taking the largest head among the lanes
  float myv = -__builtin_inff();
  int myi = -1;
  for (int m = 0; m < p.k; ++m) {
    const uint64_t w = wave_max_u64(l[0]);
    if (lane == m && w != 0) {
      myv = key_value((uint32_t)(w >> 32));
      myi = (int)~(uint32_t)w;
    }
    if (w != 0 && l[0] == w) {
#pragma unroll
      for (int j = 0; j + 1 < KL; ++j) l[j] = l[j + 1];
      l[KL - 1] = 0;
    }
  }
  uint32_t* out = static_cast<uint32_t*>(p.out) + row * p.osr;
  if (lane == 0) out[0] = p.values != nullptr ? __float_as_uint(p.values[row]) : 0u;
  if (lane < p.k) {
    out[1 + lane] = __float_as_uint(myv);
    out[1 + p.k + lane] = (uint32_t)myi;
  }
}

// out[r, j] = logits[r, tokens[r, j]] (fp32), -inf for ids outside [0, V).
__global__ __launch_bounds__(kThreads) void ply_gather_kernel(PlyGatherParams p) {
  const int64_t n = p.R * p.M;
  for (int64_t e = (int64_t)blockIdx.x * kThreads + threadIdx.x; e < n;
       e += (int64_t)gridDim.x * kThreads) {
    const int64_t r = e / p.M, j = e % p.M;
    const int32_t t = p.tokens[r * p.tsr + j];
    p.out[r * p.osr + j] =
        (t >= 0 && t < p.V) ? load_in(p.logits, r * p.lsr + t, p.dt) : -__builtin_inff();
  }
}

hipError_t launch_ply_topk(const PlyTopkParams& p, hipStream_t st) {
  if (p.R == 0) return hipSuccess;
  const dim3 grid((unsigned)((p.R + kWaves - 1) / kWaves));
  auto go = [&](auto dt_tag) {
    constexpr int DT = decltype(dt_tag)::value;
    if (p.k <= 8)
      hipLaunchKernelGGL((ply_topk_kernel<8, DT>), grid, dim3(kThreads), 0, st, p);
    else
      hipLaunchKernelGGL((ply_topk_kernel<kPlyMaxK, DT>), grid, dim3(kThreads), 0, st, p);
  };
  if (p.dt == RP_F32)
    go(std::integral_constant<int, RP_F32>{});
  else if (p.dt == RP_BF16)
    go(std::integral_constant<int, RP_BF16>{});
  else
    go(std::integral_constant<int, RP_F16>{});
  return hipGetLastError();
}

hipError_t launch_ply_gather(const PlyGatherParams& p, hipStream_t st) {
  const int64_t n = p.R * p.M;
  if (n == 0) return hipSuccess;
  const int64_t blocks = (n + kThreads - 1) / kThreads;
  hipLaunchKernelGGL(ply_gather_kernel, dim3((unsigned)(blocks < 4096 ? blocks : 4096)),
                     dim3(kThreads), 0, st, p);
  return hipGetLastError();
}

}  // namespace rp
