// scaled_quantize, quant_mode "dynamic_per_token", for gfx950: optional row gather, optional
// (per-group) smooth vector, per-row amax -> fp32 scale -> int8 codes.
//
// Semantics: reference _ops.py:3126-3253 (moe_quantize; math block :3147-3176) and
// _ops.py:4407-4492 (scaled_quantize).  Entry point: tmo_hip_scaled_quantize_per_token
// (include/tmo_hip.h).
//
// One or two wavefronts per output row, or one workgroup per row.  Every lane holds its
// 16-byte vectors of the row in registers (all loads in flight at once), so the row is read
// from HBM exactly once.  sq_dense_wg: rows without gather or groups of 256 * k vectors, one
// row per workgroup at a time in a persistent grid, the smooth values of a thread's channels in
// registers.  sq_dense: other dense rows, a grid-stride launch with a per-channel smooth vector
// staged in LDS.  sq_grp: gathered / grouped rows (MoE) with per-channel smooth rows,
// one staging of the group's smooth row in LDS per workgroup.  sq_vec: the remaining vector
// cases (other widths, 3-D rows, scalar or no smooth with gather / groups), the smooth vector
// read from L2 beside the row.  A row's group (expert) is found with a wavefront prefix scan
// of token_count and a ballot, with no host round trip.
#include <algorithm>

#include "tmo_device.h"

namespace tmo {
namespace {

struct SqParams {
  const void* x;
  int64_t n0;
  int64_t inner;
  int64_t channels;
  int64_t row_stride;  // elements
  int8_t* out;
  float* out_scale;
  const float* smooth;
  int64_t smooth_len;  // 1 or channels (0: no smooth)
  const int32_t* token_count;
  int64_t num_groups;
  const int32_t* gather_index;
  int64_t gather_len;
  const int32_t* gather_start;
  int64_t out_rows;
  int64_t total_rows;  // out_rows * inner
  int64_t dense_rows;  // min(out_rows, n0) * inner: rows produced without gather / groups
  int64_t grp_main;    // sq_grp: workgroups of the row-major part of the grid
};

// Group of row r: the g with prefix(g) <= r < prefix(g + 1) over token_count.  Returns
// false when r >= sum(token_count).  Wave-uniform.  `first` is this lane's token_count entry
// of the first 64 groups, loaded by the caller together with the row's other indices.
__device__ __forceinline__ bool find_group(const SqParams& p, int64_t r, int32_t first,
                                           int64_t& g) {
  const int lane = threadIdx.x & (kWave - 1);
  int64_t carry = 0, below = 0;
  for (int64_t base = 0; base < p.num_groups; base += kWave) {
    const int64_t k = base + lane;
    int64_t c = base == 0 ? (int64_t)first : (k < p.num_groups ? (int64_t)p.token_count[k] : 0);
    // inclusive scan across the wavefront
#pragma unroll
    for (int o = 1; o < kWave; o <<= 1) {
      const int64_t n = __shfl_up(c, o, kWave);
      if (lane >= o) c += n;
    }
    const int64_t incl = carry + c;
    const uint64_t le = __ballot(k < p.num_groups && incl <= r);
    below += __popcll(le);
    carry += __shfl(c, kWave - 1, kWave);
  }
  g = below;
  return r < carry;
}

// Source row and group of output row r (both wave-uniform): the gather-index load and the
// first token_count load are issued together.  False when the row is not produced.
__device__ __forceinline__ bool locate_row(const SqParams& p, int64_t r, int64_t& src,
                                           int64_t& g) {
  const int lane = threadIdx.x & (kWave - 1);
  int32_t tc0 = 0;
  if (p.token_count && lane < p.num_groups) tc0 = p.token_count[lane];
  src = r;
  if (p.gather_index) {
    const int64_t gi = (p.gather_start ? (int64_t)p.gather_start[0] : 0) + r;
    if (gi < 0 || gi >= p.gather_len) return false;
    src = p.gather_index[gi];
  }
  if (src < 0 || src >= p.n0) return false;
  g = 0;
  if (p.token_count && !find_group(p, r, tc0, g)) return false;
  return true;
}

#ifndef TMO_SQ_LDS_SMOOTH
#define TMO_SQ_LDS_SMOOTH 1
#endif
// Workgroups per CU of the dense kernel's grid-stride launch (0: one workgroup per 4 rows).
// configs[3] (8192 x 4096 bf16) on MI355X, per-channel / scalar / no smooth: one-shot grid
// 22.9 / 19.4 / 19.2 us; 1: 24.9 / 23.9 / 23.2; 2: 19.6 / 18.9 / 18.8; 3: 19.4 / 18.8 / 18.7;
// 6: 20.2 / 19.7 / 19.5 (with the smooth vector staged in LDS).
#ifndef TMO_SQ_WG_PER_CU
#define TMO_SQ_WG_PER_CU 3
#endif
#ifndef TMO_SQ_WAVES_PER_ROW
#define TMO_SQ_WAVES_PER_ROW 2
#endif

// Vector path: channels % kPerVec == 0, 16-byte aligned rows and smooth, and
// channels / kPerVec <= 64 * kWPR * kMaxV.  A row is kWPR wavefronts (lanes take 16-byte
// vectors lane + 64 * (part + kWPR * i)); two wavefronts per row (amax combined through LDS)
// serve rows too long for one wavefront's registers.  kStream: the rows are read
// exactly once (no gather), so they are loaded non-temporally; a gathered row may be read
// again for another output row (MoE top-k), and then the cached load lets the repeat hit
// L2 / MALL.
template <class Tag, int kMaxV, bool kStream, int kWPR>
__global__ __launch_bounds__(256) void sq_vec(SqParams p) {
  constexpr int kPer = Tag::kPerVec;
  constexpr int kRowsPerWG = 4 / kWPR;
  __shared__ uint32_t red[4];
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
  const int part = wave % kWPR;
  const int64_t orow = (int64_t)blockIdx.x * kRowsPerWG + wave / kWPR;
  // 2-D inputs (inner == 1, the common case) skip the 64-bit division
  const int64_t r = p.inner == 1 ? orow : orow / p.inner;
  const int64_t jn = orow - r * p.inner;
  int64_t src = 0, g = 0;
  const bool valid = orow < p.total_rows && locate_row(p, r, src, g);  // wave-uniform
  if (kWPR == 1 && !valid) return;

  const int64_t nvec = p.channels / kPer;
  const char* xrow = static_cast<const char*>(p.x) + (src * p.inner + jn) * p.row_stride * Tag::kBytes;
  const float* sm = p.smooth ? p.smooth + (p.token_count ? g * p.smooth_len : 0) : nullptr;
  const bool per_channel = sm && p.smooth_len != 1;
  // Issue every load of the row -- x vectors and the matching smooth vectors -- before the
  // first wait, so the row costs one HBM round trip plus one L2 round trip, overlapped.
  u32x4 w[kMaxV];
  u32x4 sv[kMaxV][kPer / 4];
#pragma unroll
  for (int i = 0; i < kMaxV; ++i) {
    const int64_t u = lane + (int64_t)(part + kWPR * i) * kWave;
    if (valid && u < nvec) {
      const u32x4* xp = reinterpret_cast<const u32x4*>(xrow + u * 16);
      if constexpr (kStream) {
        w[i] = __builtin_nontemporal_load(xp);
      } else {
        w[i] = *xp;
      }
      if (per_channel) {
        const u32x4* sp = reinterpret_cast<const u32x4*>(sm + u * kPer);
#pragma unroll
        for (int q = 0; q < kPer / 4; ++q) sv[i][q] = sp[q];
      }
    }
  }
  const float s_scalar = (sm && !per_channel) ? sm[0] : 1.0f;
  float v[kMaxV][kPer];
  float m = 0.0f;
#pragma unroll
  for (int i = 0; i < kMaxV; ++i) {
    const int64_t u = lane + (int64_t)(part + kWPR * i) * kWave;
    if (valid && u < nvec) {
      unpack(Tag{}, w[i], v[i]);
      if (per_channel) {
#pragma unroll
        for (int e = 0; e < kPer; ++e) v[i][e] = v[i][e] * __uint_as_float(sv[i][e / 4][e % 4]);
      } else if (sm) {
#pragma unroll
        for (int e = 0; e < kPer; ++e) v[i][e] = v[i][e] * s_scalar;  // RN(x * smooth), no FMA
      }
#pragma unroll
      for (int e = 0; e < kPer; ++e) m = abs_max(m, v[i][e]);
    }
  }
  uint32_t mb = group_max_u32<kWave>(__float_as_uint(m));
  if constexpr (kWPR > 1) {
    if (lane == 0) red[wave] = mb;
    __syncthreads();
    const int first = wave - part;
#pragma unroll
    for (int k = 0; k < kWPR; ++k) mb = max(mb, red[first + k]);
    if (!valid) return;
  }
  const RowScale rs = make_row_scale(__uint_as_float((uint32_t)__builtin_amdgcn_readfirstlane((int)mb)));
  int8_t* orow_ptr = p.out + orow * p.channels;
#pragma unroll
  for (int i = 0; i < kMaxV; ++i) {
    const int64_t u = lane + (int64_t)(part + kWPR * i) * kWave;
    if (u < nvec) {
      uint32_t c[kPer / 4];
      encode_row<kPer>(v[i], rs, c);
      if constexpr (kPer == 8) {
        u32x2 c2;
        c2[0] = c[0];
        c2[1] = c[1];
        store_nt(reinterpret_cast<u32x2*>(orow_ptr + u * 8), c2);
      } else {
        store_nt(reinterpret_cast<uint32_t*>(orow_ptr + u * 4), c[0]);
      }
    }
  }
  if (lane == 0 && part == 0) p.out_scale[orow] = rs.s;
}

// Smooth values (u32x4 quarter q of vector i of this lane) from a staged LDS row (lane-major,
// see sq_grp).
template <int kSV>
struct SmoothLds {
  const u32x4* lds;
  int lane;
  __device__ __forceinline__ u32x4 operator()(int i, int q) const {
    return lds[(i * kSV + q) * kWave + lane];
  }
};

// One row of 64 * kV 16-byte vectors (this lane's vectors lane + 64 * i in w) -> smoothed
// int8 codes (RN(x * smooth) per element, no FMA) and the row scale.
template <class Tag, int kV, class SmoothAt>
__device__ __forceinline__ void quant_row(const u32x4 (&w)[kV], SmoothAt sm, int8_t* orow,
                                             float* scale_out, int lane) {
  constexpr int kPer = Tag::kPerVec;
  constexpr int kSV = kPer / 4;
  float v[kV][kPer];
  float mx = 0.0f;
#pragma unroll
  for (int i = 0; i < kV; ++i) {
    unpack(Tag{}, w[i], v[i]);
#pragma unroll
    for (int q = 0; q < kSV; ++q) {
      const u32x4 sv = sm(i, q);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        v[i][4 * q + e] = v[i][4 * q + e] * __uint_as_float(sv[e]);
        mx = abs_max(mx, v[i][4 * q + e]);
      }
    }
  }
  const RowScale rs = make_row_scale(wave_max_uniform(mx));
#pragma unroll
  for (int i = 0; i < kV; ++i) {
    uint32_t c[kPer / 4];
    encode_row<kPer>(v[i], rs, c);
    if constexpr (kPer == 8) {
      u32x2 c2;
      c2[0] = c[0];
      c2[1] = c[1];
      store_nt(reinterpret_cast<u32x2*>(orow + i * kWave * 8), c2);
    } else {
      store_nt(reinterpret_cast<uint32_t*>(orow + i * kWave * 4), c[0]);
    }
  }
  if (lane == 0) *scale_out = rs.s;
}

#ifndef TMO_SQ_GRP_WAVES
#define TMO_SQ_GRP_WAVES 4
#endif

// Groups over token_count, wave-uniform results from one pass (a wavefront prefix scan per 64
// groups, a ballot per row): ga / gb = the first group whose inclusive prefix exceeds row a /
// row b (-1 when none: the row is at or past sum(token_count)); for group gq its exclusive and
// inclusive prefixes; total = sum(token_count).  `first` is this lane's entry of the first 64
// groups.  The whole wavefront must be active.
__device__ __forceinline__ void group_scan(const SqParams& p, int32_t first, int64_t a, int64_t b,
                                           int64_t gq, int64_t& ga, int64_t& gb,
                                           int64_t& q_excl, int64_t& q_incl, int64_t& total) {
  const int lane = threadIdx.x & (kWave - 1);
  int64_t carry = 0;
  ga = gb = -1;
  q_excl = q_incl = 0;
  for (int64_t base = 0; base < p.num_groups; base += kWave) {
    const int64_t k = base + lane;
    int64_t c = base == 0 ? (int64_t)first : (k < p.num_groups ? (int64_t)p.token_count[k] : 0);
    const int64_t own = c;
    // counts in [0, 2^25) sum to below 2^31 over 64 lanes: a 32-bit DPP scan; otherwise
    // (negative or huge counts) 64-bit lane shuffles
    if (!__ballot(c < 0 || c >= (1 << 25))) {
      c = (int64_t)wave_incl_sum_u32((uint32_t)c);
    } else {
#pragma unroll
      for (int o = 1; o < kWave; o <<= 1) {
        const int64_t n = __shfl_up(c, o, kWave);
        if (lane >= o) c += n;
      }
    }
    const int64_t incl = carry + c;
    const bool in = k < p.num_groups;
    const uint64_t ha = __ballot(in && incl > a);
    const uint64_t hb = __ballot(in && incl > b);
    if (ga < 0 && ha) ga = base + __builtin_ctzll(ha);
    if (gb < 0 && hb) gb = base + __builtin_ctzll(hb);
    if (gq >= base && gq < base + kWave) {
      const int f = (int)(gq - base);
      q_incl = __shfl(incl, f, kWave);
      q_excl = q_incl - __shfl(own, f, kWave);
    }
    carry += __shfl(c, kWave - 1, kWave);
  }
  total = carry;
}

// The part of sq_grp after the indices: stage smooth row g_stage in LDS, load row `src`, encode
// it into output row r when `valid`.  Every thread of the workgroup calls it (it holds a
// barrier).  The staging loads (L2 hits) are issued before the row loads: the memory counter
// is in order, so the LDS writes then wait for the staging data only, and the barrier does
// not wait for the slowest row of the workgroup to arrive from HBM.  The row loads are
// unconditional (a row that is not produced reads row 0, which exists since n0 > 0): under a
// branch, the wait before the LDS writes would have to assume the loads were issued on one
// path and not on the other, and would wait for them as well.
template <class Tag, int kV, int kW, bool kGather>
__device__ __forceinline__ void sq_grp_row(const SqParams& p, u32x4* lds, int64_t g_stage,
                                           int64_t r, int64_t src, bool valid) {
  constexpr int kPer = Tag::kPerVec;
  constexpr int kSV = kPer / 4;              // u32x4 of smooth values per x vector
  constexpr int kSlot = kV * kSV * kWave;    // u32x4 of one staged smooth row
  constexpr int kStage = (kSlot + kWave * kW - 1) / (kWave * kW);  // staged u32x4 per thread
  const int lane = threadIdx.x & (kWave - 1);
  const u32x4* sg = reinterpret_cast<const u32x4*>(p.smooth + g_stage * p.smooth_len);
  u32x4 st[kStage];
#pragma unroll
  for (int j = 0; j < kStage; ++j) {
    const int m = threadIdx.x + j * kWave * kW;
    const int i = m / (kSV * kWave), rem = m % (kSV * kWave);
    if (kSlot % (kWave * kW) == 0 || m < kSlot)
      st[j] = sg[(i * kWave + rem % kWave) * kSV + rem / kWave];
  }
  u32x4 w[kV];
  {
    const int64_t lsrc = valid ? src : 0;
    const char* xrow = static_cast<const char*>(p.x) + lsrc * p.row_stride * Tag::kBytes + lane * 16;
#pragma unroll
    for (int i = 0; i < kV; ++i) {
      const u32x4* xp = reinterpret_cast<const u32x4*>(xrow + i * kWave * 16);
      // a gathered row may be read again for another output row (top-k): cached loads let the
      // repeat hit L2 / MALL
      w[i] = kGather ? *xp : __builtin_nontemporal_load(xp);
    }
  }
#pragma unroll
  for (int j = 0; j < kStage; ++j) {
    const int m = threadIdx.x + j * kWave * kW;
    if (kSlot % (kWave * kW) == 0 || m < kSlot) lds[m] = st[j];
  }
  __syncthreads();
  if (!valid) return;
  quant_row<Tag, kV>(w, SmoothLds<kSV>{lds, lane}, p.out + r * p.channels + lane * kPer,
                     p.out_scale + r, lane);
}

// Gathered and / or grouped rows (MoE) with a per-channel smooth vector, rows of exactly
// 64 * kV 16-byte vectors, 2-D input, one output row per wavefront.  The grid has two parts.
//
// Row-major workgroups (blockIdx.x < grp_main) own rows [kW * b, kW * b + kW).  A wavefront
// issues its index loads (its gather index and its lane's token_count entry, together), finds
// the groups of its row and of the workgroup's first row with one DPP prefix scan, and the
// workgroup stages the smooth row of the first row's group in LDS and encodes the rows of that
// group.  Rows of a later group inside the workgroup (a group starting mid-workgroup: with
// expert-sorted rows, the moe_gen_idx order, at most kW - 1 rows per group) are left to the
// boundary workgroups, one per group (blockIdx.x = grp_main + g), which encode rows
// [excl_g, min(incl_g, kW * ceil(excl_g / kW))).  Every produced row is written by exactly one
// wavefront.
//
// From LDS the smooth row costs one staging per workgroup; read from L2 instead, every row
// fetches its whole smooth row -- twice the row's own bytes, and twice its vector loads.
// configs[3]-MoE on MI355X: 38.6 us with per-row L2 smooth reads (one wavefront per row,
// index and group lookups serialised in front of the row loads), 34.0 us here.  Measured and
// rejected: a fifth, staging-only wavefront per workgroup (37.0 us), 8 rows per workgroup
// (35.8 us), a two-pass encoder that keeps only the raw row (60 VGPRs, 8 waves per SIMD,
// 35.0 us).  A minimal kernel that only gathers and copies the same bytes takes 27.4 us.
template <class Tag, int kV, int kW, bool kGroups, bool kGather>
__global__ __launch_bounds__(64 * kW) void sq_grp(SqParams p) {
  constexpr int kSlot = kV * (Tag::kPerVec / 4) * kWave;
  // staged smooth row, lane-major: vector i, quarter q of lane l at (i * kSV + q) * 64 + l, so
  // a wavefront's 16-byte reads of one (i, q) are 64 consecutive vectors
  __shared__ u32x4 lds[kSlot];
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
  const int64_t gstart = (kGather && p.gather_start) ? (int64_t)p.gather_start[0] : 0;
  if (kGroups && blockIdx.x >= p.grp_main) {  // boundary workgroup (workgroup-uniform)
    const int32_t t = p.token_count[lane < p.num_groups ? lane : 0];
    const int32_t tc0 = lane < p.num_groups ? t : 0;
    const int64_t g = (int64_t)blockIdx.x - p.grp_main;
    int64_t unused, excl, incl, total;
    group_scan(p, tc0, 0, 0, g, unused, unused, excl, incl, total);
    const int64_t r = excl + wave;
    const int64_t aligned = (excl + kW - 1) / kW * kW;
    bool valid = r < incl && r < aligned && r < p.total_rows;
    int64_t src = r;
    if constexpr (kGather) {
      const int64_t gi = gstart + r;
      const bool in = gi >= 0 && gi < p.gather_len;
      src = p.gather_index[in ? gi : 0];
      valid = valid && in;
    }
    valid = valid && src >= 0 && src < p.n0;
    sq_grp_row<Tag, kV, kW, kGather>(p, lds, g, r, src, valid);
    return;
  }
  // Row-major workgroup.  The index loads come first, all unconditional (clamped in-bounds
  // addresses, masked afterwards), so they issue back to back and one wait covers them.
  int32_t tc0 = 0;
  if constexpr (kGroups) {
    const int32_t t = p.token_count[lane < p.num_groups ? lane : 0];
    tc0 = lane < p.num_groups ? t : 0;
  }
  const int64_t r = (int64_t)blockIdx.x * kW + wave;
  bool valid = r < p.total_rows;
  int64_t src = r;
  if constexpr (kGather) {
    const int64_t gi = gstart + r;
    const bool in = gi >= 0 && gi < p.gather_len;
    src = p.gather_index[in ? gi : 0];
    valid = valid && in;
  }
  int64_t g_stage = 0;
  if constexpr (kGroups) {
    int64_t g_row, excl, incl, total;
    group_scan(p, tc0, (int64_t)blockIdx.x * kW, r, -1, g_stage, g_row, excl, incl, total);
    valid = valid && g_row >= 0 && g_row == g_stage && r < total;
    if (g_stage < 0) g_stage = 0;  // no row of this workgroup is produced
  }
  valid = valid && src >= 0 && src < p.n0;
  sq_grp_row<Tag, kV, kW, kGather>(p, lds, g_stage, r, src, valid);
}

template <class Tag, int kV>
int launch_grp(SqParams p, hipStream_t stream) {
  constexpr int kW = TMO_SQ_GRP_WAVES;
  if (p.gather_index && p.gather_len == 0) return TMO_OK;  // no row is produced
  p.grp_main = (p.total_rows + kW - 1) / kW;
  const int64_t blocks = p.grp_main + (p.token_count ? p.num_groups : 0);
  if (blocks > 0x7fffffffLL) return TMO_ERR_INVALID_ARGUMENT;
  const dim3 grid((unsigned)blocks), block(64 * kW);
  if (p.token_count && p.gather_index)
    return launch_kernel(sq_grp<Tag, kV, kW, true, true>, grid, block, stream, p);
  if (p.token_count) return launch_kernel(sq_grp<Tag, kV, kW, true, false>, grid, block, stream, p);
  return launch_kernel(sq_grp<Tag, kV, kW, false, true>, grid, block, stream, p);
}

// Dense rows (no gather, no groups) of exactly 64 * kV 16-byte vectors: output row r reads
// input row r (r = s * inner + j), so the row address needs no division, every lane loads
// exactly kV vectors with no bounds checks, and the smooth mode is fixed at compile time
// (kScalar: one smooth value; kChan: a per-channel vector).  The grid is a few workgroups per
// CU that stride over the rows (TMO_SQ_WG_PER_CU); each first copies a per-channel smooth
// vector into LDS, since every row reads all of it (16 KiB for 4096 channels: twice the row's
// own bytes) and L1 could not serve that beside the row loads -- 22.9 -> 19.4 us on
// configs[3]'s shape.
template <class Tag, int kV, bool kScalar, bool kChan>
__global__ __launch_bounds__(256) void sq_dense(SqParams p) {
  constexpr int kPer = Tag::kPerVec;
  const int lane = threadIdx.x & (kWave - 1);
#if TMO_SQ_LDS_SMOOTH
  // per-channel smooth vector staged in LDS once per workgroup (kV * 64 * kPer floats)
  __shared__ u32x4 lds_smooth[kChan ? kV * kWave * (kPer / 4) : 1];
  if constexpr (kChan) {
    const u32x4* g = reinterpret_cast<const u32x4*>(p.smooth);
    for (int k = threadIdx.x; k < kV * kWave * (kPer / 4); k += 256) lds_smooth[k] = g[k];
    __syncthreads();
  }
  const u32x4* sp = lds_smooth + lane * (kPer / 4);
#else
  const u32x4* sp = reinterpret_cast<const u32x4*>(p.smooth) + lane * (kPer / 4);
#endif
  for (int64_t wg = blockIdx.x;; wg += gridDim.x) {
    const int64_t row = wg * 4 + __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
    if (row >= p.dense_rows) return;
    const char* xrow = static_cast<const char*>(p.x) + row * p.row_stride * Tag::kBytes + lane * 16;
    u32x4 w[kV];
    u32x4 sv[kV][kPer / 4];
#pragma unroll
    for (int i = 0; i < kV; ++i)
      w[i] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(xrow + i * kWave * 16));
    if constexpr (kChan) {
#pragma unroll
      for (int i = 0; i < kV; ++i)
#pragma unroll
        for (int q = 0; q < kPer / 4; ++q) sv[i][q] = sp[i * kWave * (kPer / 4) + q];
    }
    // Keep every load of the row ahead of the first use: without this barrier the scheduler
    // moved the unpack of the first vector (and its wait) between the loads, so the second half
    // of the row was requested only after the first vector had arrived.
    __builtin_amdgcn_sched_barrier(0);
    const float s_scalar = kScalar ? p.smooth[0] : 1.0f;
    float v[kV][kPer];
    float m = 0.0f;
#pragma unroll
    for (int i = 0; i < kV; ++i) {
      unpack(Tag{}, w[i], v[i]);
#pragma unroll
      for (int e = 0; e < kPer; ++e) {
        // RN(x * smooth), no FMA
        if constexpr (kScalar) v[i][e] = v[i][e] * s_scalar;
        if constexpr (kChan) v[i][e] = v[i][e] * __uint_as_float(sv[i][e / 4][e % 4]);
        m = abs_max(m, v[i][e]);
      }
    }
    const RowScale rs = make_row_scale(wave_max_uniform(m));
    int8_t* orow = p.out + row * p.channels + lane * kPer;
#pragma unroll
    for (int i = 0; i < kV; ++i) {
      uint32_t c[kPer / 4];
      encode_row<kPer>(v[i], rs, c);
      if constexpr (kPer == 8) {
        u32x2 c2;
        c2[0] = c[0];
        c2[1] = c[1];
        store_nt(reinterpret_cast<u32x2*>(orow + i * kWave * 8), c2);
      } else {
        store_nt(reinterpret_cast<uint32_t*>(orow + i * kWave * 4), c[0]);
      }
    }
    if (lane == 0) p.out_scale[row] = rs.s;
  }
}

template <class Tag, int kV>
int launch_dense(const SqParams& p, hipStream_t stream) {
  int64_t blocks = (p.dense_rows + 3) / 4;
  if (TMO_SQ_WG_PER_CU > 0) {
    int device = 0, cus = 0;
    if (hipGetDevice(&device) != hipSuccess ||
        hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, device) != hipSuccess)
      return TMO_ERR_LAUNCH;
    blocks = std::min<int64_t>(blocks, (int64_t)cus * TMO_SQ_WG_PER_CU);
  }
  if (blocks > 0x7fffffffLL) return TMO_ERR_INVALID_ARGUMENT;
  const dim3 grid((unsigned)blocks), block(256);
  if (p.smooth && p.smooth_len != 1)
    return launch_kernel(sq_dense<Tag, kV, false, true>, grid, block, stream, p);
  if (p.smooth) return launch_kernel(sq_dense<Tag, kV, true, false>, grid, block, stream, p);
  return launch_kernel(sq_dense<Tag, kV, false, false>, grid, block, stream, p);
}

#ifndef TMO_SQ_DENSE_WG
#define TMO_SQ_DENSE_WG 1
#endif
// Workgroups per CU of sq_dense_wg's persistent grid.  configs[3] (8192 x 4096 bf16,
// per-channel smooth) on MI355X, us per call in HIP-graph replays, against 19.38 for sq_dense:
// 2: 20.86, 3: 18.99, 4: 19.18, 5: 20.56, 6: 20.10, 8: 20.95.
#ifndef TMO_SQ_WG_ROW_PER_CU
#define TMO_SQ_WG_ROW_PER_CU 3
#endif

// Dense rows of exactly 256 * kV 16-byte vectors, one row per workgroup at a time: thread t
// owns vectors t + 256 * i of every row, so its smooth values are fixed and held in registers
// (kV * 8 floats), a row is kV fully coalesced 4 KiB load instructions, and the workgroup's
// next row is loaded while the current one is reduced, scaled and encoded.  The row maximum
// meets across the four wavefronts in LDS (two slots, alternating by row, so one barrier per
// row suffices: a wavefront writes slot k again only after the barrier of the row in between,
// which every wavefront reaches after reading slot k).  The grid is persistent, a few
// workgroups per CU striding over the rows.  When no row follows, the prefetch reads the first
// 16 bytes of x (one line for the whole workgroup, in bounds) so the loads carry no branch.
// Measured against sq_dense (side by side, identical output): 19.38 -> 18.99 us on configs[3].
// What it is not: a build of this kernel with all arithmetic removed (no smooth, reduction,
// barrier or encoder; the row bytes xor-folded into the stores) takes 19.3 us, and one without
// the scale stores 19.1 us, while a bare streaming copy of the same bytes in the same grid
// (two 16-byte loads and two 8-byte stores per thread per row) takes 17.8 us.  Rows mapped to
// workgroups in contiguous blocks instead of strides, or loaded without the prefetch, were
// 0.5-3 us slower.
template <class Tag, int kV, bool kScalar, bool kChan>
__global__ __launch_bounds__(256) void sq_dense_wg(SqParams p) {
  constexpr int kPer = Tag::kPerVec;
  constexpr int kT = 256;
  __shared__ uint32_t red[2][4];
  const int tid = threadIdx.x;
  const int lane = tid & (kWave - 1);
  const int wave = __builtin_amdgcn_readfirstlane(tid / kWave);
  const int64_t rows = p.dense_rows;
  int64_t row = blockIdx.x;
  if (row >= rows) return;  // workgroup-uniform
  const int64_t row_bytes = p.row_stride * Tag::kBytes;
  const char* xb = static_cast<const char*>(p.x);

  // Offsets are masked rather than branched on: a branch let the compiler merge the two paths'
  // loads through register copies (and drop the non-temporal hint of one of them).
  auto load_row = [&](u32x4 (&w)[kV], int64_t r, bool real) {
    const int64_t mask = -(int64_t)real;
#pragma unroll
    for (int i = 0; i < kV; ++i) {
      const int64_t off = (r * row_bytes + (int64_t)(tid + kT * i) * 16) & mask;
      w[i] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(xb + off));
    }
  };
  // The first row's loads go out before the smooth values' (which every workgroup reads from
  // L2 at once when the kernel starts), so the two round trips overlap: with the smooth loads
  // first and waited for, each workgroup started its row stream one round trip late -- about
  // 1.5 us of configs[3]'s 19 us.
  u32x4 wa[kV], wb[kV];
  load_row(wa, row, true);
  __builtin_amdgcn_sched_barrier(0);
  float smv[kV][kPer];
  if constexpr (kChan) {
#pragma unroll
    for (int i = 0; i < kV; ++i) {
      const u32x4* sp = reinterpret_cast<const u32x4*>(p.smooth + (int64_t)(tid + kT * i) * kPer);
#pragma unroll
      for (int q = 0; q < kPer / 4; ++q) {
        const u32x4 s4 = sp[q];
#pragma unroll
        for (int e = 0; e < 4; ++e) smv[i][4 * q + e] = __uint_as_float(s4[e]);
      }
    }
  }
  float s_scalar = kScalar ? p.smooth[0] : 1.0f;
  // Wait for the smooth values here, once: left pending into the row loop, they made the
  // compiler's wait analysis flush every outstanding load and store at the loop head.
  if constexpr (kChan) {
#pragma unroll
    for (int i = 0; i < kV; ++i)
#pragma unroll
      for (int e = 0; e < kPer; ++e) asm volatile("" : "+v"(smv[i][e]));
  }
  if constexpr (kScalar) asm volatile("" : "+v"(s_scalar));

  // Prefetch the next row into `nxt`, then quantise `cur` (row r) and write it; its codes stay
  // in `keep` until the end of the next row's step.
  //
  // Why the stores and the keep: the compiler's wait analysis does not let a register that
  // held a pending store's data be overwritten before that store completes, and with the
  // memory counter in order such a wait also waits for every load issued before the store --
  // the next row's prefetch included.  Holding each row's codes until the following row's
  // codes are stored means their registers are only reused a whole row later, when the store
  // has long completed.  The stores are the compiler's own (not inline assembly), so that the
  // same analysis counts them and waits for a row's loads with the exact number of later
  // memory operations outstanding.
  constexpr int kC = kV * kPer / 4;
  auto step = [&](u32x4 (&cur)[kV], u32x4 (&nxt)[kV], int64_t r, int par, uint32_t (&keep)[kC],
                  uint32_t (&prev)[kC]) -> bool {
    const int64_t nr = r + gridDim.x;
    const bool more = nr < rows;  // workgroup-uniform
    load_row(nxt, nr, more);
    __builtin_amdgcn_sched_barrier(0);
    float v[kV][kPer];
    float m = 0.0f;
#pragma unroll
    for (int i = 0; i < kV; ++i) {
      unpack(Tag{}, cur[i], v[i]);
#pragma unroll
      for (int e = 0; e < kPer; ++e) {
        // RN(x * smooth), no FMA
        if constexpr (kScalar) v[i][e] = v[i][e] * s_scalar;
        if constexpr (kChan) v[i][e] = v[i][e] * smv[i][e];
        m = abs_max(m, v[i][e]);
      }
    }
    const uint32_t mw = wave_max_u32_sgpr(__float_as_uint(m));
    if (lane == 0) red[par][wave] = mw;
    __syncthreads();
    const uint32_t mb = max(max(red[par][0], red[par][1]), max(red[par][2], red[par][3]));
    const RowScale rs =
        make_row_scale(__uint_as_float((uint32_t)__builtin_amdgcn_readfirstlane((int)mb)));
    int8_t* orow = p.out + r * p.channels;  // uniform base, 32-bit lane offsets
#pragma unroll
    for (int i = 0; i < kV; ++i) encode_row<kPer>(v[i], rs, keep + i * (kPer / 4));
#pragma unroll
    for (int i = 0; i < kV; ++i) {
      const uint32_t off = (uint32_t)(tid + kT * i) * kPer;
      if constexpr (kPer == 8) {
        u32x2 c2;
        c2[0] = keep[2 * i];
        c2[1] = keep[2 * i + 1];
        __builtin_nontemporal_store(c2, reinterpret_cast<u32x2*>(orow + off));
      } else {
        __builtin_nontemporal_store(keep[i], reinterpret_cast<uint32_t*>(orow + off));
      }
    }
    if (tid == 0) p.out_scale[r] = rs.s;
#pragma unroll
    for (int j = 0; j < kC; ++j) asm volatile("" : : "v"(prev[j]));
    return more;
  };
  uint32_t ka[kC], kb[kC];
#pragma unroll
  for (int j = 0; j < kC; ++j) kb[j] = 0;
  for (;;) {
    if (!step(wa, wb, row, 0, ka, kb)) return;
    row += gridDim.x;
    if (!step(wb, wa, row, 1, kb, ka)) return;
    row += gridDim.x;
  }
}

template <class Tag, int kV>
int launch_dense_wg(const SqParams& p, hipStream_t stream) {
  int device = 0, cus = 0;
  if (hipGetDevice(&device) != hipSuccess ||
      hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, device) != hipSuccess)
    return TMO_ERR_LAUNCH;
  const int64_t blocks = std::min<int64_t>(p.dense_rows, (int64_t)cus * TMO_SQ_WG_ROW_PER_CU);
  const dim3 grid((unsigned)blocks), block(256);
  if (p.smooth && p.smooth_len != 1)
    return launch_kernel(sq_dense_wg<Tag, kV, false, true>, grid, block, stream, p);
  if (p.smooth) return launch_kernel(sq_dense_wg<Tag, kV, true, false>, grid, block, stream, p);
  return launch_kernel(sq_dense_wg<Tag, kV, false, false>, grid, block, stream, p);
}

// Generic path: any channel count / alignment; one wavefront per row, two passes.
template <class Tag>
__global__ __launch_bounds__(256) void sq_generic(SqParams p) {
  const int lane = threadIdx.x & (kWave - 1);
  const int64_t orow = (int64_t)blockIdx.x * (256 / kWave) +
                       __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
  if (orow >= p.total_rows) return;
  const int64_t r = orow / p.inner;
  const int64_t jn = orow - r * p.inner;
  int64_t src, g;
  if (!locate_row(p, r, src, g)) return;
  const int64_t base = (src * p.inner + jn) * p.row_stride;
  const float* sm = p.smooth ? p.smooth + (p.token_count ? g * p.smooth_len : 0) : nullptr;
  float m = 0.0f;
  for (int64_t d = lane; d < p.channels; d += kWave) {
    float xv = load1(Tag{}, p.x, base + d);
    if (sm) xv = xv * sm[p.smooth_len == 1 ? 0 : d];
    m = abs_max(m, xv);
  }
  const RowScale rs = make_row_scale(wave_max_uniform(m));
  int8_t* o = p.out + orow * p.channels;
  for (int64_t d = lane; d < p.channels; d += kWave) {
    float xv = load1(Tag{}, p.x, base + d);
    if (sm) xv = xv * sm[p.smooth_len == 1 ? 0 : d];
    o[d] = encode1(xv, rs);
  }
  if (lane == 0) p.out_scale[orow] = rs.s;
}


template <class Tag, bool kStream, int kWPR>
int launch_vec(const SqParams& p, int64_t per_lane, hipStream_t stream) {
  const int64_t blocks = (p.total_rows + (4 / kWPR) - 1) / (4 / kWPR);
  if (blocks > 0x7fffffffLL) return TMO_ERR_INVALID_ARGUMENT;
  const dim3 grid((unsigned)blocks), block(256);
  if (per_lane <= 1) return launch_kernel(sq_vec<Tag, 1, kStream, kWPR>, grid, block, stream, p);
  if (per_lane <= 2) return launch_kernel(sq_vec<Tag, 2, kStream, kWPR>, grid, block, stream, p);
  if (per_lane <= 4) return launch_kernel(sq_vec<Tag, 4, kStream, kWPR>, grid, block, stream, p);
  if (per_lane <= 8) return launch_kernel(sq_vec<Tag, 8, kStream, kWPR>, grid, block, stream, p);
  return launch_kernel(sq_vec<Tag, 16, kStream, kWPR>, grid, block, stream, p);
}

template <class Tag>
int launch(const SqParams& p, hipStream_t stream) {
  constexpr int kPer = Tag::kPerVec;
  const int64_t blocks = (p.total_rows + 3) / 4;
  if (blocks > 0x7fffffffLL) return TMO_ERR_INVALID_ARGUMENT;
  const bool aligned =
      p.channels % kPer == 0 && reinterpret_cast<uintptr_t>(p.x) % 16 == 0 &&
      (p.row_stride * Tag::kBytes) % 16 == 0 && reinterpret_cast<uintptr_t>(p.out) % 8 == 0 &&
      (!p.smooth || p.smooth_len == 1 || reinterpret_cast<uintptr_t>(p.smooth) % 16 == 0);
  const int64_t nvec = p.channels / kPer;
  // One wavefront per row measured fastest (4096 channels: 20.4 us vs 23.0 us split over two);
  // rows longer than 16 vectors per lane are split over two wavefronts rather than falling
  // back to the scalar kernel.
  constexpr int kW = TMO_SQ_WAVES_PER_ROW;
  const bool split = kW > 1 && nvec > 16 * kWave;
  const int64_t per_lane = (nvec + kWave * (split ? kW : 1) - 1) / (kWave * (split ? kW : 1));
  if (!aligned || per_lane > 16)
    return launch_kernel(sq_generic<Tag>, dim3((unsigned)blocks), dim3(256), stream, p);
  if (split) {
    if (p.gather_index) return launch_vec<Tag, false, kW>(p, per_lane, stream);
    return launch_vec<Tag, true, kW>(p, per_lane, stream);
  }
  if (TMO_SQ_DENSE_WG && !p.gather_index && !p.token_count && nvec % 256 == 0) {
    switch (nvec / 256) {
      case 1: return launch_dense_wg<Tag, 1>(p, stream);
      case 2: return launch_dense_wg<Tag, 2>(p, stream);
      case 4: return launch_dense_wg<Tag, 4>(p, stream);
      default: break;
    }
  }
  if (!p.gather_index && !p.token_count && nvec % kWave == 0) {
    switch (nvec / kWave) {
      case 1: return launch_dense<Tag, 1>(p, stream);
      case 2: return launch_dense<Tag, 2>(p, stream);
      case 4: return launch_dense<Tag, 4>(p, stream);
      case 8: return launch_dense<Tag, 8>(p, stream);
      case 16: return launch_dense<Tag, 16>(p, stream);
      default: break;
    }
  }
  if ((p.gather_index || p.token_count) && p.inner == 1 && p.smooth && p.channels > 1 &&
      p.smooth_len == p.channels && nvec % kWave == 0) {
    switch (nvec / kWave) {
      case 1: return launch_grp<Tag, 1>(p, stream);
      case 2: return launch_grp<Tag, 2>(p, stream);
      case 4: return launch_grp<Tag, 4>(p, stream);
      case 8: return launch_grp<Tag, 8>(p, stream);
      default: break;
    }
  }
  if (p.gather_index) return launch_vec<Tag, false, 1>(p, per_lane, stream);
  return launch_vec<Tag, true, 1>(p, per_lane, stream);
}

}  // namespace
}  // namespace tmo

extern "C" int tmo_hip_scaled_quantize_per_token(
    const void* x, int64_t n0, int64_t inner, int64_t channels, int64_t x_row_stride,
    int8_t* out, float* out_scale, const float* smooth, int64_t smooth_len,
    const int32_t* token_count, int64_t num_groups, const int32_t* gather_index,
    int64_t gather_len, const int32_t* gather_start, int64_t out_rows, int dtype, void* stream) {
  using namespace tmo;
  if (dtype != TMO_DTYPE_F32 && dtype != TMO_DTYPE_F16 && dtype != TMO_DTYPE_BF16)
    return TMO_ERR_UNSUPPORTED_DTYPE;
  if (!x || !out || !out_scale) return TMO_ERR_INVALID_ARGUMENT;
  if (n0 < 0 || inner <= 0 || channels <= 0 || x_row_stride < channels || out_rows < 0)
    return TMO_ERR_INVALID_ARGUMENT;
  if (smooth && smooth_len != 1 && smooth_len != channels) return TMO_ERR_INVALID_ARGUMENT;
  if (token_count && num_groups <= 0) return TMO_ERR_INVALID_ARGUMENT;
  if (gather_index && gather_len < 0) return TMO_ERR_INVALID_ARGUMENT;
  if (gather_start && !gather_index) return TMO_ERR_INVALID_ARGUMENT;
  if (out_rows == 0 || n0 == 0) return TMO_OK;

  SqParams p{};
  p.x = x;
  p.n0 = n0;
  p.inner = inner;
  p.channels = channels;
  p.row_stride = x_row_stride;
  p.out = out;
  p.out_scale = out_scale;
  p.smooth = smooth;
  p.smooth_len = smooth ? smooth_len : 0;
  p.token_count = token_count;
  p.num_groups = token_count ? num_groups : 0;
  p.gather_index = gather_index;
  p.gather_len = gather_index ? gather_len : 0;
  p.gather_start = gather_start;
  p.out_rows = out_rows;
  p.total_rows = out_rows * inner;
  p.dense_rows = (out_rows < n0 ? out_rows : n0) * inner;
  hipStream_t s = static_cast<hipStream_t>(stream);
  switch (dtype) {
    case TMO_DTYPE_F32: return launch<F32>(p, s);
    case TMO_DTYPE_F16: return launch<F16>(p, s);
    default: return launch<BF16>(p, s);
  }
}
