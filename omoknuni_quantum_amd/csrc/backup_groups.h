// The ordered group backup and the signed leaf values per simulation, as device functions:
// the kernels of tree_backup.hip, and the expansion-and-backup kernels of tree_expand.hip, run
// them.  Ordered mode uses the group log of the selection: a node appears in exactly one group
// per wave, and the group's members are in simulation order, so folding the members' signed
// values into W[x] in that order gives the sequential result bit for bit, with no atomics.
#pragma once
#include <algorithm>

#include "omq_common.h"

namespace omq {

constexpr int kBackupThreads = 256;

// Workgroups per tree of the group backup: sized for a typical wave (groups ~ W * depth); the
// blocks stride over the rest.
inline int backup_group_blocks(int W) {
  const int est_groups = W * 8;
  return std::min(std::max((est_groups + kBackupThreads - 1) / kBackupThreads, 1), 1024);
}
constexpr int kBigGroup = 32;
constexpr int kBigChunk = 8;  // member values per lane held per chunk of a big group

// signed value of simulation s of tree t: v(leaf), negated when the leaf depth is odd in
// leaf-positive mode, so that the contribution at depth d is (d odd ? -sv : sv)
__device__ inline void sim_value_at(const omq_forest& f, const omq_wave& w, int t, int s,
                                    int sign_mode) {
  const int64_t wb = (int64_t)t * w.max_wave;
  const float v = w.values[wb + w.sim_uid[wb + s]];
  const int L = w.path_len[wb + s];
  const bool neg = sign_mode == OMQ_SIGN_LEAF_POSITIVE && ((L - 1) & 1);
  w.sim_value[wb + s] = neg ? -v : v;
}

// Groups are dealt to the lanes of all waves in a strided order (lane l of wave w takes groups
// w + (l + 64*i) * waves), so the few big groups of a level -- they are logged next to each
// other -- land in different waves.  A small group is folded by its lane after all of its
// member values have been fetched (the loads of a lane are issued together); a big group is
// folded by its wave: 64 member values at a time, one per lane, are read into scalar
// registers and added in order (the loads of the next 256 are in flight meanwhile).
//
// FUSED: the signed leaf value of a member is formed here from its unique leaf's value and its
// path length (as sim_value_kernel forms it), which saves that kernel's launch; used for waves
// of at most kFuseMaxWave simulations.  Larger waves have more groups per lane, and there the
// extra dependent load costs more than the launch (C3 and C4 backups were 6 % and 15 % slower).
constexpr int kFuseMaxWave = 512;

// The group backup of block bx of nblocks (kBackupThreads threads each) of tree t.
template <bool FUSED>
__device__ inline void backup_groups_block(const omq_forest& f, const omq_wave& w, int vli,
                                           int sign_mode, int bx, int t, int nblocks) {
  const int lane = lane_id();
  const int wib = threadIdx.x / kWave;
  const int64_t tb = (int64_t)t * f.capacity;
  const int64_t wb = (int64_t)t * w.max_wave;
  const int MW = w.max_wave, MD = w.max_depth;
  const int64_t gmax = (int64_t)MW * MD;
  const int G = w.gcount[t];
  const int waves_total = nblocks * (kBackupThreads / kWave);
  const int wave_global = bx * (kBackupThreads / kWave) + wib;
  const int32_t* uid = w.sim_uid + wb;
  const int32_t* plen = w.path_len + wb;
  const float* uval = w.values + wb;
  const float* svals = w.sim_value + wb;
  const bool leaf_pos = sign_mode == OMQ_SIGN_LEAF_POSITIVE;
  // signed leaf value of simulation s (sim_value_kernel's value)
  auto sv = [&](int s) {
    if (!FUSED) return svals[s];
    const float v = uval[uid[s]];
    return (leaf_pos && ((plen[s] - 1) & 1)) ? -v : v;
  };
  for (int i0 = 0; wave_global + i0 * waves_total < G; i0 += kWave) {
    const int g = wave_global + (i0 + lane) * waves_total;
    int p = 0, d = 0, seg = 0, m = 0;
    if (g < G) {
      const int4 rec = *reinterpret_cast<const int4*>(w.glog + ((int64_t)t * gmax + g) * 4);
      p = rec.x;
      d = rec.y;
      seg = rec.z;
      m = rec.w;
    }
    if (g < G && m <= kBigGroup) {
      const uint16_t* mem = w.gmembers + ((int64_t)t * MD + d) * MW + seg;
      float vals[kBigGroup];
#pragma unroll
      for (int i = 0; i < kBigGroup; ++i) vals[i] = i < m ? sv(mem[i]) : 0.0f;
      float acc = f.value_sums[tb + p];
      const bool odd = d & 1;
#pragma unroll
      for (int i = 0; i < kBigGroup; ++i)
        if (i < m) acc = acc + (odd ? -vals[i] : vals[i]);
      f.value_sums[tb + p] = acc;
      f.visit_counts[tb + p] += m - vli * m;
    }
    // big groups: the whole wave, one group at a time
    uint64_t big = __ballot(g < G && m > kBigGroup);
    while (big) {
      const int l = lowest_lane(big);
      big &= big - 1;
      const int bp = readlane_i(p, l), bd = readlane_i(d, l), bseg = readlane_i(seg, l),
                bm = readlane_i(m, l);
      const uint16_t* bmem = w.gmembers + ((int64_t)t * MD + bd) * MW + bseg;
      const bool odd = bd & 1;
      float acc = f.value_sums[tb + bp];
      // chunks of kBigChunk*64 members, software-pipelined over the two dependent loads: while
      // chunk c is folded in order, the values of chunk c+1 (from member ids loaded one chunk
      // earlier) and the member ids of chunk c+2 are in flight
      constexpr int kCh = kBigChunk * kWave;
      float xa[kBigChunk], xb[kBigChunk];
      int ib[kBigChunk];
#pragma unroll
      for (int u = 0; u < kBigChunk; ++u) {
        const int c = u * kWave + lane;
        xa[u] = c < bm ? sv(bmem[c]) : 0.0f;
        const int c1 = kCh + c;
        ib[u] = c1 < bm ? (int)bmem[c1] : 0;
      }
      for (int c0 = 0; c0 < bm; c0 += kCh) {
        const int cn = c0 + kCh;
#pragma unroll
        for (int u = 0; u < kBigChunk; ++u) {
          const int c = cn + u * kWave + lane;
          xb[u] = c < bm ? sv(ib[u]) : 0.0f;
          const int c2 = cn + kCh + u * kWave + lane;
          ib[u] = c2 < bm ? (int)bmem[c2] : 0;
        }
#pragma unroll
        for (int u = 0; u < kBigChunk; ++u) {
          const int cb = c0 + u * kWave;
          if (cb >= bm) break;
          // lanes 0..63 hold members cb..cb+63: add them in order from scalar registers (the
          // reads are independent, only the adds form a chain)
          const float x = odd ? -xa[u] : xa[u];
          if (bm - cb >= kWave) {
#pragma unroll
            for (int l = 0; l < kWave; ++l) acc = acc + readlane_f(x, l);
          } else {
            for (int l = 0; l < bm - cb; ++l) acc = acc + readlane_f(x, l);
          }
        }
#pragma unroll
        for (int u = 0; u < kBigChunk; ++u) xa[u] = xb[u];
      }
      if (lane == 0) {
        f.value_sums[tb + bp] = acc;
        f.visit_counts[tb + bp] += bm - vli * bm;
      }
    }
  }
}

}  // namespace omq
