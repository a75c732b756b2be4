// trie_chain.h — head_dim 64, bf16 kernels for plans whose trie is a forest
// of chains (every row's parent is the row before it or none: independent
// sequences, C5). Included by trie_attn.hip after trie_deep.h.
//
// On such a plan the trie attention of a chain is plain causal attention
// over its rows, so the general kernels' per-tile key lists, interval tables
// and per-pair interval tests are overhead. Here a unit is (chain, head): the
// chain's K and V rows of the head (query side) or Q and dO rows (key side),
// at most 256, are loaded into LDS once, and the eight waves of the
// workgroup take the chain's 16-row blocks, costliest first in snake order.
// A block pair is masked only on the diagonal (key <= query inside the
// block) and past the chain's end; rows past the end repeat the chain's last
// row in LDS, so a masked pair never multiplies stale data. Each key's dK/dV and each
// query's dQ is complete within its unit: no partials, no reduction. The
// backward runs both sides in one launch (bwd_kernel: per unit the query
// side, then the key side in the same LDS); bwd_q_kernel + bwd_kv_kernel
// are the two-launch form.
//
// Lane layouts and products are those of trie_deep.h: 16x16 blocks on the
// bf16 matrix instructions, lane l = 16g + c.
#pragma once

namespace agpt_chain {

using namespace agpt;
using agpt_blk::group_max;
using agpt_blk::group_sum;
using agpt_blk::kBlk;
using agpt_blk::kRescaleLog2;
using agpt_blk::pack_bf16;
using agpt_blk::Slice;
using agpt_blk::slice_dot;
using agpt_deep::kNoMax;
using agpt_deep::mfma_a_bf16;
using agpt_deep::mfma_a2_bf16;
using agpt_deep::opaque_tid;
using agpt_deep::read_tr;
using agpt_fast::f4;
using agpt_fast::u4;
using agpt_fast::uniform;

constexpr int kWaves = 8;
constexpr int kThreads = 64 * kWaves;
constexpr int kRows = kMaxDepth;  // longest chain
constexpr int kHD = 64;
constexpr int WS = kHD + 8;       // LDS row stride (bf16 elements): 144 bytes
constexpr int kPieces = kHD / 8;  // 16-byte pieces per row of a head

// Dynamic LDS: two row tiles [kRows][WS] of bf16 (K and V, or Q and dO).
__host__ __device__ constexpr size_t lds_bytes() { return 2u * kRows * WS * sizeof(bf16_t); }

// Block k (0, 1, ..) of wave w among nb blocks: positions dealt in snake
// order (wave 0..7, then 7..0, ..); position p is block nb-1-p on the query
// side (block i has i+1 key blocks) and block p on the key side (block j
// has nb-j query blocks), so each wave's blocks are costliest first and
// the waves' totals are close. -1 past the end.
__device__ __forceinline__ int snake_block(int k, int w, int nb, bool key_side) {
  const int pos = kWaves * k + ((k & 1) ? kWaves - 1 - w : w);
  if (pos >= nb) return -1;
  return key_side ? pos : nb - 1 - pos;
}

// The unit's chain and head: unit u is chain u / H of the plan's order
// (longest first), head u % H; (first row, rows) in one 8-byte read.
struct ChainUnit {
  int64_t c0;  // first row
  int L;       // rows
  int nb;      // 16-row blocks
  int h;
  // Element offsets of the unit's first row, head h, in a [T, D] tensor and
  // in a [T, H] table (uniform; rows within the unit are added as 32-bit
  // offsets, so that per-lane addresses are a scalar base and one VGPR).
  __device__ __forceinline__ int64_t at(int D) const { return c0 * D + h * kHD; }
  __device__ __forceinline__ int64_t tab(int H) const { return c0 * H + h; }
};
template <typename PlanT>
__device__ __forceinline__ int2 load_info(const PlanT& pl, int u, int H, int64_t n_units) {
  return u < n_units ? *reinterpret_cast<const int2*>(pl.chain_info + 2 * (u / H)) : int2{0, 1};
}
__device__ __forceinline__ ChainUnit unit_of(int2 info, int u, int H) {
  ChainUnit x;
  x.c0 = uniform(info.x);
  x.L = uniform(info.y);
  x.nb = (x.L + kBlk - 1) / kBlk;
  x.h = u % H;
  return x;
}

// A unit's rows 0 .. 16 nb - 1 (chain rows of head h) of tensors A and B,
// fetched into registers and then stored into the LDS tiles As and Bs;
// with kTabs also lse * log2(e) of those rows (key side), and with
// kTabs == kLseDelta their δ too (kLseOnly: δ is already in LDS). Rows past
// the chain repeat its last row (finite values that the masks give zero
// weight), so every load is unconditional and in bounds.
constexpr int kLseDelta = 1;
constexpr int kLseOnly = 2;
template <int kTabs>
struct Rows {
  static constexpr int kPer = kRows * kPieces / kThreads;  // 4 rows of each tensor per thread
  u4 a[kPer], b[kPer];
  float rl, rd;
  // Thread t fetches 16-byte piece t % 8 of rows t / 8 + 64 k.
  __device__ __forceinline__ void fetch(const bf16_t* __restrict__ A, const bf16_t* __restrict__ B,
                                        const float* __restrict__ lse, const float* __restrict__ Dl,
                                        const ChainUnit& x, int D, int H) {
    const int tid = opaque_tid();
    const int r0 = tid / kPieces;
    const int col = (tid % kPieces) * 8;
    const bf16_t* Au = A + x.at(D);
    const bf16_t* Bu = B + x.at(D);
#pragma unroll
    for (int k = 0; k < kPer; ++k) {
      const unsigned o = static_cast<unsigned>(min(r0 + k * (kThreads / kPieces), x.L - 1) * D + col);
      a[k] = *reinterpret_cast<const u4*>(Au + o);
      b[k] = *reinterpret_cast<const u4*>(Bu + o);
    }
    if constexpr (kTabs != 0) {
      const unsigned o = static_cast<unsigned>(min(tid, x.L - 1) * H);
      rl = lse[x.tab(H) + o];
      if constexpr (kTabs == kLseDelta) rd = Dl[x.tab(H) + o];
    }
  }
  __device__ __forceinline__ void store(bf16_t* As, bf16_t* Bs, float* l2s, float* dls, const ChainUnit& x) const {
    const int tid = opaque_tid();
    const int r0 = tid / kPieces;
    const int col = (tid % kPieces) * 8;
#pragma unroll
    for (int k = 0; k < kPer; ++k) {
      const int r = r0 + k * (kThreads / kPieces);
      if (r < kBlk * x.nb) {
        *reinterpret_cast<u4*>(As + r * WS + col) = a[k];
        *reinterpret_cast<u4*>(Bs + r * WS + col) = b[k];
      }
    }
    if constexpr (kTabs != 0) {
      if (tid < kRows) {
        l2s[tid] = rl * kLog2e;
        if constexpr (kTabs == kLseDelta) dls[tid] = rd;
      }
    }
  }
};

// Unit k of this workgroup: the plan's units (longest chains first) dealt
// to the G workgroups in snake order (0 .. G-1, then G-1 .. 0, ..), so the
// workgroups' totals are close. The deal is fixed by the grid: no claim
// counters, so nothing needs clearing before a launch.
__device__ __forceinline__ int dealt_unit(int k) {
  const int G = static_cast<int>(gridDim.x), b = static_cast<int>(blockIdx.x);
  return k * G + ((k & 1) ? G - 1 - b : b);
}

// The unit loop of a chain kernel: body(x) works on unit x with its rows in
// As, Bs (and l2s, dls). The next unit's chain (first row, rows) is read
// while the current unit's rows are fetched. (Row loads a unit ahead were
// measured: with two workgroups per CU one's compute already covers the
// other's loads, and the registers they took cost the backward kernels
// more than they saved.)
template <int kTabs, typename PlanT, typename Body>
__device__ __forceinline__ void unit_loop(const PlanT& pl, int H, const bf16_t* __restrict__ A,
                                          const bf16_t* __restrict__ B, const float* __restrict__ lse,
                                          const float* __restrict__ Dl, bf16_t* As, bf16_t* Bs, float* l2s,
                                          float* dls, Body&& body) {
  const int D = H * kHD;
  const int64_t n_units = static_cast<int64_t>(pl.n_chains) * H;
  int k = 0;
  int u = dealt_unit(0);
  int2 info = load_info(pl, u, H, n_units);
  while (u < n_units) {
    const int nu = dealt_unit(++k);
    const ChainUnit x = unit_of(info, u, H);
    // The rows' loads, stores and barrier at a higher wave priority than the
    // blocks, so they go out ahead of the other workgroup's block steps
    // (forward 0.077-0.079 -> 0.074 ms).
    __builtin_amdgcn_s_setprio(3);
    {
      Rows<kTabs> rows;
      rows.fetch(A, B, lse, Dl, x, D, H);
      rows.store(As, Bs, l2s, dls, x);
    }
    const int2 ni = load_info(pl, nu, H, n_units);
    __syncthreads();
    __builtin_amdgcn_s_setprio(0);
    body(x);
    __syncthreads();  // the unit's rows are no longer read
    u = nu;
    info = ni;
  }
}

// ---------------------------------------------------------------------------
// Forward: O and lse. Query block i of the chain against key blocks 0 .. i:
// S^T = K Q^T puts query c in lane column c (keys 4g .. 4g+3 in its
// registers); online softmax with the lazy rescale; O^T += V^T P^T with V^T
// read transposed from the V rows.
// ---------------------------------------------------------------------------
template <typename PlanT>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(4))) void fwd_kernel(PlanT pl, const bf16_t* __restrict__ Q,
                                                       const bf16_t* __restrict__ K,
                                                       const bf16_t* __restrict__ V, bf16_t* __restrict__ O,
                                                       float* __restrict__ lse, int H, float scale) {
  constexpr int KD = kHD / 4;
  constexpr int MT = kHD / 16;
  extern __shared__ __align__(16) unsigned char dyn[];
  bf16_t* Ks = reinterpret_cast<bf16_t*>(dyn);
  bf16_t* Vs = Ks + kRows * WS;
  const int lane = threadIdx.x & 63;
  const int wave = uniform(static_cast<int>(threadIdx.x >> 6));
  const int g = lane >> 4, c = lane & 15;
  const int D = H * kHD;
  const float sfac = scale * kLog2e;  // bf16 scores come unscaled
  unit_loop<0>(pl, H, K, V, nullptr, nullptr, Ks, Vs, nullptr, nullptr,
                   [&](const ChainUnit& x) {
    // The wave's blocks, costliest first: at most two (nb <= 16, eight
    // waves). Both blocks' Q slices are requested at once, so the second's
    // arrive while the first block is worked on. (Both blocks in one pass
    // over the key blocks, sharing the K and V^T reads, was measured no
    // faster.)
    const int iA = snake_block(0, wave, x.nb, false);
    if (iA < 0) return;
    const int iB = snake_block(1, wave, x.nb, false);
    Slice<bf16_t, KD> qs[2];
    qs[0].load(Q + x.at(D) + static_cast<unsigned>(min(kBlk * iA + c, x.L - 1) * D + KD * g));
    qs[1].load(Q + x.at(D) + static_cast<unsigned>(min(kBlk * max(iB, 0) + c, x.L - 1) * D + KD * g));
    auto block = [&](int i, const Slice<bf16_t, KD>& qf) {
      const int q = kBlk * i + c;  // this lane's query (chain index)
      float m = kNoMax, l = 0.0f;
      f4 o[MT];
#pragma unroll
      for (int j = 0; j < MT; ++j) o[j] = f4{0.0f, 0.0f, 0.0f, 0.0f};
      // key 16kb + 4g + r is live iff it is <= min(q, L - 1), i.e. r <= t
      const int tq = min(q, x.L - 1) - 4 * g;
      // Key blocks kb and kb + 1 in one step: one online-softmax update for
      // both and one 32-deep O^T product per output tile. Only the step
      // that holds the diagonal block i is masked (blocks below i are whole
      // chain rows); past block i its second half reads block i again with
      // every weight masked to 0.
      auto step = [&](int kb, auto masked) {
        const int kb1 = min(kb + 1, i);
        Slice<bf16_t, KD> kf0, kf1;
        kf0.load(Ks + (kBlk * kb + c) * WS + KD * g);
        kf1.load(Ks + (kBlk * kb1 + c) * WS + KD * g);
        const f4 sv0 = slice_dot(kf0, qf, f4{0.0f, 0.0f, 0.0f, 0.0f});  // key 16kb+4g+r against query q
        const f4 sv1 = slice_dot(kf1, qf, f4{0.0f, 0.0f, 0.0f, 0.0f});  // key 16(kb+1)+4g+r
        float sc[8];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          sc[r] = sv0[r];
          sc[4 + r] = sv1[r];
        }
        if constexpr (decltype(masked)::value) {
          const int t = tq - kBlk * kb;
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            sc[r] = r <= t ? sc[r] : -__builtin_inff();
            sc[4 + r] = r + kBlk <= t ? sc[4 + r] : -__builtin_inff();
          }
        }
        const float lmx = fmaxf(fmaxf(fmaxf(sc[0], sc[1]), fmaxf(sc[2], sc[3])),
                                fmaxf(fmaxf(sc[4], sc[5]), fmaxf(sc[6], sc[7]))) * sfac;
        if (__any(lmx > m + kRescaleLog2)) {
          const float mx = group_max(lmx);
          const bool resc = mx > m + kRescaleLog2;
          const float a = resc ? fast_exp2(m - mx) : 1.0f;
          m = resc ? mx : m;
          l *= a;
#pragma unroll
          for (int j = 0; j < MT; ++j) o[j] *= a;
        }
        float p[8];
#pragma unroll
        for (int r = 0; r < 8; ++r) {
          p[r] = fast_exp2(__builtin_fmaf(sc[r], sfac, -m));  // masked: exp2(-inf) = 0
          l += p[r];
        }
        const float p0[4] = {p[0], p[1], p[2], p[3]}, p1[4] = {p[4], p[5], p[6], p[7]};
        const uint2 pw0 = pack_bf16(p0), pw1 = pack_bf16(p1);
#pragma unroll
        for (int j = 0; j < MT; ++j)  // V^T blocks: dims 16j .., keys 16kb .. and 16kb1 ..
          o[j] = mfma_a2_bf16(read_tr(Vs, WS, kBlk * kb, kBlk * j, lane), read_tr(Vs, WS, kBlk * kb1, kBlk * j, lane),
                              pw0, pw1, o[j]);
      };
      int kb = 0;
      for (; kb + 1 < i; kb += 2) step(kb, std::false_type{});
      step(kb, std::true_type{});
      const float le = group_sum(l);
      // Every slice has arrived: waiting here, before this block's stores,
      // the next block starts with no wait (one after the stores would
      // also wait for them).
      agpt_deep::wait_loads();
      if (q < x.L) {
        const float inv = __builtin_amdgcn_rcpf(le);
#pragma unroll
        for (int j = 0; j < MT; ++j) {
          float v[4] = {o[j][0] * inv, o[j][1] * inv, o[j][2] * inv, o[j][3] * inv};
          store_vec<4>(O + x.at(D) + static_cast<unsigned>(q * D + kBlk * j + 4 * g), v);
        }
        if (g == 0) lse[x.tab(H) + static_cast<unsigned>(q * H)] = (m + fast_log2(le)) * kLn2;
      }
    };
    block(iA, qs[0]);
    if (iB >= 0) block(iB, qs[1]);
  });
}

// ---------------------------------------------------------------------------
// Backward, query side: δ and dQ in one pass over key blocks 0 .. i, as the
// deep dQ kernel does (batched_depth_backward.cr:637-646 for δ): with
// a_j = w_j dw_j, dQ = scale (Σ_j a_j k_j − δ Σ_j w_j k_j), δ = Σ_j a_j; the
// bf16 operands a_j and w_j enter as high and low bf16 parts. dQ gets the
// inverse rotation at the query's depth.
// ---------------------------------------------------------------------------
// The query side of unit x (its K, V rows in Ks, Vs): this wave's query
// blocks. δ, for the key side, goes to Dl [T, H] and/or to the unit's LDS
// table dls, where non-null.
template <bool kAhead, typename RopeT>
__device__ __forceinline__ void q_side(const ChainUnit& x, const bf16_t* Ks, const bf16_t* Vs,
                                       const bf16_t* __restrict__ Q, const float* __restrict__ lse,
                                       const bf16_t* __restrict__ dO, float* __restrict__ dQ,
                                       float* __restrict__ Dl, float* dls, const RopeT& rope, int H, float scale) {
  constexpr int KD = kHD / 4;
  constexpr int MT = kHD / 16;
  const int tid = opaque_tid();
  const int lane = tid & 63;
  const int wave = uniform(tid >> 6);
  const int g = lane >> 4, c = lane & 15;
  const int D = H * kHD;
  const float sfac = scale * kLog2e;
  {
    // The wave's (at most two) blocks, costliest first; with kAhead both
    // blocks' Q and dO slices and lse are requested at once (16 more
    // registers: the one-launch backward loads the second block's after the
    // first block instead).
    const int iA = snake_block(0, wave, x.nb, false);
    if (iA < 0) return;
    const int iB = snake_block(1, wave, x.nb, false);
    struct QIn {
      Slice<bf16_t, KD> qf, gf;
      float ls;
    } in[kAhead ? 2 : 1];
    auto load_in = [&](QIn& d, int i) {
      const int qr = min(kBlk * i + c, x.L - 1);
      d.qf.load(Q + x.at(D) + static_cast<unsigned>(qr * D + KD * g));
      d.gf.load(dO + x.at(D) + static_cast<unsigned>(qr * D + KD * g));
      d.ls = lse[x.tab(H) + static_cast<unsigned>(qr * H)];
    };
    load_in(in[0], iA);
    if constexpr (kAhead) load_in(in[kAhead ? 1 : 0], max(iB, 0));
    auto block = [&](int i, const QIn& qin) {
      const int q = kBlk * i + c;
      const Slice<bf16_t, KD>& qf = qin.qf;
      const Slice<bf16_t, KD>& gf = qin.gf;
      const float l2 = qin.ls * kLog2e;
      f4 dq[MT], dqw[MT];  // Σ a_j k_j and Σ w_j k_j
#pragma unroll
      for (int j = 0; j < MT; ++j) {
        dq[j] = f4{0.0f, 0.0f, 0.0f, 0.0f};
        dqw[j] = dq[j];
      }
      float acc = 0.0f;
      const int tq = min(q, x.L - 1) - 4 * g;  // key 16kb + 4g + r is live iff r <= tq - 16kb
      for (int kb = 0; kb <= i; ++kb) {
        Slice<bf16_t, KD> kf, vf;
        kf.load(Ks + (kBlk * kb + c) * WS + KD * g);
        vf.load(Vs + (kBlk * kb + c) * WS + KD * g);
        const f4 sv = slice_dot(kf, qf, f4{0.0f, 0.0f, 0.0f, 0.0f});  // key 16kb+4g+r against query q
        const f4 tv = slice_dot(vf, gf, f4{0.0f, 0.0f, 0.0f, 0.0f});  // dO_q . v_key
        agpt_blk::bf16x4_bits tkv[MT];  // K^T blocks: dims 16j .., keys 16kb ..
#pragma unroll
        for (int j = 0; j < MT; ++j) tkv[j] = read_tr(Ks, WS, kBlk * kb, kBlk * j, lane);
        __builtin_amdgcn_sched_barrier(0);
        float pw[4], aw[4];
        const int t = tq - kBlk * kb;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          pw[r] = fast_exp2(r <= t ? __builtin_fmaf(sv[r], sfac, -l2) : -__builtin_inff());
          aw[r] = pw[r] * tv[r];
          acc += aw[r];
        }
        const uint2 ph = pack_bf16(pw), ah = pack_bf16(aw);
        const float plo[4] = {pw[0] - __uint_as_float(ph.x << 16), pw[1] - __uint_as_float(ph.x & 0xffff0000u),
                              pw[2] - __uint_as_float(ph.y << 16), pw[3] - __uint_as_float(ph.y & 0xffff0000u)};
        const float alo[4] = {aw[0] - __uint_as_float(ah.x << 16), aw[1] - __uint_as_float(ah.x & 0xffff0000u),
                              aw[2] - __uint_as_float(ah.y << 16), aw[3] - __uint_as_float(ah.y & 0xffff0000u)};
        const uint2 pl2 = pack_bf16(plo), al2 = pack_bf16(alo);
#pragma unroll
        for (int j = 0; j < MT; ++j) {
          dq[j] = mfma_a2_bf16(tkv[j], tkv[j], ah, al2, dq[j]);  // high and low bf16 parts in one step
          dqw[j] = mfma_a2_bf16(tkv[j], tkv[j], ph, pl2, dqw[j]);
        }
      }
      const float dl = group_sum(acc);
      agpt_deep::wait_loads();  // every input has arrived; the next block then starts with no wait
      if (q < x.L) {
        const int pos = rope.cos_t ? rope_pos(q + 1, rope.seq_len) : 0;  // a chain's row q is at depth q + 1
#pragma unroll
        for (int j = 0; j < MT; ++j) {
          float v[4];
#pragma unroll
          for (int r = 0; r < 4; ++r) v[r] = (dq[j][r] - dl * dqw[j][r]) * scale;
          if (rope.cos_t) agpt_fast::rope_inverse_part<4, kHD>(v, rope.cos_t, rope.sin_t, pos, kBlk * j + 4 * g);
          store_vec<4>(dQ + x.at(D) + static_cast<unsigned>(q * D + kBlk * j + 4 * g), v);
        }
        if (g == 0) {
          if (Dl) Dl[x.tab(H) + static_cast<unsigned>(q * H)] = dl;
          if (dls) dls[q] = dl;
        }
      }
    };
    block(iA, in[0]);
    if (iB >= 0) {
      if constexpr (kAhead) {
        block(iB, in[kAhead ? 1 : 0]);
      } else {
        load_in(in[0], iB);
        block(iB, in[0]);
      }
    }
  }
}

template <typename PlanT, typename RopeT>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(4))) void bwd_q_kernel(PlanT pl, const bf16_t* __restrict__ Q,
                                                         const bf16_t* __restrict__ K,
                                                         const bf16_t* __restrict__ V,
                                                         const float* __restrict__ lse,
                                                         const bf16_t* __restrict__ dO, float* __restrict__ dQ,
                                                         float* __restrict__ Dl, RopeT rope, int H, float scale) {
  extern __shared__ __align__(16) unsigned char dyn[];
  bf16_t* Ks = reinterpret_cast<bf16_t*>(dyn);
  bf16_t* Vs = Ks + kRows * WS;
  unit_loop<0>(pl, H, K, V, nullptr, nullptr, Ks, Vs, nullptr, nullptr, [&](const ChainUnit& x) {
    q_side<true>(x, Ks, Vs, Q, lse, dO, dQ, Dl, nullptr, rope, H, scale);
  });
}

// ---------------------------------------------------------------------------
// Backward, key side: dK, dV of key block j against query blocks j .. nb-1,
// the chain's Q and dO rows (and lse, δ) in LDS. S = Q_i K^T puts key c in
// lane column c (queries 4g .. 4g+3 in its registers); dV^T += dO^T P,
// dK^T += Q^T dS with the transposed operands read from the row tiles. dS
// leaves out the softmax scale, applied once per key (a power of two at
// head_dim 64, so the bf16 rounding is unchanged).
// ---------------------------------------------------------------------------
// The key side of unit x (its Q, dO rows in Qs, Gs, lse * log2(e) and δ
// of those rows in l2s, dls): this wave's key blocks.
template <typename RopeT>
__device__ __forceinline__ void kv_side(const ChainUnit& x, const bf16_t* Qs, const bf16_t* Gs, const float* l2s,
                                        const float* dls, const bf16_t* __restrict__ K,
                                        const bf16_t* __restrict__ V, float* __restrict__ dK,
                                        float* __restrict__ dV, const float* __restrict__ acc_dk,
                                        const float* __restrict__ acc_dv, const RopeT& rope, int H, float scale) {
  constexpr int KD = kHD / 4;
  constexpr int MT = kHD / 16;
  const int tid = opaque_tid();
  const int lane = tid & 63;
  const int wave = uniform(tid >> 6);
  const int g = lane >> 4, c = lane & 15;
  const int D = H * kHD;
  const float sfac = scale * kLog2e;
  {
    for (int k = 0;; ++k) {
      const int j = snake_block(k, wave, x.nb, true);
      if (j < 0) break;
      const int key = kBlk * j + c;  // this lane's key (chain index)
      const int kr = min(key, x.L - 1);
      Slice<bf16_t, KD> kf, vf;
      kf.load(K + x.at(D) + static_cast<unsigned>(kr * D + KD * g));
      vf.load(V + x.at(D) + static_cast<unsigned>(kr * D + KD * g));
      f4 dk[MT], dv[MT];
#pragma unroll
      for (int t = 0; t < MT; ++t) {
        dk[t] = f4{0.0f, 0.0f, 0.0f, 0.0f};
        dv[t] = dk[t];
      }
      // query q0 + r sees the key iff key <= q0 + r < L: (q0 + r - key) < len
      // as unsigned, len = L - key (0 for a key past the end)
      const unsigned len = static_cast<unsigned>(max(x.L - key, 0));
      // Query blocks in pairs (i, i + 1), their dV and dK products summed by
      // one 32-deep step per output tile; past the last block the pair's
      // second half reads block i again, with every weight masked to 0.
      for (int i = j; i < x.nb; i += 2) {
        const int ib[2] = {i, min(i + 1, x.nb - 1)};
        uint2 pw[2], dw[2];
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          const int qr = kBlk * ib[h] + c;  // query row this lane supplies
          const int q0 = kBlk * ib[h] + 4 * g;
          const int base = kBlk * (i + h) + 4 * g - key;
          Slice<bf16_t, KD> qa, ga;
          qa.load(Qs + qr * WS + KD * g);
          ga.load(Gs + qr * WS + KD * g);
          const f4 sv = slice_dot(qa, kf, f4{0.0f, 0.0f, 0.0f, 0.0f});  // query q0+r against the key
          const f4 tv = slice_dot(ga, vf, f4{0.0f, 0.0f, 0.0f, 0.0f});
          const f4 l2v = *reinterpret_cast<const f4*>(&l2s[q0]);
          const f4 dlv = *reinterpret_cast<const f4*>(&dls[q0]);
          float p[4], ds[4];
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            p[r] = fast_exp2(static_cast<unsigned>(base + r) < len ? __builtin_fmaf(sv[r], sfac, -l2v[r])
                                                                  : -__builtin_inff());
            ds[r] = p[r] * (tv[r] - dlv[r]);
          }
          pw[h] = pack_bf16(p);
          dw[h] = pack_bf16(ds);
        }
#pragma unroll
        for (int t = 0; t < MT; ++t) {  // dO^T, Q^T blocks: dims 16t .., queries 16 ib[h] ..
          dv[t] = mfma_a2_bf16(read_tr(Gs, WS, kBlk * ib[0], kBlk * t, lane), read_tr(Gs, WS, kBlk * ib[1], kBlk * t, lane),
                               pw[0], pw[1], dv[t]);
          dk[t] = mfma_a2_bf16(read_tr(Qs, WS, kBlk * ib[0], kBlk * t, lane), read_tr(Qs, WS, kBlk * ib[1], kBlk * t, lane),
                               dw[0], dw[1], dk[t]);
        }
      }
      if (key < x.L) {
        const int pos = rope.cos_t ? rope_pos(key + 1, rope.seq_len) : 0;
#pragma unroll
        for (int t = 0; t < MT; ++t) {
          const int d0 = kBlk * t + 4 * g;
          const unsigned ko = static_cast<unsigned>(kr * D + d0);
          float gk[4] = {dk[t][0] * scale, dk[t][1] * scale, dk[t][2] * scale, dk[t][3] * scale};
          float gv[4] = {dv[t][0], dv[t][1], dv[t][2], dv[t][3]};
          if (acc_dk) {
            float y[4];
            load_vec<4>(acc_dk + x.at(D) + ko, y);
#pragma unroll
            for (int e = 0; e < 4; ++e) gk[e] += y[e];
          }
          if (acc_dv) {
            float y[4];
            load_vec<4>(acc_dv + x.at(D) + ko, y);
#pragma unroll
            for (int e = 0; e < 4; ++e) gv[e] += y[e];
          }
          if (rope.cos_t) agpt_fast::rope_inverse_part<4, kHD>(gk, rope.cos_t, rope.sin_t, pos, d0);
          store_vec<4>(dK + x.at(D) + ko, gk);
          store_vec<4>(dV + x.at(D) + ko, gv);
        }
      }
    }
  }
}

template <typename PlanT, typename RopeT>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(4))) void bwd_kv_kernel(
    PlanT pl, const bf16_t* __restrict__ Q, const bf16_t* __restrict__ K, const bf16_t* __restrict__ V,
    const float* __restrict__ lse, const float* __restrict__ Dl, const bf16_t* __restrict__ dO,
    float* __restrict__ dK, float* __restrict__ dV, const float* __restrict__ acc_dk,
    const float* __restrict__ acc_dv, RopeT rope, int H, float scale) {
  __shared__ alignas(16) float l2s[kRows];  // lse * log2(e) of the chain's rows (past the end: the last row's)
  __shared__ alignas(16) float dls[kRows];  // δ of the chain's rows
  extern __shared__ __align__(16) unsigned char dyn[];
  bf16_t* Qs = reinterpret_cast<bf16_t*>(dyn);
  bf16_t* Gs = Qs + kRows * WS;
  unit_loop<kLseDelta>(pl, H, Q, dO, lse, Dl, Qs, Gs, l2s, dls, [&](const ChainUnit& x) {
    kv_side(x, Qs, Gs, l2s, dls, K, V, dK, dV, acc_dk, acc_dv, rope, H, scale);
  });
}

// ---------------------------------------------------------------------------
// Backward in one launch: per unit the query side (dQ, δ) over the chain's
// K, V rows in LDS, then the key side (dK, dV) over its Q, dO rows in the
// same LDS, with δ handed over in LDS. The key side's rows are fetched as
// each wave finishes its query blocks, and stored once every wave has.
// Each key's dK/dV needs the δ of every later row of its chain, which the
// unit has just computed: no δ table in HBM, no second launch, and no
// drain between the two halves (the next unit's query side follows the key
// side's tail on the CU). Results are bitwise those of bwd_q_kernel then
// bwd_kv_kernel.
// ---------------------------------------------------------------------------
template <typename PlanT, typename RopeT>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(4))) void bwd_kernel(
    PlanT pl, const bf16_t* __restrict__ Q, const bf16_t* __restrict__ K, const bf16_t* __restrict__ V,
    const float* __restrict__ lse, const bf16_t* __restrict__ dO, float* __restrict__ dQ,
    float* __restrict__ dK, float* __restrict__ dV, const float* __restrict__ acc_dk,
    const float* __restrict__ acc_dv, RopeT rope, int H, float scale) {
  __shared__ alignas(16) float l2s[kRows];
  __shared__ alignas(16) float dls[kRows];
  extern __shared__ __align__(16) unsigned char dyn[];
  bf16_t* As = reinterpret_cast<bf16_t*>(dyn);  // K then Q rows
  bf16_t* Bs = As + kRows * WS;                 // V then dO rows
  const int D = H * kHD;
  const int64_t n_units = static_cast<int64_t>(pl.n_chains) * H;
  int k = 0;
  int u = dealt_unit(0);
  int2 info = load_info(pl, u, H, n_units);
  while (u < n_units) {
    const int nu = dealt_unit(++k);
    const ChainUnit x = unit_of(info, u, H);
    __builtin_amdgcn_s_setprio(3);  // rows and barriers ahead of block steps, as in unit_loop
    {
      Rows<0> rows;
      rows.fetch(K, V, nullptr, nullptr, x, D, H);
      rows.store(As, Bs, nullptr, nullptr, x);
    }
    const int2 ni = load_info(pl, nu, H, n_units);
    __syncthreads();
    __builtin_amdgcn_s_setprio(0);
    q_side<false>(x, As, Bs, Q, lse, dO, dQ, nullptr, dls, rope, H, scale);
    // (the scheduler would hoist the key side's row loads into the query
    // side, whose registers are already full)
    __builtin_amdgcn_sched_barrier(0);
    __builtin_amdgcn_s_setprio(3);
    {
      Rows<kLseOnly> rows;
      rows.fetch(Q, dO, lse, nullptr, x, D, H);
      __syncthreads();  // every wave is done with the K, V rows; δ of rows < L is in dls
      const int t = opaque_tid();
      if (t >= x.L && t < kRows) dls[t] = 0.0f;  // past the end: finite, and masked to zero weight
      rows.store(As, Bs, l2s, nullptr, x);
    }
    __syncthreads();
    __builtin_amdgcn_s_setprio(0);
    kv_side(x, As, Bs, l2s, dls, K, V, dK, dV, acc_dk, acc_dv, rope, H, scale);
    __syncthreads();  // the unit's rows are no longer read
    u = nu;
    info = ni;
  }
}

}  // namespace agpt_chain
