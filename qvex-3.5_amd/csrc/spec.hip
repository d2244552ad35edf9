// Fused speculative acceptance sampling over the vocabulary.
//
// Reference: engine/speculative.py:74-81 (greedy draft: accept iff U < p(draft),
// resample from p with the draft masked; bonus from the last row) and
// engine/sampler.py:30-58 (temperature softmax, argmax when greedy). Generalised
// to k drafts sampled from a draft distribution q (Leviathan et al. 2023; Chen et
// al. 2023): accept d_i iff u_i * q_i(d_i) < p_i(d_i); at the first rejection n
// sample from max(0, p_n - q_n); if all k pass, sample the bonus from p_k.
// Without draft logits q is one-hot at d_i, which is the reference's rule.
//
// Division-free form, with e = exp(z - max), S = sum(e), z = logits * inv_temp:
//   accept iff (u * e_q(d)) * S_p < e_p(d) * S_q
//   residual weight w_j = max(0, e_p(j) * S_q - e_q(j) * S_p);  bonus w_j = e_p(j)
// Every value is fp32 and the reduction order is fixed, so a CPU emulation
// reproduces accept counts and tokens bit for bit (this unit is built with
// -ffp-contract=off):
//   * a row is cut into parts of 8192; thread t of a 256-thread block owns the
//     elements base + 4*(t + 256*i) + e (i = 0..7, e = 0..3), summed in that order;
//   * thread sums combine by an xor butterfly (32..1) per wave, then
//     ((w0 + w1) + w2) + w3 over the 4 waves;
//   * parts combine as m = max m_p, S = sum_p S_p * exp(m_p - m), left to right;
//   * inverse-CDF sampling walks parts, then threads, then elements with running
//     fp32 prefix sums; if rounding leaves the walk without a hit, the last
//     positive weight of the scope is taken.
//
// Kernel 1 (grid parts x rows) makes one pass over every logit row of every step
// and leaves (m_p, S_p) per part: the single HBM pass over (2k+1) x V floats.
// Kernel 2 (grid parts x steps) combines parts, runs the k accept tests on
// gathered elements and makes the sampling weights' thread and part sums over
// the one or two rows the draw needs, every part in its own block.
// Kernel 3 (one block per step) walks the stored sums to the drawn token.
//
// Filtering of the target rows (Sampler.scores, engine/sampler.py:30-52), when
// asked for: presence penalty x - pen * s(j) with s(j) = 1 for `seen` tokens and,
// in verify row i, for the drafts d_0..d_{i-1} before it; top-k and top-p; every
// token outside z >= cutoff has probability 0. Two forms give (c_0, S_p, cutoff)
// per target row to kernels 2 and 3, which only add the z >= cutoff test:
//   * list form (1 <= top_k <= 64, optional top-p over the top-k): kernel 1 also
//     leaves each part's k largest values (taken one block maximum at a time) and
//     how many of its values equal the k-th; a filter kernel (one block per
//     verify row) merges them into the row's k largest, applies top-p in order
//     and counts the ties at the cutoff exactly;
//   * wide form (64 < top_k < V, or top-p over the whole vocabulary): one
//     1024-thread block per verify row finds the k-th largest value exactly by a
//     radix descent over order-preserving 32-bit keys (11/11/10-bit digits,
//     counts), and the top-p cutoff by a second descent over fixed-point masses
//     m(z) = trunc(exp(z - c_0) * 2^32) (uint64, so the sums are exact and
//     order-free): cutoff = the smallest value v >= v_k with
//     M(> v) < top_p * S_cand (M(> v) = sum of m over z > v; S_cand = the mass of
//     the k candidates, the whole row without top-k), the cumulative rule of
//     engine/sampler.py:47-50 on exact sums. S_p = sum of exp(z - c_0) over
//     z >= cutoff in fp32, in a fixed order (thread t of 1024 owns elements
//     4 (t + 1024 i) + e, summed in (i, e) order; xor butterflies per wave, then
//     the 16 wave sums in wave order).
#include "qvex_common.h"

#include <mutex>

// Workspace of qvex_spec_accept_filtered_bf16_noalloc: one array per GPU, at
// an address looked up once per device (the name is a host-side stand-in, not
// a device address).
static __device__ __align__(256) unsigned char scratch[QVEX_SPEC_SCRATCH_BYTES];

namespace {

constexpr int PART = 8192;
constexpr int NT = 256;
constexpr int NI = 8;   // float4 loads per thread per part

// exp(x): Cody-Waite reduction x = n*ln2 + r with ln2 split in hi/lo parts,
// degree-7 Taylor polynomial for e^r (|r| <= ln2/2) in Horner form with fmaf,
// scaled by 2^n built in the exponent field. Returns 0 below -69 so every
// product formed with it stays in the normal range. Branch-free: the
// polynomial runs on the argument clamped to [-69, 88] (equal to x wherever its
// value is used) and the out-of-range results are selected afterwards, so the
// bits are those of the form that returns early (NaN gives 0 as there).
__device__ __forceinline__ float qx_expf(float x) {
  const float xc = fminf(fmaxf(x, -69.0f), 88.0f);
  const float n = rintf(xc * 1.44269504f);
  float r = fmaf(n, -0.693145751953125f, xc);
  r = fmaf(n, -1.428606765330187e-06f, r);
  float p = 1.0f / 5040.0f;
  p = fmaf(p, r, 1.0f / 720.0f);
  p = fmaf(p, r, 1.0f / 120.0f);
  p = fmaf(p, r, 1.0f / 24.0f);
  p = fmaf(p, r, 1.0f / 6.0f);
  p = fmaf(p, r, 0.5f);
  p = fmaf(p, r, 1.0f);
  p = fmaf(p, r, 1.0f);
  const int e = (int)n;
  const float v = p * __uint_as_float((uint32_t)(e + 127) << 23);
  return x >= -69.0f ? (x > 88.0f ? __builtin_inff() : v) : 0.0f;
}

__device__ __forceinline__ float wave_bfly_sum(float v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v = v + __shfl_xor(v, o, 64);
  return v;
}

// ((w0 + w1) + w2) + w3 of the four wave sums; result valid in every thread.
__device__ __forceinline__ float block_sum(float v, float* red) {
  v = wave_bfly_sum(v);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  __syncthreads();
  if (lane == 0) red[wave] = v;
  __syncthreads();
  return ((red[0] + red[1]) + red[2]) + red[3];
}

__device__ __forceinline__ float block_max(float v, float* red) {
  v = wave_allmax(v);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  __syncthreads();
  if (lane == 0) red[wave] = v;
  __syncthreads();
  return fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
}

template <int CTRL, int ROW_MASK = 0xf, bool BOUND_CTRL = true>
__device__ __forceinline__ int dpp_i(int v) {
  return __builtin_amdgcn_update_dpp(0, v, CTRL, ROW_MASK, 0xf, BOUND_CTRL);
}

// Exclusive prefix sum over the block's threads of v; *total = the sum. sh: 4
// ints. The wave's inclusive scan runs on DPP row shifts and row broadcasts.
__device__ __forceinline__ int block_excl_scan(int v, int* sh, int* total) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  int x = v;
  x += dpp_i<DPP_ROW_SHR(1)>(x);
  x += dpp_i<DPP_ROW_SHR(2)>(x);
  x += dpp_i<DPP_ROW_SHR(4)>(x);
  x += dpp_i<DPP_ROW_SHR(8)>(x);
  x += dpp_i<DPP_ROW_BCAST15, 0xa, false>(x);
  x += dpp_i<DPP_ROW_BCAST31, 0xc, false>(x);
  __syncthreads();
  if (lane == 63) sh[wave] = x;
  __syncthreads();
  int off = 0;
#pragma unroll
  for (int w = 0; w < NT / 64; ++w) off += w < wave ? sh[w] : 0;
  *total = ((sh[0] + sh[1]) + sh[2]) + sh[3];
  return off + x - v;
}

// Candidates kept per part and target row for the one-kernel list form: every
// index with z above the part's k-th value (at most k - 1 <= 63, in slots
// [0, CAND_GT)) and up to CAND_CAP - CAND_GT of the ties at it (slots after)
constexpr int CAND_CAP = 96;
constexpr int CAND_GT = 64;
constexpr int CAND_IT = 16;         // slots per thread of the draw: P * CAND_CAP <= NT * CAND_IT
constexpr int CAND_LIST_FLOATS = 42 * 65;   // the row's part lists in LDS: P (<= 42) x (top_k + 1)

struct SpecArgs {
  const void* target;     // [S, k+1, V] fp32, or bf16 when bf
  const void* draft;      // [S, k, V] or nullptr, same type
  const int32_t* ids;     // [S, k]
  const float* u_acc;     // [S, k]
  const float* u_smp;     // [S]
  float inv_temp;
  int greedy;
  int32_t* n_accept;      // [S]
  int32_t* out_token;     // [S]
  float* ws;              // [S * rps, P, 2]
  int S, k, V, P, rps;    // rps = rows per step
  const float* seen;      // [V] presence mask or nullptr
  float pen;              // presence penalty
  int top_k;              // list form: 1..64; 0 = off (also in the wide form)
  float top_p;            // top-p when 0 < top_p < 1
  float* fws;             // [S * (k+1), P, top_k + 1] part lists + tie counts (list form)
  float* frow;            // [S * (k+1), 4] (c_0, S_p, cutoff)
  int bf;                 // logits are bf16 (widened exactly to fp32 on load)
  int filt;               // 0: no filter, 1: list form, 2: wide form
  int wide_k;             // wide form: top-k (0 = off)
  // list form without draft logits (one kernel after the statistics):
  int fast;
  int32_t* cand;          // [S * (k+1), P, CAND_CAP] indices of z >= the part's k-th value
  float* cand_z;          // [S * (k+1), P, CAND_CAP] their z
  int32_t* ncand;         // [S * (k+1), P, 2] how many the part has above / at its k-th value
  int32_t* ctr;           // [S] blocks of the step that finished their row
  int32_t* rres;          // [S * (k+1), 2] each row's accept flag and draw
  int rows_only;          // one-kernel form: leave (flag, draw) per row in rres; no step decision
};

__device__ __forceinline__ const void* row_ptr(const SpecArgs& a, int step, int i) {
  const long es = a.bf ? 2 : 4;
  // both pointers as opaque values: a choice between the two fields' addresses
  // would keep the argument struct in scratch memory for an indexed load
  const char* tp = (const char*)a.target;
  const char* dp = (const char*)a.draft;
  asm volatile("" : "+v"(tp), "+v"(dp));
  if (i <= a.k) return tp + ((long)step * (a.k + 1) + i) * a.V * es;
  return dp + ((long)step * a.k + (i - a.k - 1)) * a.V * es;
}

// Logit j of a row as fp32 (bf16 rows widen exactly).
__device__ __forceinline__ float lg(const void* row, long j, int bf) {
  return bf ? bf16_to_f32(reinterpret_cast<const uint16_t*>(row)[j]) : reinterpret_cast<const float*>(row)[j];
}

// Presence penalty of a target row at token j: x - pen * s(j), s(j) = 1 for the
// n_extra drafts that precede the row, else seen[j]; no subtraction at all when
// there is no penalty (so the unfiltered rule keeps its bits).
__device__ __forceinline__ float pen_x(const float* seen, float pen, float x, int j, const int32_t* extra,
                                       int n_extra) {
  if (pen == 0.0f || (!seen && n_extra == 0)) return x;
  float sj = seen ? seen[j] : 0.0f;
  for (int q = 0; q < n_extra; ++q)
    if (extra[q] == j) sj = 1.0f;
  return x - pen * sj;
}

// A thread's next NB values in (value descending, slot ascending) order after
// (lv, li), into bv/bi (descending): strictly greater values move ahead, so an
// earlier slot wins a tie. Empty entries are (-inf, NS).
constexpr int TOPK_BUF = 8;
template <int NS>
__device__ __forceinline__ void next_buf(const float (&v)[NS], float lv, int li, float (&bv)[TOPK_BUF],
                                         int (&bi)[TOPK_BUF]) {
#pragma unroll
  for (int e = 0; e < TOPK_BUF; ++e) {
    bv[e] = -__builtin_inff();
    bi[e] = NS;
  }
#pragma unroll
  for (int q = 0; q < NS; ++q) {
    // bitwise, not short-circuit: a per-element branch here is what the
    // compiler makes of ||, and a rescan then costs a branch per slot
    const bool after = (v[q] < lv) | ((v[q] == lv) & (q > li));
    const float x = after ? v[q] : -__builtin_inff();
    bool gt[TOPK_BUF];
#pragma unroll
    for (int e = 0; e < TOPK_BUF; ++e) gt[e] = x > bv[e];
#pragma unroll
    for (int e = TOPK_BUF - 1; e > 0; --e) {
      bv[e] = gt[e - 1] ? bv[e - 1] : (gt[e] ? x : bv[e]);
      bi[e] = gt[e - 1] ? bi[e - 1] : (gt[e] ? q : bi[e]);
    }
    bv[0] = gt[0] ? x : bv[0];
    bi[0] = gt[0] ? q : bi[0];
  }
}

// 1 when value e ranks ahead of v (greater, or equal and `first`), as plain bit
// operations: the short-circuit form compiles to a branch per comparison.
__device__ __forceinline__ int ahead(float e, float v, bool first) {
  return (int)(e > v) | ((int)(e == v) & (int)first);
}

// The K largest of the block's values (with multiplicity) into lst[0..K-1],
// descending; v holds the calling thread's NS values, -inf for none. Each wave
// extracts its own K largest, one wave maximum per round (ties: lowest lane),
// with no block barrier inside the rounds; a thread serves its values from a
// TOPK_BUF-entry buffer and rescans its registers only when the buffer runs
// dry (a lane must win TOPK_BUF rounds first).
// The four sorted lists are then merged by rank: entry i of wave w lands at
// i + #(entries of other waves that are larger, or equal and from a lower
// wave), which is unique. wl: 4 * 64 floats, 16-byte aligned (wave w's list at 64 w).
template <int NS>
__device__ __forceinline__ void block_topk(const float (&v)[NS], int K, float* lst, float* wl) {
  float bv[TOPK_BUF];
  int bi[TOPK_BUF];
  next_buf(v, __builtin_inff(), -1, bv, bi);
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  for (int r = 0; r < K; ++r) {
    const float m = wave_allmax(bv[0]);
    const unsigned long long msk = __ballot(bv[0] == m);
    if (lane == 0) wl[wave * 64 + r] = m;
    if (lane == __ffsll(msk) - 1) {
      const float lv = bv[0];
      const int li = bi[0];
#pragma unroll
      for (int e = 0; e + 1 < TOPK_BUF; ++e) {
        bv[e] = bv[e + 1];
        bi[e] = bi[e + 1];
      }
      bv[TOPK_BUF - 1] = -__builtin_inff();
      bi[TOPK_BUF - 1] = NS;
      if (bi[0] == NS && li < NS) next_buf(v, lv, li, bv, bi);
    }
  }
  __syncthreads();
  if (t < 4 * K) {
    const int w = t / K, r = t - w * K;
    const float x = wl[w * 64 + r];
    int rank = r;
    for (int w2 = 0; w2 < 4; ++w2) {
      if (w2 == w) continue;
      const float4* o = reinterpret_cast<const float4*>(wl + w2 * 64);
      for (int j4 = 0; j4 < (K + 3) / 4; ++j4) {   // four entries per LDS read
        const float4 q = o[j4];
        const float e[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
        for (int i = 0; i < 4; ++i)
          rank += (int)(4 * j4 + i < K) & ahead(e[i], x, w2 < w);
      }
    }
    if (rank < K) lst[rank] = x;
  }
  __syncthreads();
}

__device__ __forceinline__ float readlane_f(float v, int l) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), l));
}

// Threshold selection of a part's K largest values (K <= 64), the same multiset
// block_topk gives, without its K serial rounds. tau = the K-th largest of the
// block's 256 lane maxima (ties by lane): the K lanes whose maxima rank first
// hold K distinct values >= tau, so the part's K-th value is >= tau and every
// value it keeps (and every value equal to the K-th) is among the candidates
// {valid z >= tau} - about K of them for a row of random logits (a lane holds
// 32 of the part's values). tau comes from each wave's K largest lane maxima
// (ranked within the wave), ranked again across the 4K of them. The candidates
// are gathered in LDS and ranked (ties by index). Returns false, with nothing
// written, when more than TK_CMAX values reach tau (rows of equal values, or
// tau = -inf when fewer than K lanes hold a valid value); the caller then runs
// block_topk.
constexpr int TK_CMAX = 512;
struct TopkSh {
  __align__(16) float v[TK_CMAX];
  __align__(16) int j[TK_CMAX];
  __align__(16) float lm[NT];     // lane maxima, wave-major
  float tau[4];
  int scan[8];
  int n;
};

// zz: the thread's 4 * NI values (-inf where !ok), element index of value q is
// jb + 4 * NT * (q >> 2) + (q & 3) with jb = part base + 4 t.
__device__ __forceinline__ bool topk_thresh(const float (&zz)[4 * NI], const bool (&ok)[NI], int jb, int K,
                                            float* lst, TopkSh& S) {
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  float tm = -__builtin_inff();
#pragma unroll
  for (int q = 0; q < 4 * NI; ++q) tm = fmaxf(tm, zz[q]);
  S.lm[t] = tm;
  __syncthreads();
  {
    // rank of this lane's maximum within its wave (ties: lower lane first)
    const float4* w4 = reinterpret_cast<const float4*>(S.lm + wave * 64);
    int r = 0;
#pragma unroll
    for (int q4 = 0; q4 < 16; ++q4) {
      const float4 o = w4[q4];
      const float e[4] = {o.x, o.y, o.z, o.w};
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int l2 = 4 * q4 + i;
        r += ahead(e[i], tm, l2 < lane);
      }
    }
    if (r < K) S.v[wave * K + r] = tm;    // the wave's K largest lane maxima
  }
  __syncthreads();
  if (t < 4 * K) {                      // the K-th largest of the 4K (ties by slot)
    const float v = S.v[t];
    int r = 0;
#pragma unroll 4
    for (int q = 0; q < 4 * K; q += 4) {
      const float4 o = *reinterpret_cast<const float4*>(&S.v[q]);
      const float e[4] = {o.x, o.y, o.z, o.w};
#pragma unroll
      for (int i = 0; i < 4; ++i) r += ahead(e[i], v, q + i < t);
    }
    if (r == K - 1) S.tau[0] = v;
  }
  __syncthreads();
  const float tau = S.tau[0];
  int c = 0;
#pragma unroll
  for (int q = 0; q < 4 * NI; ++q) c += (int)ok[q >> 2] & (int)(zz[q] >= tau);
  int n;
  int off = block_excl_scan(c, S.scan, &n);
  if (n > TK_CMAX) return false;      // block-uniform
#pragma unroll
  for (int q = 0; q < 4 * NI; ++q)
    if (ok[q >> 2] && zz[q] >= tau) {
      S.v[off] = zz[q];
      S.j[off] = jb + 4 * NT * (q >> 2) + (q & 3);
      ++off;
    }
  if (t == 0) S.n = n;
  // pad to a multiple of 8 with entries that never rank ahead (-inf, last index)
  if (t < 8 && n + t < TK_CMAX) {
    S.v[n + t] = -__builtin_inff();
    S.j[n + t] = 0x7fffffff;
  }
  __syncthreads();
  const int n8 = min((n + 7) & ~7, TK_CMAX);
  for (int cc = t; cc < n; cc += NT) {
    const float v = S.v[cc];
    const int j = S.j[cc];
    int r = 0;
#pragma unroll 2
    for (int q = 0; q < n8; q += 8) {     // eight entries per round of two 16-byte reads each
      const float4 va = *reinterpret_cast<const float4*>(&S.v[q]);
      const float4 vb = *reinterpret_cast<const float4*>(&S.v[q + 4]);
      const int4 ja = *reinterpret_cast<const int4*>(&S.j[q]);
      const int4 jb2 = *reinterpret_cast<const int4*>(&S.j[q + 4]);
      const float vv[8] = {va.x, va.y, va.z, va.w, vb.x, vb.y, vb.z, vb.w};
      const int jj[8] = {ja.x, ja.y, ja.z, ja.w, jb2.x, jb2.y, jb2.z, jb2.w};
#pragma unroll
      for (int e = 0; e < 8; ++e) r += ahead(vv[e], v, jj[e] < j);
    }
    if (r < K) lst[r] = v;
  }
  if (t >= n && t < K) lst[t] = -__builtin_inff();   // fewer than K valid values
  __syncthreads();
  return true;
}

// ---------------------------------------------------------------- kernel 1: part statistics

// Part p of row `row` (the block's work in spec_rowstats_kernel); zero_ctr:
// this block clears the one-kernel finish counters (part 0 of row 0).
template <bool BF>
__device__ __forceinline__ void rowstats_block(const SpecArgs& a, int p, int row, bool zero_ctr) {
  __shared__ float red[4];
  __shared__ int redi[4];
  const int step = row / a.rps, i = row % a.rps;
  const void* src = row_ptr(a, step, i);
  const int base = p * PART;
  const int end = min(a.V, base + PART);
  const int t = threadIdx.x;

  float x[NI][4];
  bool ok[NI];
#pragma unroll
  for (int it = 0; it < NI; ++it) {
    const int j = base + 4 * (t + NT * it);
    ok[it] = j < end;
    if (ok[it]) {
      if constexpr (BF) {
        const u32x2 v = __builtin_nontemporal_load(reinterpret_cast<const u32x2*>(
            reinterpret_cast<const uint16_t*>(src) + j));
        x[it][0] = bf16_lo(v.x);
        x[it][1] = bf16_hi(v.x);
        x[it][2] = bf16_lo(v.y);
        x[it][3] = bf16_hi(v.y);
      } else {
        const u32x4 v = load_nt16(reinterpret_cast<const float*>(src) + j);
        x[it][0] = __uint_as_float(v.x);
        x[it][1] = __uint_as_float(v.y);
        x[it][2] = __uint_as_float(v.z);
        x[it][3] = __uint_as_float(v.w);
      }
    }
  }
  const bool tgt = i <= a.k;
  if (tgt && a.pen != 0.0f) {
    const int32_t* extra = a.ids + (long)step * a.k;
#pragma unroll
    for (int it = 0; it < NI; ++it)
      if (ok[it]) {
        const int j = base + 4 * (t + NT * it);
#pragma unroll
        for (int e = 0; e < 4; ++e) x[it][e] = pen_x(a.seen, a.pen, x[it][e], j + e, extra, i);
      }
  }
  float* out = a.ws + ((long)row * a.P + p) * 2;
  if (a.greedy) {
    // first index of the maximum raw logit within the part
    float bv = -__builtin_inff();
    int bj = 0x7fffffff;
#pragma unroll
    for (int it = 0; it < NI; ++it)
      if (ok[it]) {
        const int j = base + 4 * (t + NT * it);
#pragma unroll
        for (int e = 0; e < 4; ++e)
          if (x[it][e] > bv || (x[it][e] == bv && j + e < bj)) { bv = x[it][e]; bj = j + e; }
      }
    const float m = block_max(bv, red);
    int cand = (bv == m) ? bj : 0x7fffffff;
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) cand = min(cand, __shfl_xor(cand, o, 64));
    __syncthreads();
    if ((t & 63) == 0) redi[t >> 6] = cand;
    __syncthreads();
    if (t == 0) {
      out[0] = m;
      out[1] = __int_as_float(min(min(redi[0], redi[1]), min(redi[2], redi[3])));
    }
    return;
  }
  float z[NI][4];
#pragma unroll
  for (int it = 0; it < NI; ++it)
#pragma unroll
    for (int e = 0; e < 4; ++e) z[it][e] = x[it][e] * a.inv_temp;
  // (m_p, S_p) of the part, which the unfiltered rules combine; the list form
  // without draft logits (the finish kernel) takes (c_0, S_p, cutoff) from the
  // lists alone, so its target rows skip the exponentials
  if (!(a.fast && tgt && a.filt == 1)) {
    float m = -__builtin_inff();
#pragma unroll
    for (int it = 0; it < NI; ++it)
      if (ok[it]) {
#pragma unroll
        for (int e = 0; e < 4; ++e) m = fmaxf(m, z[it][e]);
      }
    m = block_max(m, red);
    float acc = 0.0f;
#pragma unroll
    for (int it = 0; it < NI; ++it)
      if (ok[it]) {
#pragma unroll
        for (int e = 0; e < 4; ++e) acc = acc + qx_expf(z[it][e] - m);
      }
    const float s = block_sum(acc, red);
    if (t == 0) {
      out[0] = m;
      out[1] = s;
    }
  }
  if (tgt && a.filt == 1) {
    // this part's top_k largest z and the count of its values equal to the k-th
    __shared__ float lst[64];
    __shared__ __align__(16) float wl[4 * 64];
    __shared__ TopkSh tks;
    const int K = a.top_k;
    float zz[4 * NI];
#pragma unroll
    for (int q = 0; q < 4 * NI; ++q) zz[q] = ok[q >> 2] ? z[q >> 2][q & 3] : -__builtin_inff();
    const bool thr = topk_thresh(zz, ok, base + 4 * t, K, lst, tks);
    float* L = a.fws + (((long)step * (a.k + 1) + i) * a.P + p) * (K + 1);
    const long crow = (long)step * (a.k + 1) + i;
    if (thr) {
      // every value equal to the K-th is a candidate: the tie count and the
      // stored candidates come from the gathered values alone
      const float vk = lst[K - 1];
      const int n = tks.n;
      int ceq = 0;
      for (int cc = t; cc < n; cc += NT) ceq += tks.v[cc] == vk ? 1 : 0;
      int neq_total;
      block_excl_scan(ceq, tks.scan, &neq_total);
      if (t < K) L[t] = lst[t];
      if (t == 0) L[K] = (float)neq_total;
      if (a.fast) {
        __shared__ int c_gt2, c_eq2;
        if (t == 0) {
          c_gt2 = 0;
          c_eq2 = 0;
        }
        __syncthreads();
        int32_t* C = a.cand + (crow * a.P + p) * CAND_CAP;
        float* Zc = a.cand_z + (crow * a.P + p) * CAND_CAP;
        for (int cc = t; cc < n; cc += NT) {
          const float zv = tks.v[cc];
          if (zv > vk) {
            const int q = atomicAdd(&c_gt2, 1);           // < K - 1 <= CAND_GT
            C[q] = tks.j[cc];
            Zc[q] = zv;
          } else if (zv == vk) {
            const int q = atomicAdd(&c_eq2, 1);
            if (q < CAND_CAP - CAND_GT) {
              C[CAND_GT + q] = tks.j[cc];
              Zc[CAND_GT + q] = zv;
            }
          }
        }
        __syncthreads();
        if (t == 0) {
          a.ncand[(crow * a.P + p) * 2] = c_gt2;
          a.ncand[(crow * a.P + p) * 2 + 1] = c_eq2;
        }
        if (zero_ctr && p == 0 && row == 0)
          for (int q = t; q < a.S; q += NT) a.ctr[q] = 0;
      }
      return;
    }
    block_topk(zz, K, lst, wl);
    const float vk = lst[K - 1];
    float cnt = 0.0f;
#pragma unroll
    for (int it = 0; it < NI; ++it)
      if (ok[it]) {
#pragma unroll
        for (int e = 0; e < 4; ++e) cnt += (z[it][e] == vk) ? 1.0f : 0.0f;
      }
    cnt = block_sum(cnt, red);
    if (t < K) L[t] = lst[t];
    if (t == 0) L[K] = cnt;
    if (a.fast) {
      // the part's indices and z above vk, then up to CAND_CAP - CAND_GT of those
      // equal to vk, in any order (the consumer orders them): the row's kept set
      // (z >= cutoff, cutoff >= every part's vk) lies in them unless the part
      // holds more ties and the cutoff is vk itself
      __shared__ int c_gt, c_eq;
      if (t == 0) {
        c_gt = 0;
        c_eq = 0;
      }
      __syncthreads();
      int32_t* C = a.cand + (crow * a.P + p) * CAND_CAP;
      float* Zc = a.cand_z + (crow * a.P + p) * CAND_CAP;
#pragma unroll
      for (int it = 0; it < NI; ++it)
        if (ok[it]) {
          const int j = base + 4 * (t + NT * it);
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const float zv = z[it][e];
            if (zv > vk) {
              const int q = atomicAdd(&c_gt, 1);          // < K - 1 <= CAND_GT
              C[q] = j + e;
              Zc[q] = zv;
            } else if (zv == vk) {
              const int q = atomicAdd(&c_eq, 1);
              if (q < CAND_CAP - CAND_GT) {
                C[CAND_GT + q] = j + e;
                Zc[CAND_GT + q] = zv;
              }
            }
          }
        }
      __syncthreads();
      if (t == 0) {
        a.ncand[(crow * a.P + p) * 2] = c_gt;
        a.ncand[(crow * a.P + p) * 2 + 1] = c_eq;
      }
      if (zero_ctr && p == 0 && row == 0)
        for (int q = t; q < a.S; q += NT) a.ctr[q] = 0;
    }
  }
}

template <bool BF>
__global__ __launch_bounds__(NT) void spec_rowstats_kernel(SpecArgs a) {
  rowstats_block<BF>(a, blockIdx.x, blockIdx.y, true);
}

// ---------------------------------------------------------------- filter kernel (top-k / top-p)

// One block per verify row: the row's top_k largest values from the parts'
// lists, the top-p cutoff over them in order (exp(c_i - c_0) / S, running sums
// r_i, keep iff r_i - p_i < top_p, cutoff = min kept c_i), and
// S_p = sum_{c_i > cutoff} exp(c_i - c_0) + n_eq * exp(cutoff - c_0) with n_eq the
// row's count of values equal to the cutoff: a part whose k-th value is the
// cutoff contributes its tie count, any other part its list entries equal to it
// (the cutoff is never below a part's k-th value).
__device__ __forceinline__ void filter_row(const SpecArgs& a, int row, float* lst, float* wl, float& cut_s,
                                           int& neq_s) {
  const int K = a.top_k, P = a.P;
  const int n = P * K;                  // <= 16 * NT, checked by the host
  const float* L = a.fws + (long)row * P * (K + 1);
  const int t = threadIdx.x;
  // candidate i = t + NT * q in slot q: four slots cover n <= 1024 (the
  // 9B vocabulary's 31 parts x top-k 20), sixteen the rest; the list is the same
  float v[16];
#pragma unroll
  for (int q = 0; q < 16; ++q) {
    const int i = t + NT * q;
    const int pp = i / K;
    v[q] = i < n ? L[pp * (K + 1) + (i - pp * K)] : -__builtin_inff();
  }
  if (n <= 4 * NT) {
    const float v4[4] = {v[0], v[1], v[2], v[3]};
    block_topk(v4, K, lst, wl);
  } else {
    block_topk(v, K, lst, wl);
  }
  // Wave 0 holds the candidates c_i = lst[i] and e_i = exp(c_i - c_0) one per
  // lane; the ordered sums run over them with readlane, in index order.
  const int lane = t & 63;
  const float c0 = lst[0];
  const float cl = lane < K ? lst[lane] : -__builtin_inff();
  const float el = lane < K ? qx_expf(cl - c0) : 0.0f;
  if (t < 64) {
    float cutoff = lst[K - 1];
    if (a.top_p > 0.0f && a.top_p < 1.0f) {
      float Ssum = 0.0f;
      for (int q = 0; q < K; ++q) Ssum = Ssum + readlane_f(el, q);
      const float pl = el / Ssum;
      float run = 0.0f, mn = __builtin_inff();
      for (int q = 0; q < K; ++q) {
        const float pi = readlane_f(pl, q);
        const float cq = readlane_f(cl, q);
        const float incl = run + pi;
        if ((incl - pi) < a.top_p && cq < mn) mn = cq;
        run = incl;
      }
      cutoff = mn;
    }
    if (t == 0) {
      cut_s = cutoff;
      neq_s = 0;
    }
  }
  __syncthreads();
  // Values equal to the cutoff: a part whose K-th value is the cutoff
  // contributes its tie count (every element of the part equal to that value),
  // any other part its list entries equal to it. Integer sum, so order-free.
  const float cutoff = cut_s;
  int my_eq = 0;
#pragma unroll
  for (int q = 0; q < 16; ++q) {
    const int i = t + NT * q;
    if (i < n && v[q] == cutoff) {
      const int pp = i / K;
      if (L[pp * (K + 1) + K - 1] != cutoff) ++my_eq;
    }
  }
  for (int q = t; q < P; q += NT)
    if (L[q * (K + 1) + K - 1] == cutoff) my_eq += (int)L[q * (K + 1) + K];
  if (my_eq) atomicAdd(&neq_s, my_eq);
  __syncthreads();
  if (t < 64) {
    // lst is descending, so the values above the cutoff are a prefix
    const int n_gt = __popcll(__ballot(lane < K && cl > cutoff));
    float S = 0.0f;
    for (int q = 0; q < n_gt; ++q) S = S + readlane_f(el, q);
    S = S + (float)neq_s * qx_expf(cutoff - c0);
    if (t == 0) {
      float* fr = a.frow + (long)row * 4;
      fr[0] = c0;
      fr[1] = S;
      fr[2] = cutoff;
    }
  }
}

__global__ __launch_bounds__(NT) void spec_filter_kernel(SpecArgs a) {
  __shared__ float lst[64];
  __shared__ __align__(16) float wl[4 * 64];
  __shared__ float cut_s;
  __shared__ int neq_s;
  filter_row(a, blockIdx.x, lst, wl, cut_s, neq_s);   // row = step * (k + 1) + i
}

// ---------------------------------------------------------------- wide filter (top-k > 64, top-p over the vocabulary)

constexpr int WT = 1024;        // threads of a wide-filter block
constexpr int WB = 2048;        // buckets per radix level (11-bit digits)

// order-preserving key: a < b as floats iff okey(a) < okey(b) (no NaN)
__device__ __forceinline__ uint32_t okey(float z) {
  const uint32_t u = __float_as_uint(z);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}
__device__ __forceinline__ float okey_val(uint32_t k) {
  return __uint_as_float((k & 0x80000000u) ? (k & 0x7fffffffu) : ~k);
}
// fixed-point mass of a value: trunc(exp(z - c0) * 2^32), <= 2^32
__device__ __forceinline__ uint64_t fx_mass(float z, float c0) {
  return (uint64_t)(qx_expf(z - c0) * 4294967296.0f);
}

// The four values of thread t's group i (elements 4 (t + WT i) .. + 3) of a
// target row as z = penalised logit * inv_temp.
struct WRow {
  const void* src;
  int bf;
  const float* seen;
  float pen;
  const int32_t* extra;
  int n_extra;
  float inv_temp;
};

__device__ __forceinline__ void wide_z4(const WRow& r, int j, float (&z)[4]) {
  if (r.bf) {
    const u32x2 v = *reinterpret_cast<const u32x2*>(reinterpret_cast<const uint16_t*>(r.src) + j);
    z[0] = bf16_lo(v.x);
    z[1] = bf16_hi(v.x);
    z[2] = bf16_lo(v.y);
    z[3] = bf16_hi(v.y);
  } else {
    const u32x4 v = *reinterpret_cast<const u32x4*>(reinterpret_cast<const float*>(r.src) + j);
    z[0] = __uint_as_float(v.x);
    z[1] = __uint_as_float(v.y);
    z[2] = __uint_as_float(v.z);
    z[3] = __uint_as_float(v.w);
  }
#pragma unroll
  for (int e = 0; e < 4; ++e) z[e] = pen_x(r.seen, r.pen, z[e], j + e, r.extra, r.n_extra) * r.inv_temp;
}

__device__ __forceinline__ uint64_t shfl_down_u64(uint64_t v, int o) {
  const uint32_t lo = __shfl_down((uint32_t)v, o, 64), hi = __shfl_down((uint32_t)(v >> 32), o, 64);
  return ((uint64_t)hi << 32) | lo;
}

// Exclusive suffix sum over the block's threads: sum of v over threads t' > t.
__device__ __forceinline__ uint64_t block_suffix_excl(uint64_t v, uint64_t* sh) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  uint64_t x = v;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const uint64_t y = shfl_down_u64(x, o);
    if (lane + o < 64) x += y;
  }
  __syncthreads();
  if (lane == 0) sh[wave] = x;
  __syncthreads();
  uint64_t hi = 0;
  for (int w = wave + 1; w < WT / 64; ++w) hi += sh[w];
  return x - v + hi;
}

// One block per target row (grid S * (k + 1)): (c_0, S_p, cutoff) into frow.
__global__ __launch_bounds__(WT) void spec_wide_filter_kernel(SpecArgs a) {
  __shared__ unsigned long long hmass[WB];
  __shared__ uint32_t hcnt[WB];
  __shared__ uint64_t sh[WT / 64];
  __shared__ float shf[WT / 64];
  __shared__ int s_pick;
  __shared__ uint64_t s_val;
  const int row = blockIdx.x;                   // step * (k + 1) + i
  const int step = row / (a.k + 1), i = row % (a.k + 1);
  const int t = threadIdx.x;
  WRow r;
  r.src = row_ptr(a, step, i);
  r.bf = a.bf;
  r.seen = a.seen;
  r.pen = a.pen;
  r.extra = a.ids + (long)step * a.k;
  r.n_extra = i;
  r.inv_temp = a.inv_temp;
  const int V = a.V;
  // c_0: the maximum of the part maxima kernel 1 left (order-free)
  const float* pw = a.ws + ((long)step * a.rps + i) * a.P * 2;
  float c0 = -__builtin_inff();
  for (int q = 0; q < a.P; ++q) c0 = fmaxf(c0, pw[2 * q]);

  const int shifts[3] = {21, 10, 0};
  const int widths[3] = {11, 11, 10};

  // ---- k-th largest value (counts): after the descent kk is its key, n_gt the
  // count of larger values and n_eq the count of values equal to it
  uint32_t kk = 0;
  uint32_t n_gt = 0, n_eq = 0;
  const int K = a.wide_k;
  if (K > 0) {
    uint32_t prefix = 0, pmask = 0;
    uint32_t need = (uint32_t)K;                // rank among the values matching the prefix
    for (int lv = 0; lv < 3; ++lv) {
      const int sft = shifts[lv];
      const uint32_t dmask = (1u << widths[lv]) - 1u;
      for (int b = t; b < WB; b += WT) hcnt[b] = 0;
      __syncthreads();
      for (int j = 4 * t; j < V; j += 4 * WT) {
        float z[4];
        wide_z4(r, j, z);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const uint32_t key = okey(z[e]);
          if ((key & pmask) == prefix) atomicAdd(&hcnt[(key >> sft) & dmask], 1u);
        }
      }
      __syncthreads();
      // thread t owns buckets 2t, 2t + 1; the bucket holding the need-th largest
      const uint32_t c_lo = hcnt[2 * t], c_hi = hcnt[2 * t + 1];
      const uint64_t above = block_suffix_excl((uint64_t)c_lo + c_hi, sh);
      if (t == 0) s_pick = -1;
      __syncthreads();
      if (above < need && need <= above + c_hi) {
        s_pick = 2 * t + 1;
        s_val = above;
      } else if (above + c_hi < need && need <= above + c_hi + c_lo) {
        s_pick = 2 * t;
        s_val = above + c_hi;
      }
      __syncthreads();
      const int bsel = s_pick;
      need -= (uint32_t)s_val;
      prefix |= (uint32_t)bsel << sft;
      pmask |= dmask << sft;
      if (lv == 2) n_eq = hcnt[bsel];
      __syncthreads();
    }
    kk = prefix;
    n_gt = (uint32_t)K - need;
  }
  const float vk = K > 0 ? okey_val(kk) : -__builtin_inff();

  // ---- top-p cutoff over the candidates (fixed-point masses, exact sums)
  float cutoff = vk;
  if (a.top_p > 0.0f && a.top_p < 1.0f) {
    const uint32_t kmin = K > 0 ? kk : 0u;      // values below v_k are not candidates
    uint32_t prefix = 0, pmask = 0;
    uint64_t base = 0;                          // mass of candidates above the prefix's range
    double T = 0.0;
    for (int lv = 0; lv < 3; ++lv) {
      const int sft = shifts[lv];
      const uint32_t dmask = (1u << widths[lv]) - 1u;
      for (int b = t; b < WB; b += WT) {
        hmass[b] = 0;
        hcnt[b] = 0;
      }
      __syncthreads();
      for (int j = 4 * t; j < V; j += 4 * WT) {
        float z[4];
        wide_z4(r, j, z);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const uint32_t key = okey(z[e]);
          if (key >= kmin && (key & pmask) == prefix) {
            const uint32_t b = (key >> sft) & dmask;
            atomicAdd(&hmass[b], (unsigned long long)fx_mass(z[e], c0));
            atomicAdd(&hcnt[b], 1u);
          }
        }
      }
      __syncthreads();
      const uint64_t m_lo = hmass[2 * t], m_hi = hmass[2 * t + 1];
      const uint64_t above = block_suffix_excl(m_lo + m_hi, sh);
      if (lv == 0) {
        // S_cand: every candidate is in this level's histogram; with top-k the
        // values equal to v_k count only up to the k candidates
        uint64_t total = above + m_lo + m_hi;   // thread 0 holds the whole sum
        if (t == 0) s_val = total;
        __syncthreads();
        total = s_val;
        if (K > 0) {
          const uint64_t mk = fx_mass(vk, c0);
          total = total - (uint64_t)n_eq * mk + (uint64_t)(K - n_gt) * mk;
        }
        T = (double)a.top_p * (double)total;
        __syncthreads();
      }
      // lowest non-empty bucket whose largest value still has M(> v) < T
      if (t == 0) s_pick = 0x7fffffff;
      __syncthreads();
      if (hcnt[2 * t] && (double)(base + above + m_hi) < T) atomicMin(&s_pick, 2 * t);
      else if (hcnt[2 * t + 1] && (double)(base + above) < T) atomicMin(&s_pick, 2 * t + 1);
      __syncthreads();
      const int bsel = s_pick;
      if (bsel == 2 * t) s_val = above + m_hi;
      if (bsel == 2 * t + 1) s_val = above;
      __syncthreads();
      base += s_val;
      prefix |= (uint32_t)bsel << sft;
      pmask |= dmask << sft;
      __syncthreads();
    }
    cutoff = okey_val(prefix);
  }

  // ---- S_p = sum of exp(z - c0) over z >= cutoff, fixed order
  float acc = 0.0f;
  for (int j = 4 * t; j < V; j += 4 * WT) {
    float z[4];
    wide_z4(r, j, z);
#pragma unroll
    for (int e = 0; e < 4; ++e) acc = acc + (z[e] >= cutoff ? qx_expf(z[e] - c0) : 0.0f);
  }
  acc = wave_bfly_sum(acc);
  if ((t & 63) == 0) shf[t >> 6] = acc;
  __syncthreads();
  if (t == 0) {
    float S = shf[0];
    for (int w = 1; w < WT / 64; ++w) S = S + shf[w];
    float* fr = a.frow + (long)row * 4;
    fr[0] = c0;
    fr[1] = S;
    fr[2] = cutoff;
  }
}

// ---------------------------------------------------------------- kernel 2: accept + sample

struct WCtx {
  const void* tp;
  const void* tq;
  int bf;
  int d;
  int mode;   // 0 residual, 1 plain p
  float inv_temp, mp, sp, mq, sq;
  float cutoff;             // -inf when the target row is not filtered
  const float* seen;        // presence penalty of the target row
  float pen;
  const int32_t* extra;
  int n_extra;
};

__device__ __forceinline__ float weight(const WCtx& c, int j) {
  const float z = pen_x(c.seen, c.pen, lg(c.tp, j, c.bf), j, c.extra, c.n_extra) * c.inv_temp;
  const float ep = z >= c.cutoff ? qx_expf(z - c.mp) : 0.0f;
  if (c.mode == 1) return ep;
  float eq, Sq;
  if (c.tq) {
    eq = qx_expf(lg(c.tq, j, c.bf) * c.inv_temp - c.mq);
    Sq = c.sq;
  } else {
    eq = (j == c.d) ? 1.0f : 0.0f;
    Sq = 1.0f;
  }
  const float t1 = ep * Sq;
  const float t2 = eq * c.sp;
  const float r = t1 - t2;
  return r > 0.0f ? r : 0.0f;
}

// weight() of a one-hot draft from the element's z (the value the statistics
// kernel stored for it: the same penalised logit times 1/T, so the same bits)
__device__ __forceinline__ float weight_z(const WCtx& c, int j, float z) {
  const float ep = z >= c.cutoff ? qx_expf(z - c.mp) : 0.0f;
  if (c.mode == 1) return ep;
  const float eq = (j == c.d) ? 1.0f : 0.0f;
  const float t1 = ep * 1.0f;
  const float t2 = eq * c.sp;
  const float r = t1 - t2;
  return r > 0.0f ? r : 0.0f;
}

// Inverse-CDF draw over the fixed order; returns -1 when every weight is 0.
__device__ int sample_pass(const WCtx& c, int V, int P, float u, float* Tpt, float* Wp, float* red) {
  const int t = threadIdx.x;
  for (int p = 0; p < P; ++p) {
    const int base = p * PART, end = min(V, base + PART);
    float acc = 0.0f;
#pragma unroll
    for (int it = 0; it < NI; ++it) {
      const int j = base + 4 * (t + NT * it);
      if (j < end) {
#pragma unroll
        for (int e = 0; e < 4; ++e) acc = acc + weight(c, j + e);
      }
    }
    Tpt[p * NT + t] = acc;
    const float w = block_sum(acc, red);
    if (t == 0) Wp[p] = w;
  }
  __syncthreads();
  __shared__ int result;
  if (t == 0) {
    float W = 0.0f;
    for (int p = 0; p < P; ++p) W = W + Wp[p];
    int res = -1;
    if (W > 0.0f) {
      const float th = u * W;
      float cacc = 0.0f;
      int ps = -1;
      for (int p = 0; p < P; ++p) {
        const float nx = cacc + Wp[p];
        if (nx > th) { ps = p; break; }
        cacc = nx;
      }
      bool fallback = false;
      if (ps < 0) {
        for (int p = P - 1; p >= 0; --p)
          if (Wp[p] > 0.0f) { ps = p; break; }
        fallback = true;
      }
      int ts = -1;
      if (!fallback) {
        for (int tt = 0; tt < NT; ++tt) {
          const float nx = cacc + Tpt[ps * NT + tt];
          if (nx > th) { ts = tt; break; }
          cacc = nx;
        }
      }
      if (ts < 0) {
        for (int tt = NT - 1; tt >= 0; --tt)
          if (Tpt[ps * NT + tt] > 0.0f) { ts = tt; break; }
        fallback = true;
      }
      const int base = ps * PART, end = min(V, base + PART);
      if (!fallback) {
        for (int s = 0; s < 4 * NI; ++s) {
          const int j = base + 4 * (ts + NT * (s >> 2)) + (s & 3);
          if (j >= end) break;
          cacc = cacc + weight(c, j);
          if (cacc > th) { res = j; break; }
        }
      }
      if (res < 0) {
        for (int s = 4 * NI - 1; s >= 0; --s) {
          const int j = base + 4 * (ts + NT * (s >> 2)) + (s & 3);
          if (j < end && weight(c, j) > 0.0f) { res = j; break; }
        }
      }
    }
    result = res;
  }
  __syncthreads();
  return result;
}

// Workspace after the row statistics: per step T[P][NT] thread sums of the
// sampling row, W[P] part sums and a decision record (n, mode, stats).
struct SpecWs {
  float* T;     // [S][P][NT]
  float* W;     // [S][P]
  float* dec;   // [S][8]: n, draft id, mp, sp, mq, sq, cutoff
};

__device__ __forceinline__ SpecWs spec_ws(const SpecArgs& a) {
  SpecWs w;
  w.T = a.ws + (long)a.S * a.rps * a.P * 2;
  w.W = w.T + (long)a.S * a.P * NT;
  w.dec = w.W + (long)a.S * a.P;
  return w;
}

// Kernel 2 (grid parts x steps): every block combines the step's row statistics
// and runs the k accept tests (a few gathers), then block p makes the thread and
// part sums of the sampling weights over part p of the sampling row.
__global__ __launch_bounds__(NT) void spec_decide_kernel(SpecArgs a) {
  __shared__ float rm[80], rs[80], rc[80];
  __shared__ float red[4];
  __shared__ int s_n, s_tok;
  const int p = blockIdx.x, step = blockIdx.y;
  const int t = threadIdx.x;
  const int k = a.k;
  const SpecWs W = spec_ws(a);

  // per-row statistics from the parts, one wave per row: lane q holds part q
  // (parts 64 apart in later rounds). Greedy: the first part holding the row
  // maximum gives the index (the serial rule "strictly greater replaces");
  // sampling: m = max, S = sum_q S_q e^{m_q - m} added in part order.
  {
    const int lane = t & 63, wave = t >> 6;
    for (int r = wave; r < a.rps; r += NT / 64) {
      const float* w = a.ws + ((long)step * a.rps + r) * a.P * 2;
      float cut = -__builtin_inff(), mr = 0.0f, sr = 0.0f;
      if (!a.greedy && a.filt != 0 && r <= k) {
        const float* fr = a.frow + ((long)step * (k + 1) + r) * 4;
        mr = fr[0];
        sr = fr[1];
        cut = fr[2];
      } else if (a.greedy) {
        float bv = -__builtin_inff();
        int bj = 0;
        for (int q0 = 0; q0 < a.P; q0 += 64) {
          const int q = q0 + lane;
          const float v = q < a.P ? w[2 * q] : -__builtin_inff();
          const int j = q < a.P ? __float_as_int(w[2 * q + 1]) : 0;
          const float m = wave_allmax(v);
          const unsigned long long hit = __ballot(q < a.P && v == m);
          const int src = __ffsll(hit) - 1;
          const int jm = __builtin_amdgcn_readlane(j, src);
          if (q0 == 0 || m > bv) { bv = m; bj = jm; }
        }
        mr = __int_as_float(bj);
      } else {
        float m = -__builtin_inff();
        for (int q0 = 0; q0 < a.P; q0 += 64) {
          const int q = q0 + lane;
          m = fmaxf(m, wave_allmax(q < a.P ? w[2 * q] : -__builtin_inff()));
        }
        float sum = 0.0f;
        for (int q0 = 0; q0 < a.P; q0 += 64) {
          const int q = q0 + lane;
          const float term = q < a.P ? w[2 * q + 1] * qx_expf(w[2 * q] - m) : 0.0f;
          const int n = min(64, a.P - q0);
          for (int i = 0; i < n; ++i) sum = sum + __int_as_float(__builtin_amdgcn_readlane(__float_as_int(term), i));
        }
        mr = m;
        sr = sum;
      }
      if (lane == 0) {
        rm[r] = mr;
        rs[r] = sr;
        rc[r] = cut;
      }
    }
  }
  __syncthreads();
  // the k accept tests, one thread each (their gathers in flight together);
  // thread 0 then takes the first rejection, as the serial rule does
  __shared__ int s_ok[32];
  if (!a.greedy && t < k) {
    const int i = t;
    const int32_t* d = a.ids + (long)step * k;
    const int di = d[i];
    int ok = 0;
    if (!(di < 0 || di >= a.V)) {
      const float zd = pen_x(a.seen, a.pen, lg(row_ptr(a, step, i), di, a.bf), di, d, i) * a.inv_temp;
      const float ep = zd >= rc[i] ? qx_expf(zd - rm[i]) : 0.0f;
      float eq = 1.0f, Sq = 1.0f;
      if (a.draft) {
        eq = qx_expf(lg(row_ptr(a, step, k + 1 + i), di, a.bf) * a.inv_temp - rm[k + 1 + i]);
        Sq = rs[k + 1 + i];
      }
      const float lhs = a.u_acc[(long)step * k + i] * eq * rs[i];
      const float rhs = ep * Sq;
      ok = lhs < rhs ? 1 : 0;
    }
    s_ok[i] = ok;
  }
  __syncthreads();
  if (t == 0) {
    const int32_t* d = a.ids + (long)step * k;
    int n = k, tok = -1;
    if (a.greedy) {
      for (int i = 0; i < k; ++i) {
        const int am = __float_as_int(rm[i]);
        if (am != d[i]) { n = i; tok = am; break; }
      }
      if (n == k) tok = __float_as_int(rm[k]);
    } else {
      for (int i = 0; i < k; ++i)
        if (!s_ok[i]) { n = i; break; }
    }
    s_n = n;
    s_tok = tok;
  }
  __syncthreads();
  const int n = s_n;
  if (a.greedy) {
    if (p == 0 && t == 0) {
      a.n_accept[step] = n;
      a.out_token[step] = s_tok;
    }
    return;
  }
  WCtx c;
  c.inv_temp = a.inv_temp;
  c.tp = row_ptr(a, step, n);
  c.bf = a.bf;
  c.mp = rm[n];
  c.sp = rs[n];
  c.cutoff = rc[n];
  c.seen = a.seen;
  c.pen = a.pen;
  c.extra = a.ids + (long)step * k;
  c.n_extra = n;
  if (n < k) {
    c.tq = a.draft ? row_ptr(a, step, k + 1 + n) : nullptr;
    c.d = a.ids[(long)step * k + n];
    c.mode = 0;
    c.mq = a.draft ? rm[k + 1 + n] : 0.0f;
    c.sq = a.draft ? rs[k + 1 + n] : 1.0f;
  } else {
    c.tq = nullptr;
    c.d = -1;
    c.mode = 1;
    c.mq = 0.0f;
    c.sq = 1.0f;
  }
  const int base = p * PART, end = min(a.V, base + PART);
  float acc = 0.0f;
#pragma unroll
  for (int it = 0; it < NI; ++it) {
    const int j = base + 4 * (t + NT * it);
    if (j < end) {
#pragma unroll
      for (int e = 0; e < 4; ++e) acc = acc + weight(c, j + e);
    }
  }
  W.T[((long)step * a.P + p) * NT + t] = acc;
  const float wp = block_sum(acc, red);
  if (t == 0) {
    W.W[(long)step * a.P + p] = wp;
    if (p == 0) {
      float* dd = W.dec + (long)step * 8;
      dd[0] = __int_as_float(n);
      dd[1] = __int_as_float(c.d);
      dd[2] = c.mp; dd[3] = c.sp; dd[4] = c.mq; dd[5] = c.sq;
      dd[6] = c.cutoff;
    }
  }
}

// Kernel 3 (one block per step): inverse-CDF walk over the stored part and
// thread sums; the last 32 weights are recomputed for the element walk. If the
// residual vanished in fp32 the block falls back to sampling p_n itself.
__global__ __launch_bounds__(NT) void spec_sample_kernel(SpecArgs a) {
  extern __shared__ float smem[];
  float* Tpt = smem;              // [P][NT] (fallback pass only)
  float* Wp = smem + a.P * NT;    // [P]
  __shared__ float red[4];
  __shared__ int s_tok;
  const int step = blockIdx.x;
  const int t = threadIdx.x;
  const int k = a.k;
  const SpecWs W = spec_ws(a);
  const float* dd = W.dec + (long)step * 8;
  const int n = __float_as_int(dd[0]);
  WCtx c;
  c.inv_temp = a.inv_temp;
  c.tp = row_ptr(a, step, n);
  c.bf = a.bf;
  c.d = __float_as_int(dd[1]);
  c.mp = dd[2]; c.sp = dd[3]; c.mq = dd[4]; c.sq = dd[5];
  c.cutoff = dd[6];
  c.seen = a.seen;
  c.pen = a.pen;
  c.extra = a.ids + (long)step * k;
  c.n_extra = n;
  c.tq = (n < k && a.draft) ? row_ptr(a, step, k + 1 + n) : nullptr;
  c.mode = n < k ? 0 : 1;
  const float u = a.u_smp[step];
  // The walks are sequential fp32 sums (the fixed order), done by thread 0, but
  // over values the block first stages in LDS: the part sums, then the chosen
  // part's thread sums, then the chosen thread's element weights.
  const float* Ws = W.W + (long)step * a.P;
  const float* Ts = W.T + (long)step * a.P * NT;
  float* sT = Tpt;                  // [NT] (Tpt is rebuilt by the fallback pass)
  float* sW = Wp;                   // [P]
  __shared__ float sE[4 * NI];
  __shared__ float s_cacc, s_th, s_Wt;
  __shared__ int s_ps, s_ts, s_fb;
  for (int p = t; p < a.P; p += NT) sW[p] = Ws[p];
  __syncthreads();
  if (t == 0) {
    float Wt = 0.0f;
    for (int p = 0; p < a.P; ++p) Wt = Wt + sW[p];
    int ps = -1;
    bool fallback = false;
    float cacc = 0.0f, th = 0.0f;
    if (Wt > 0.0f) {
      th = u * Wt;
      // eight values per LDS round trip; the adds stay sequential
      for (int p0 = 0; p0 < a.P && ps < 0; p0 += 8) {
        float r[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) r[e] = p0 + e < a.P ? sW[p0 + e] : 0.0f;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          if (ps < 0 && p0 + e < a.P) {
            const float nx = cacc + r[e];
            if (nx > th) ps = p0 + e;
            else cacc = nx;
          }
        }
      }
      if (ps < 0) {
        for (int p = a.P - 1; p >= 0; --p)
          if (sW[p] > 0.0f) { ps = p; break; }
        fallback = true;
      }
    }
    s_Wt = Wt;
    s_th = th;
    s_cacc = cacc;
    s_ps = ps;
    s_fb = fallback ? 1 : 0;
  }
  __syncthreads();
  const int ps = s_ps;
  if (ps >= 0) sT[t] = Ts[ps * NT + t];
  __syncthreads();
  if (t == 0 && ps >= 0) {
    bool fallback = s_fb != 0;
    float cacc = s_cacc;
    const float th = s_th;
    int ts = -1;
    if (!fallback) {
      for (int t0 = 0; t0 < NT && ts < 0; t0 += 8) {
        float r[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) r[e] = sT[t0 + e];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          if (ts < 0) {
            const float nx = cacc + r[e];
            if (nx > th) ts = t0 + e;
            else cacc = nx;
          }
        }
      }
    }
    if (ts < 0) {
      for (int tt = NT - 1; tt >= 0; --tt)
        if (sT[tt] > 0.0f) { ts = tt; break; }
      fallback = true;
    }
    s_ts = ts;
    s_fb = fallback ? 1 : 0;
    s_cacc = cacc;
  }
  __syncthreads();
  const int base = ps * PART, end = min(a.V, base + PART);
  const int ts = ps >= 0 ? s_ts : -1;
  if (ts >= 0 && t < 4 * NI) {
    const int j = base + 4 * (ts + NT * (t >> 2)) + (t & 3);
    sE[t] = j < end ? weight(c, j) : 0.0f;
  }
  __syncthreads();
  if (t == 0) {
    int res = -1;
    if (s_Wt > 0.0f && ts >= 0) {
      const float th = s_th;
      float cacc = s_cacc;
      if (!s_fb) {
        bool stop = false;
        for (int q0 = 0; q0 < 4 * NI && !stop; q0 += 8) {
          float r[8];
#pragma unroll
          for (int e = 0; e < 8; ++e) r[e] = sE[q0 + e];
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            const int j = base + 4 * (ts + NT * ((q0 + e) >> 2)) + ((q0 + e) & 3);
            if (!stop) {
              if (j >= end) {
                stop = true;
              } else {
                cacc = cacc + r[e];
                if (cacc > th) { res = j; stop = true; }
              }
            }
          }
        }
      }
      if (res < 0) {
        for (int q = 4 * NI - 1; q >= 0; --q) {
          const int j = base + 4 * (ts + NT * (q >> 2)) + (q & 3);
          if (j < end && sE[q] > 0.0f) { res = j; break; }
        }
      }
    }
    s_tok = res;
  }
  __syncthreads();
  int tok = s_tok;
  if (tok < 0 && c.mode == 0) {     // residual vanished: sample p_n
    c.mode = 1;
    tok = sample_pass(c, a.V, a.P, u, Tpt, Wp, red);
  }
  if (t == 0) {
    a.n_accept[step] = n;
    a.out_token[step] = tok;
  }
}

// ---------------------------------------------------------------- one kernel after the statistics (list form)

// The sampling walk's order (parts, then threads, then each thread's (i, e)) as
// one integer: key = ((part * NT + thread) * NI + i) * 4 + e, so key >> 5 is the
// thread slot, key >> 11 its wave quarter and key >> 13 the part.
__device__ __forceinline__ int walk_key(int j) {
  const int p = j / PART, l = j - p * PART;
  return ((p * NT + ((l >> 2) & (NT - 1))) * NI + (l >> 10)) * 4 + (l & 3);
}
__device__ __forceinline__ int key_index(int key) {
  return (key >> 13) * PART + 4 * (((key >> 5) & (NT - 1)) + NT * ((key >> 2) & (NI - 1))) + (key & 3);
}

struct SparseSh {
  int key[NT];          // positive weights, in arrival order
  float w[NT];
  int skey[NT];         // the same in walk order
  float sw[NT];
  float ssum[NT];       // at the first entry of a thread slot: the slot's thread sum
  int gstart[NT];       // first entry of each (part, quarter) group
  float gsum[NT];       // the group's wave butterfly sum
  int pstart[NT];       // first group of each part present
  float psum[NT];       // the part's block sum
  int scan[8];
  int n, fb, ng, np;
};

// A row's stored candidates, requested at kernel start: thread t holds slots
// t + NT q (unused slots hold stale values, dropped by the counts) and, for
// t < P, part t's tie count.
struct CandRegs {
  int j[CAND_IT], ngt[CAND_IT], neq[CAND_IT];
  float z[CAND_IT];
  int part_neq;
};

__device__ __forceinline__ void load_cands(const SpecArgs& a, long crow, CandRegs& r) {
  const int t = threadIdx.x, P = a.P;
  const int* cn = a.ncand + crow * P * 2;
  const int32_t* cl = a.cand + crow * P * CAND_CAP;
  const float* cz = a.cand_z + crow * P * CAND_CAP;
#pragma unroll
  for (int q = 0; q < CAND_IT; ++q) {
    const int i = min(t + NT * q, P * CAND_CAP - 1), p = i / CAND_CAP;
    r.j[q] = cl[i];
    r.z[q] = cz[i];
    r.ngt[q] = cn[2 * p];
    r.neq[q] = cn[2 * p + 1];
  }
  r.part_neq = cn[2 * min(t, P - 1) + 1];
}

// The draw of the fixed-order walk (spec_decide_kernel + spec_sample_kernel)
// from the candidate lists alone. Weights outside the kept set are zero and
// x + 0 = x exactly in fp32, so every thread sum, wave butterfly, part sum and
// running prefix of the walk over the whole row equals the same operations over
// the positive weights only, applied in walk order with the same tree: thread
// sums from 0 in (i, e) order, each wave quarter through wave_bfly_sum with the
// absent threads as zeros, parts as ((q0 + q1) + q2) + q3, then the walks.
// lists: the row's part lists in LDS ([P][K + 1]). Returns the token, -1 when
// no weight is positive, -2 when the lists do not hold every kept index (a
// part with more than CAND_CAP - CAND_GT ties at a cutoff equal to its k-th
// value) or more than NT weights are positive.
__device__ __forceinline__ int sparse_sample(const SpecArgs& a, const WCtx& c, const CandRegs& r, const float* lists,
                                             float u, SparseSh& L) {
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const int K = a.top_k, P = a.P;
  if (t == 0) {
    L.n = 0;
    L.fb = 0;
  }
  __syncthreads();
  if (t < P && r.part_neq > CAND_CAP - CAND_GT && !(c.cutoff > lists[t * (K + 1) + K - 1])) L.fb = 1;
#pragma unroll
  for (int q = 0; q < CAND_IT; ++q) {
    const int i = t + NT * q;
    if (i < P * CAND_CAP) {
      const int sl = i % CAND_CAP;
      const bool stored = sl < CAND_GT ? sl < r.ngt[q] : sl - CAND_GT < r.neq[q];
      if (stored && r.z[q] >= c.cutoff) {
        const float w = weight_z(c, r.j[q], r.z[q]);
        if (w > 0.0f) {
          const int e = atomicAdd(&L.n, 1);
          if (e < NT) {
            L.key[e] = walk_key(r.j[q]);
            L.w[e] = w;
          }
        }
      }
    }
  }
  __syncthreads();
  const int n = L.n;
  if (L.fb || n > NT) return -2;
  if (n == 0) return -1;
  if (t < n) {                          // keys are distinct: rank = position in walk order
    const int key = L.key[t];
    int r = 0;
    for (int q = 0; q < n; ++q) r += L.key[q] < key ? 1 : 0;
    L.skey[r] = key;
    L.sw[r] = L.w[t];
  }
  __syncthreads();
  bool gfirst = false;
  if (t < n) {
    const int key = L.skey[t];
    if (t == 0 || (L.skey[t - 1] >> 5) != (key >> 5)) {
      float acc = 0.0f;
      for (int q = t; q < n && (L.skey[q] >> 5) == (key >> 5); ++q) acc = acc + L.sw[q];
      L.ssum[t] = acc;
    }
    gfirst = t == 0 || (L.skey[t - 1] >> 11) != (key >> 11);
  }
  int ng;
  const int gi = block_excl_scan(gfirst ? 1 : 0, L.scan, &ng);
  if (gfirst) L.gstart[gi] = t;
  __syncthreads();
  for (int g = wave; g < ng; g += NT / 64) {
    const int s0 = L.gstart[g], s1 = g + 1 < ng ? L.gstart[g + 1] : n;
    float v = 0.0f;
    for (int q = s0; q < s1; ++q) {
      const int key = L.skey[q];
      const bool first = q == 0 || (L.skey[q - 1] >> 5) != (key >> 5);
      if (first && ((key >> 5) & 63) == lane) v = L.ssum[q];
    }
    v = wave_bfly_sum(v);
    if (lane == 0) L.gsum[g] = v;
  }
  __syncthreads();
  bool pfirst = false;
  if (t < ng) pfirst = t == 0 || (L.skey[L.gstart[t - 1]] >> 13) != (L.skey[L.gstart[t]] >> 13);
  int np;
  const int pi = block_excl_scan(pfirst ? 1 : 0, L.scan, &np);
  if (pfirst) {
    const int part = L.skey[L.gstart[t]] >> 13;
    float b0 = 0.0f, b1 = 0.0f, b2 = 0.0f, b3 = 0.0f;
    for (int g = t; g < ng && (L.skey[L.gstart[g]] >> 13) == part; ++g) {
      const int q = (L.skey[L.gstart[g]] >> 11) & 3;
      const float v = L.gsum[g];
      b0 = q == 0 ? v : b0;
      b1 = q == 1 ? v : b1;
      b2 = q == 2 ? v : b2;
      b3 = q == 3 ? v : b3;
    }
    L.psum[pi] = ((b0 + b1) + b2) + b3;
    L.pstart[pi] = t;
  }
  __syncthreads();
  // the walks of spec_sample_kernel, over the positive entries only
  __shared__ int s_res;
  if (t == 0) {
    float Wt = 0.0f;
    for (int q = 0; q < np; ++q) Wt = Wt + L.psum[q];
    const float th = u * Wt;
    float cacc = 0.0f;
    int ps = -1;
    for (int q = 0; q < np; ++q) {
      const float nx = cacc + L.psum[q];
      if (nx > th) { ps = q; break; }
      cacc = nx;
    }
    bool fallback = false;
    if (ps < 0) {                       // every present part is positive: the last one
      ps = np - 1;
      fallback = true;
    }
    const int e0 = L.gstart[L.pstart[ps]];
    const int e1 = ps + 1 < np ? L.gstart[L.pstart[ps + 1]] : n;
    int ts = -1;                        // entry index of the chosen slot's first entry
    if (!fallback) {
      for (int q = e0; q < e1; ++q) {
        if (q != e0 && (L.skey[q - 1] >> 5) == (L.skey[q] >> 5)) continue;
        const float nx = cacc + L.ssum[q];
        if (nx > th) { ts = q; break; }
        cacc = nx;
      }
    }
    if (ts < 0) {                       // the last slot of the part
      for (int q = e0; q < e1; ++q)
        if (q == e0 || (L.skey[q - 1] >> 5) != (L.skey[q] >> 5)) ts = q;
      fallback = true;
    }
    int res = -1, last = ts;
    for (int q = ts; q < e1 && (L.skey[q] >> 5) == (L.skey[ts] >> 5); ++q) {
      last = q;
      if (!fallback && res < 0) {
        cacc = cacc + L.sw[q];
        if (cacc > th) res = q;
      }
    }
    if (res < 0) res = last;            // the slot's last positive weight
    s_res = key_index(L.skey[res]);
  }
  __syncthreads();
  return s_res;
}

// The filter of spec_filter_kernel for one row in wave 0, from the row's part
// lists in LDS (fl, [P][K + 1], P <= 64): the row's K largest values come from a
// tournament over the lists' heads (one lane per part, one wave maximum per
// round), the same multiset as the block merge; then the top-p cutoff, the
// ties at it and S_p exactly as there. Results in (c0, S, cutoff).
__device__ __forceinline__ void filter_wave(const SpecArgs& a, const float* fl, float& c0_out, float& S_out,
                                            float& cut_out) {
  const int lane = threadIdx.x & 63, K = a.top_k, P = a.P;
  const float* my = fl + min(lane, P - 1) * (K + 1);
  int ptr = 0;
  float h = lane < P ? my[0] : -__builtin_inff();
  float hn = lane < P && K > 1 ? my[1] : -__builtin_inff();
  float cl = -__builtin_inff();
  for (int r = 0; r < K; ++r) {
    const float m = wave_allmax(h);
    cl = lane == r ? m : cl;
    const unsigned long long hit = __ballot(h == m);
    if (lane == __ffsll(hit) - 1) {
      ++ptr;
      h = hn;
      hn = lane < P && ptr + 1 < K ? my[ptr + 1] : -__builtin_inff();
    }
  }
  const float c0 = readlane_f(cl, 0);
  const float el = lane < K ? qx_expf(cl - c0) : 0.0f;
  float cutoff = readlane_f(cl, K - 1);
  if (a.top_p > 0.0f && a.top_p < 1.0f) {
    float Ssum = 0.0f;
    for (int q = 0; q < K; ++q) Ssum = Ssum + readlane_f(el, q);
    const float pl = el / Ssum;
    float run = 0.0f, mn = __builtin_inff();
    for (int q = 0; q < K; ++q) {
      const float pi = readlane_f(pl, q);
      const float cq = readlane_f(cl, q);
      const float incl = run + pi;
      if ((incl - pi) < a.top_p && cq < mn) mn = cq;
      run = incl;
    }
    cutoff = mn;
  }
  // ties at the cutoff: a part whose K-th value is the cutoff contributes its
  // tie count, any other part its list entries equal to it (integer, order-free)
  int eq = 0;
  if (lane < P) {
    if (my[K - 1] == cutoff) {
      eq = (int)my[K];
    } else {
#pragma unroll 8
      for (int q = 0; q < K; ++q) eq += my[q] == cutoff ? 1 : 0;
    }
  }
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) eq += __shfl_xor(eq, o, 64);
  const int n_gt = __popcll(__ballot(lane < K && cl > cutoff));
  float S = 0.0f;
  for (int q = 0; q < n_gt; ++q) S = S + readlane_f(el, q);
  S = S + (float)eq * qx_expf(cutoff - c0);
  c0_out = c0;
  S_out = S;
  cut_out = cutoff;
}

// List form without draft logits, one block per target row i of a step: the
// row's filter, its accept test (i < k: spec_decide_kernel's rule) and its draw
// (i < k: the residual at a rejection there, falling back to p_i when it
// vanishes; i = k: the bonus) from the candidate lists, or from the full
// fixed-order pass when the lists do not hold the kept set. The last block of
// the step (a device-scope counter, zeroed by the statistics kernel) takes the
// first rejection's draw, or the bonus.
// Target row `row`'s filter, accept test and draw (the block's work in
// spec_finish_kernel) from the statistics kernel's part lists and candidates;
// the flag and token are returned to every thread. smem: the full pass's
// [P][NT] thread sums and [P] part sums.
__device__ __forceinline__ void finish_row(const SpecArgs& a, int row, float* smem, int& ok_out, int& tok_out) {
  __shared__ float fl[CAND_LIST_FLOATS];
  __shared__ float s_c0, s_S, s_cut;
  __shared__ SparseSh sh;
  __shared__ float red[4];
  __shared__ int s_ok, s_tok;
  const int k = a.k, step = row / (k + 1), i = row - step * (k + 1);
  const int t = threadIdx.x, K = a.top_k, P = a.P;
  // requests first: the part lists, the candidates, the draft's logit
  const float* L = a.fws + (long)row * P * (K + 1);
  float lv[CAND_LIST_FLOATS / NT + 1];
#pragma unroll
  for (int q = 0; q < CAND_LIST_FLOATS / NT + 1; ++q) lv[q] = L[min(t + NT * q, P * (K + 1) - 1)];
  CandRegs cr;
  load_cands(a, row, cr);
  const int32_t* d = a.ids + (long)step * k;
  const int di = i < k ? d[i] : -1;
  const bool din = i < k && !(di < 0 || di >= a.V);
  const float xd = din ? lg(row_ptr(a, step, i), di, a.bf) : 0.0f;
  const float ua = i < k ? a.u_acc[(long)step * k + i] : 0.0f;
  const float u = a.u_smp[step];
#pragma unroll
  for (int q = 0; q < CAND_LIST_FLOATS / NT + 1; ++q)
    if (t + NT * q < P * (K + 1)) fl[t + NT * q] = lv[q];
  __syncthreads();
  if (t < 64) {
    float c0, S, cut;
    filter_wave(a, fl, c0, S, cut);
    if (t == 0) {
      s_c0 = c0;
      s_S = S;
      s_cut = cut;
      float* fr = a.frow + (long)row * 4;
      fr[0] = c0;
      fr[1] = S;
      fr[2] = cut;
    }
  }
  __syncthreads();
  WCtx c;
  c.inv_temp = a.inv_temp;
  c.tp = row_ptr(a, step, i);
  c.tq = nullptr;
  c.bf = a.bf;
  c.mp = s_c0;
  c.sp = s_S;
  c.cutoff = s_cut;
  c.seen = a.seen;
  c.pen = a.pen;
  c.extra = d;
  c.n_extra = i;
  c.d = i < k ? di : -1;
  c.mode = i < k ? 0 : 1;
  c.mq = 0.0f;
  c.sq = 1.0f;
  int ok = 0;
  if (din) {
    const float zd = pen_x(a.seen, a.pen, xd, di, d, i) * a.inv_temp;
    const float ep = zd >= c.cutoff ? qx_expf(zd - c.mp) : 0.0f;
    const float eq = 1.0f, Sq = 1.0f;
    const float lhs = ua * eq * c.sp;
    const float rhs = ep * Sq;
    ok = lhs < rhs ? 1 : 0;
  }
  int tok = sparse_sample(a, c, cr, fl, u, sh);
  if (tok == -1 && c.mode == 0) {       // residual vanished: sample p_i
    c.mode = 1;
    tok = sparse_sample(a, c, cr, fl, u, sh);
  }
  while (tok == -2) {                   // the full pass in the mode reached, then p_i if needed
    tok = sample_pass(c, a.V, P, u, smem, smem + P * NT, red);
    if (tok < 0 && c.mode == 0) {
      c.mode = 1;
      tok = -2;
    }
  }
  if (t == 0) {
    s_ok = ok;
    s_tok = tok;
  }
  __syncthreads();
  ok_out = s_ok;
  tok_out = s_tok;
}

// Thread 0 of each target row's block: store the row's (accept flag, draw) and
// count the row in; the last row of the step to arrive (a device-scope
// acquire-release counter) takes the first rejection's draw, or the bonus, and
// puts the counter back to 0, so the counters are zero between calls.
__device__ __forceinline__ void finish_decide(const SpecArgs& a, int row, int ok, int tok) {
  const int k = a.k, step = row / (k + 1);
  a.rres[2 * row] = ok;
  a.rres[2 * row + 1] = tok;
  const int old = __hip_atomic_fetch_add(a.ctr + step, 1, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT);
  if (old == k) {
    // every row of the step is in (their results read after the acquire)
    int n = k;
    for (int r = 0; r < k; ++r)
      if (!a.rres[2 * (step * (k + 1) + r)]) {
        n = r;
        break;
      }
    a.n_accept[step] = n;
    a.out_token[step] = a.rres[2 * (step * (k + 1) + n) + 1];
    __hip_atomic_store(a.ctr + step, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
}

__global__ __launch_bounds__(NT) void spec_finish_kernel(SpecArgs a) {
  extern __shared__ float smem[];
  int ok, tok;
  finish_row(a, blockIdx.x, smem, ok, tok);
  if (threadIdx.x == 0) finish_decide(a, blockIdx.x, ok, tok);
}


// ---------------------------------------------------------------- list form from tile maxima (one kernel)

// The list form without draft logits and without a presence penalty, given
// each target row's 16-column tile maxima (the bf16 maximum of logits
// 16 t .. 16 t + 15, which the verify lm_head's epilogue writes): one block per
// target row finds its top_k and every value at or above the k-th from the few
// tiles that can hold them, instead of a pass over the row.
//   * tau = the top_k-th largest of the block's NT thread maxima of the tile
//     maxima (ties by thread): top_k tiles hold a value >= tau, so the row's
//     k-th value v_k >= tau, and every logit >= v_k lies in a tile whose maximum
//     is >= tau (z = x / T keeps the order of distinct bf16 logits);
//   * those tiles' logits >= tau are gathered and ranked (z descending, index
//     ascending): the first top_k are the row's k largest values, and every
//     value equal to one of them is in the gathered set, so the ties at the
//     cutoff are counted exactly;
//   * the filter is filter_wave's arithmetic on those values (the same
//     sequential sums), the accept test is spec_decide_kernel's, and the kept
//     set (z >= cutoff) is the first n_gt + ties entries, drawn through the
//     fixed-order walk over its positive weights (sparse_sample's sums, here in
//     one wave: tile_walk).
// More candidate tiles or values than fit, or more than 64 kept values, send
// the row through the two-kernel path's code in this block (every part's
// statistics, then finish_row). The last row of a step to finish takes the
// decision (finish_decide).
constexpr int TM_PER = 8;      // 16-byte loads of 8 tile maxima per thread: NT * 64 = 16384 tiles
constexpr int TM_CT = 256;     // candidate tiles
constexpr int TM_CE = 512;     // candidate values

struct TmSh {
  __align__(16) float ev[TM_CE];       // candidate values (z) and indices, gathered
  __align__(16) int ej[TM_CE];
  __align__(16) float sv[TM_CE];       // the same ranked
  __align__(16) int sj[TM_CE];
  __align__(16) uint32_t ek[TM_CE];     // candidates' rank keys
  int tiles[TM_CT];                    // candidate tiles, wave w's in [64 w, 64 w + 64)
  int scan[8];
  uint32_t tauw[4];
  int wcnt[4];                         // each wave's candidate tiles
  float f[3];                          // c_0, S_p, cutoff
  int ok, tok, nkeep;
  // the draw, wave 0
  __align__(16) int wkey[64];
  int skey[64];
  float sw[64];
  int slot_key[64], slot_first[64];
  float slot_sum[64];
  int grp_key[64], grp_first[64];
  float grp_sum[64];
  float part_sum[64];
  int part_first[64];
};

// Orders a wave's LDS writes before its later reads of other lanes' entries
// (LDS serves one wave's requests in order; this keeps the compiler from
// moving the accesses across).
__device__ __forceinline__ void wave_lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

__device__ __forceinline__ int rl_i(int v, int l) { return __builtin_amdgcn_readlane(v, l); }
__device__ __forceinline__ float rl_f(float v, int l) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), l));
}

// 16-bit key of the bf16 in the low half of h with the order of the values
// (negative values flipped, positive ones above them), NaN mapped to 0, below
// every value
__device__ __forceinline__ uint32_t bf16_key(uint32_t h) {
  h &= 0xffffu;
  const uint32_t neg = (uint32_t)((int32_t)(h << 16) >> 31);
  const uint32_t kk = (h ^ (neg | 0x8000u)) & 0xffffu;
  uint32_t d = 0x7f80u - (h & 0x7fffu);                   // negative: exponent all ones, mantissa non-zero
  asm("" : "+v"(d));
  return kk & ((d >> 31) - 1u);
}
// a >= b and a > b for keys below 2^31, as 0/1 from the sign of a difference
// (the empty asm keeps the compiler from turning it back into a compare, whose
// lane masks it would keep in scalar registers)
__device__ __forceinline__ int key_ge(uint32_t a, uint32_t b) {
  uint32_t d = a - b;
  asm("" : "+v"(d));
  return (int)((d >> 31) ^ 1u);
}
__device__ __forceinline__ int key_gt(uint32_t a, uint32_t b) {
  uint32_t d = b - a;
  asm("" : "+v"(d));
  return (int)(d >> 31);
}

// The fixed-order walk's draw over n <= 64 positive weights in one wave: lane
// e < n holds the e-th in walk-key order (key kv, weight wv). The sums are
// sparse_sample's (spec_sample_kernel's with every zero weight dropped, x + 0 =
// x): a thread slot's sum from 0 in key order; a (part, wave quarter) group's
// sum through the full pass's xor butterfly, which with one or two non-zero
// lanes is that lane or their sum (a + b = b + a), and with more is the
// butterfly itself, run on the slots' lanes; a part's ((q0 + q1) + q2) + q3;
// then the walk over parts, the chosen part's slots and the chosen slot's
// elements with running prefixes, each the sequential fp32 chain. Slots, groups
// and parts are found by ballots over the sorted keys. Returns the drawn index
// in every lane.
__device__ int tile_walk(int n, int kv, float wv, float u, TmSh& S) {
  const int lane = threadIdx.x & 63;
  const bool valid = lane < n;
  const unsigned long long upto = lane == 63 ? ~0ull : ((2ull << lane) - 1ull);   // lanes <= lane
  const int prv = lane > 0 ? lane - 1 : 0, nxl = lane < 63 ? lane + 1 : 63;
  // slots (key >> 5)
  const int kp = __shfl(kv, prv, 64), kn = __shfl(kv, nxl, 64);
  const bool sfirst = valid && (lane == 0 || (kp >> 5) != (kv >> 5));
  const bool slast = valid && (lane == n - 1 || (kn >> 5) != (kv >> 5));
  const unsigned long long fm = __ballot(sfirst);
  const int ns = __popcll(fm);
  const int si = __popcll(fm & upto) - 1;                   // this entry's slot
  const int pos = valid ? lane - (63 - __clzll(fm & upto)) : 0;
  int maxpos = pos;
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) maxpos = max(maxpos, __shfl_xor(maxpos, o, 64));
  float run = wv;                                           // 0 + w = w
  for (int d = 1; d <= maxpos; ++d) {                       // slots of several weights, in order
    const float prev = __shfl(run, prv, 64);
    run = pos == d ? prev + wv : run;
  }
  if (sfirst) {
    S.slot_key[si] = kv;
    S.slot_first[si] = lane;
  }
  if (slast) S.slot_sum[si] = run;
  wave_lds_sync();
  const bool vs = lane < ns;
  const int sk = vs ? S.slot_key[lane] : 0x7fffffff;
  const float ss = vs ? S.slot_sum[lane] : 0.0f;
  const int sfl = vs ? S.slot_first[lane] : n;
  // groups (key >> 11): consecutive slots
  const int skp = __shfl(sk, prv, 64);
  const bool gfirst = vs && (lane == 0 || (skp >> 11) != (sk >> 11));
  const unsigned long long gm = __ballot(gfirst);
  const int ng = __popcll(gm);
  const unsigned long long gabove = gm & ~upto;
  const int gnext = gabove ? __ffsll((long long)gabove) - 1 : ns;
  const int m = gnext - lane;
  const float ss1 = __shfl(ss, nxl, 64);
  float gs = m == 1 ? ss : ss + ss1;
  unsigned long long big = __ballot(gfirst && m >= 3);
  while (big) {                                             // three or more slots: the butterfly itself
    const int g0 = __ffsll((long long)big) - 1;
    big &= big - 1;
    const int g1 = rl_i(gnext, g0);
    float x = 0.0f;
    for (int q = g0; q < g1; ++q) {
      const int L = (rl_i(sk, q) >> 5) & 63;
      x = lane == L ? rl_f(ss, q) : x;
    }
    const float v = rl_f(wave_bfly_sum(x), 0);
    gs = lane == g0 ? v : gs;
  }
  const int gi = __popcll(gm & upto) - 1;
  if (gfirst) {
    S.grp_key[gi] = sk;
    S.grp_sum[gi] = gs;
    S.grp_first[gi] = lane;
  }
  wave_lds_sync();
  const bool vg = lane < ng;
  const int gk = vg ? S.grp_key[lane] : 0x7fffffff;
  const float gv = vg ? S.grp_sum[lane] : 0.0f;
  const int gfl = vg ? S.grp_first[lane] : ns;
  // parts (key >> 13): ((q0 + q1) + q2) + q3 over a part's (at most four) groups
  const int gkp = __shfl(gk, prv, 64);
  const bool pfirst = vg && (lane == 0 || (gkp >> 13) != (gk >> 13));
  const unsigned long long pm = __ballot(pfirst);
  const int np = __popcll(pm);
  float b0 = 0.0f, b1 = 0.0f, b2 = 0.0f, b3 = 0.0f;
#pragma unroll
  for (int dd = 0; dd < 4; ++dd) {
    const int src = min(lane + dd, 63);
    const int gkd = __shfl(gk, src, 64);
    const float gvd = __shfl(gv, src, 64);
    if (lane + dd < ng && (gkd >> 13) == (gk >> 13)) {
      const int q = (gkd >> 11) & 3;
      b0 = q == 0 ? gvd : b0;
      b1 = q == 1 ? gvd : b1;
      b2 = q == 2 ? gvd : b2;
      b3 = q == 3 ? gvd : b3;
    }
  }
  const int pi = __popcll(pm & upto) - 1;
  if (pfirst) {
    S.part_sum[pi] = ((b0 + b1) + b2) + b3;
    S.part_first[pi] = lane;
  }
  wave_lds_sync();
  const float pv = lane < np ? S.part_sum[lane] : 0.0f;
  const int pfl = lane < np ? S.part_first[lane] : ng;
  // the walk over parts: the running prefix, sequential from 0
  float acc = 0.0f, pre = 0.0f;
  for (int q = 0; q < np; ++q) {
    acc = acc + rl_f(pv, q);
    pre = lane == q ? acc : pre;
  }
  const float th = u * acc;
  const unsigned long long hit = __ballot(lane < np && pre > th);
  bool fallback = hit == 0ull;
  const int ps = fallback ? np - 1 : __ffsll((long long)hit) - 1;
  float cacc = ps > 0 ? rl_f(pre, ps - 1) : 0.0f;
  const int gA = rl_i(pfl, ps), gB = ps + 1 < np ? rl_i(pfl, ps + 1) : ng;
  const int sA = rl_i(gfl, gA), sB = gB < ng ? rl_i(gfl, gB) : ns;
  int ts = -1;
  if (!fallback) {
    for (int q = sA; q < sB; ++q) {
      const float nx = cacc + rl_f(ss, q);
      if (nx > th) {
        ts = q;
        break;
      }
      cacc = nx;
    }
  }
  if (ts < 0) {                                             // the part's last slot
    ts = sB - 1;
    fallback = true;
  }
  const int eA = rl_i(sfl, ts), eB = ts + 1 < ns ? rl_i(sfl, ts + 1) : n;
  int res = -1;
  if (!fallback) {
    for (int e = eA; e < eB; ++e) {
      cacc = cacc + rl_f(wv, e);
      if (cacc > th) {
        res = e;
        break;
      }
    }
  }
  if (res < 0) res = eB - 1;                                // the slot's last positive weight
  return key_index(rl_i(kv, res));
}

// A row the one-kernel form's fast path cannot finish, in its block: every
// part's statistics, then the finish (the two-kernel path's code). Outlined, so
// that the fast path keeps its own register allocation; the arguments travel by
// value and the result comes back as (ok, tok).
__device__ __noinline__ int2 tiles_full_row(const SpecArgs& a, int row) {
  extern __shared__ float smem[];
  for (int p = 0; p < a.P; ++p) {
    rowstats_block<true>(a, p, row, false);
    __syncthreads();
  }
  int ok, tok;
  finish_row(a, row, smem, ok, tok);
  return make_int2(ok, tok);
}

// The tile maxima's pointer and count come first, as scalar arguments: the
// first 14 dwords of scalar kernel arguments arrive preloaded in SGPRs (an
// aggregate never does), so the row's tile-maxima loads go out at wave start
// instead of after a round trip for the argument struct. The kernel-argument
// segment then holds them and the struct as this mirror does.
struct TilesKernArgs {
  const uint16_t* tmax;
  int tiles;
  SpecArgs a;
};
constexpr size_t TILES_ARGS_OFFSET = offsetof(TilesKernArgs, a);
static_assert(TILES_ARGS_OFFSET == 16, "kernel-argument layout of spec_tiles_kernel");

__global__ __launch_bounds__(NT) void spec_tiles_kernel(const uint16_t* __restrict__ tmax, int tiles, SpecArgs a) {
  __shared__ TmSh S;
  const int row = blockIdx.x;
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  // requests first: the row's tile maxima (thread t: tiles 8 (t + NT q) + 0..7),
  // from the preloaded arguments alone (nothing may be scheduled ahead of them,
  // or they would wait for the argument struct's loads), then the draft's logit
  // and the uniforms
  const uint16_t* tr = tmax + (long)row * tiles;
  u32x4 tv[TM_PER];
#pragma unroll
  for (int q = 0; q < TM_PER; ++q) tv[q] = load16(tr + min(8 * (t + NT * q), tiles - 8));
  __builtin_amdgcn_sched_barrier(0);
  const int k = a.k, step = row / (k + 1), i = row - step * (k + 1);
  const int K = a.top_k;
  const uint16_t* xr = reinterpret_cast<const uint16_t*>(row_ptr(a, step, i));
  const int32_t* d = a.ids + (long)step * k;
  const int di = i < k ? d[i] : -1;
  const bool din = i < k && !(di < 0 || di >= a.V);
  const float xd = din ? lg(xr, di, 1) : 0.0f;
  const float ua = i < k ? a.u_acc[(long)step * k + i] : 0.0f;
  const float u = a.u_smp[step];
  // every comparison below is on 16-bit order keys of the bf16 values (the
  // order of the floats, NaN lowest), counted with integer arithmetic: no
  // compare masks, so nothing spills
  // the thread's 64 tile keys (0 for tiles past the row), computed once, and
  // the largest of each group of 8 (one load)
  uint32_t tk[8 * TM_PER], gk[TM_PER];
  uint32_t mk = 0;                                          // the thread's largest tile key
#pragma unroll
  for (int q = 0; q < TM_PER; ++q) {
    const uint32_t w4[4] = {tv[q].x, tv[q].y, tv[q].z, tv[q].w};
    gk[q] = 0;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      uint32_t dj = (uint32_t)(8 * (t + NT * q) + e) - (uint32_t)tiles;       // negative: j < tiles
      asm("" : "+v"(dj));
      tk[8 * q + e] = bf16_key(w4[e >> 1] >> (16 * (e & 1))) & (0u - (dj >> 31));
      gk[q] = max(gk[q], tk[8 * q + e]);
    }
    mk = max(mk, gk[q]);
  }
  // tau: each wave's top_k-th largest thread key (ties by thread), by a bit
  // descent over ballots; top_k threads of that wave hold a tile key >= it, so
  // the row's k-th value is at least the largest of the four
  {
    const uint32_t uk = (mk << 8) | (uint32_t)(255 - t);
    uint32_t x = 0;
    for (int b = 23; b >= 0; --b) {
      const uint32_t y = x | (1u << b);
      x = __popcll(__ballot(uk >= y)) >= K ? y : x;
    }
    if (lane == 0) S.tauw[wave] = x >> 8;
  }
  __syncthreads();
  // key 0 (no tile, or NaN) never counts
  const uint32_t tau = max(max(max(S.tauw[0], S.tauw[1]), max(S.tauw[2], S.tauw[3])), 1u);
  // the tiles that can hold a value >= tau, gathered per wave into its own 64
  // slots of S.tiles by ballots: every branch below is on a wave-wide mask
  // (uniform), and a group of 8 tiles whose largest key is below tau in every
  // lane costs one ballot (usually all of them)
  int wc = 0;                                               // uniform over the wave
  const unsigned long long below = (1ull << lane) - 1ull;
#pragma unroll
  for (int q = 0; q < TM_PER; ++q) {
    if (__ballot(gk[q] >= tau)) {
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const unsigned long long m = __ballot(tk[8 * q + e] >= tau);
        if (m) {
          const int pos = wc + __popcll(m & below);
          if (((m >> lane) & 1ull) && pos < 64) S.tiles[64 * wave + pos] = 8 * (t + NT * q) + e;
          wc += __popcll(m);
        }
      }
    }
  }
  if (lane == 0) S.wcnt[wave] = wc;
  __syncthreads();
  const int wc0 = S.wcnt[0], wc1 = S.wcnt[1], wc2 = S.wcnt[2], wc3 = S.wcnt[3];
  bool fast = max(max(wc0, wc1), max(wc2, wc3)) <= 64;     // block-uniform from here on
  if (fast) {
    // the candidate tiles' logits, lane c of wave w taking the wave's tile c
    uint32_t w8[8];
    int j0 = 0;
    if (lane < S.wcnt[wave]) {
      j0 = 16 * S.tiles[64 * wave + lane];
      const u32x4 l0 = load16(xr + j0), l1 = load16(xr + j0 + 8);
      w8[0] = l0.x; w8[1] = l0.y; w8[2] = l0.z; w8[3] = l0.w;
      w8[4] = l1.x; w8[5] = l1.y; w8[6] = l1.z; w8[7] = l1.w;
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e) w8[e] = 0xffffffffu;         // NaN: key 0
    }
    int ce = 0;
#pragma unroll
    for (int e = 0; e < 16; ++e) ce += key_ge(bf16_key(w8[e >> 1] >> (16 * (e & 1))), tau);
    int ne;
    int o2 = block_excl_scan(ce, S.scan, &ne);
    fast = ne <= TM_CE;
    if (fast) {
      if (ce > 0) {
#pragma unroll
        for (int e = 0; e < 16; ++e) {
          const uint32_t kk = bf16_key(w8[e >> 1] >> (16 * (e & 1)));
          if (kk >= tau) {
            const float xv = e & 1 ? bf16_hi(w8[e >> 1]) : bf16_lo(w8[e >> 1]);
            S.ev[o2] = xv * a.inv_temp;
            S.ej[o2] = j0 + e;
            S.ek[o2] = (kk << 15) | (uint32_t)(0x7fff - o2);   // unique, < 2^31: order of z, then slot
            ++o2;
          }
        }
      }
      if (t < 8 && ne + t < TM_CE) S.ek[ne + t] = 0;          // padding: below every key
      __syncthreads();
      // rank by key: the number of candidates with a larger key (z descending;
      // equal values in slot order, which no later step depends on)
      const int n8 = min((ne + 7) & ~7, TM_CE);
      for (int cc = t; cc < ne; cc += NT) {
        const uint32_t mykey = S.ek[cc];
        int r = 0;
#pragma unroll 2
        for (int q = 0; q < n8; q += 8) {
          const int4 ka = *reinterpret_cast<const int4*>(&S.ek[q]);
          const int4 kb = *reinterpret_cast<const int4*>(&S.ek[q + 4]);
          r += key_gt((uint32_t)ka.x, mykey) + key_gt((uint32_t)ka.y, mykey) + key_gt((uint32_t)ka.z, mykey) +
               key_gt((uint32_t)ka.w, mykey) + key_gt((uint32_t)kb.x, mykey) + key_gt((uint32_t)kb.y, mykey) +
               key_gt((uint32_t)kb.z, mykey) + key_gt((uint32_t)kb.w, mykey);
        }
        S.sv[r] = S.ev[cc];
        S.sj[r] = S.ej[cc];
      }
      __syncthreads();
      if (wave == 0) {
        // filter_wave's arithmetic on the row's k largest values S.sv[0 .. K)
        const float cl = lane < K ? S.sv[lane] : -__builtin_inff();
        const float c0 = rl_f(cl, 0);
        const float el = lane < K ? qx_expf(cl - c0) : 0.0f;
        float Ssum = 0.0f, pre = 0.0f;
        for (int q = 0; q < K; ++q) {
          Ssum = Ssum + rl_f(el, q);
          pre = lane == q ? Ssum : pre;
        }
        float cutoff = rl_f(cl, K - 1);
        if (a.top_p > 0.0f && a.top_p < 1.0f) {
          const float pl = el / Ssum;
          float run = 0.0f, mn = __builtin_inff();
          for (int q = 0; q < K; ++q) {
            const float pq = rl_f(pl, q);
            const float cq = rl_f(cl, q);
            const float incl = run + pq;
            if ((incl - pq) < a.top_p && cq < mn) mn = cq;
            run = incl;
          }
          cutoff = mn;
        }
        int eq = 0;
        for (int r0 = 0; r0 < ne; r0 += 64) {
          const float v = r0 + lane < ne ? S.sv[r0 + lane] : -__builtin_inff();
          eq += __popcll(__ballot(v == cutoff));
        }
        const int n_gt = __popcll(__ballot(lane < K && cl > cutoff));
        const float Sp = (n_gt > 0 ? rl_f(pre, n_gt - 1) : 0.0f) + (float)eq * qx_expf(cutoff - c0);
        int ok = 0;
        if (din) {
          const float zd = xd * a.inv_temp;
          const float ep = zd >= cutoff ? qx_expf(zd - c0) : 0.0f;
          const float eqd = 1.0f, Sq = 1.0f;
          const float lhs = ua * eqd * Sp;
          const float rhs = ep * Sq;
          ok = lhs < rhs ? 1 : 0;
        }
        const int nkeep = n_gt + eq;                        // the kept set: a prefix of the ranking
        if (lane == 0) {
          float* fr = a.frow + (long)row * 4;
          fr[0] = c0;
          fr[1] = Sp;
          fr[2] = cutoff;
          S.ok = ok;
          S.nkeep = nkeep;
        }
        if (nkeep <= 64) {
          WCtx cw;
          cw.mp = c0;
          cw.sp = Sp;
          cw.cutoff = cutoff;
          cw.d = i < k ? di : -1;
          const int je = lane < nkeep ? S.sj[lane] : 0;
          const float ze = lane < nkeep ? S.sv[lane] : -__builtin_inff();
          int tok = -1;
          for (int mode = i < k ? 0 : 1; mode <= 1; ++mode) {
            cw.mode = mode;
            const float w = lane < nkeep ? weight_z(cw, je, ze) : 0.0f;
            const bool pos = w > 0.0f;
            const int npos = __popcll(__ballot(pos));
            if (npos == 0) continue;                        // mode 0 with no residual weight: p_i
            const int key = pos ? walk_key(je) : 0x7fffffff;
            S.wkey[lane] = key;
            wave_lds_sync();
            int r = 0;
#pragma unroll
            for (int q4 = 0; q4 < 16; ++q4) {
              const int4 o = *reinterpret_cast<const int4*>(&S.wkey[4 * q4]);
              r += (int)(o.x < key) + (int)(o.y < key) + (int)(o.z < key) + (int)(o.w < key);
            }
            if (pos) {
              S.skey[r] = key;
              S.sw[r] = w;
            }
            wave_lds_sync();
            const int kv = lane < npos ? S.skey[lane] : 0x7fffffff;
            const float wv = lane < npos ? S.sw[lane] : 0.0f;
            tok = tile_walk(npos, kv, wv, u, S);
            break;
          }
          if (lane == 0) S.tok = tok;
        }
      }
      __syncthreads();
      fast = S.nkeep <= 64;
    }
  }
  // a row the fast path cannot finish (more candidates than it holds, or a
  // kept set over 64) runs the two-kernel path's work in this block
  int ok, tok;
  if (fast) {
    ok = S.ok;
    tok = S.tok;
  } else {
    // the arguments as they lie in the kernel-argument segment: a reference to
    // the parameter itself would make the kernel copy all of it to scratch
    // memory before its first loads
    const SpecArgs* ap =
        (const SpecArgs*)((const char*)__builtin_amdgcn_kernarg_segment_ptr() + TILES_ARGS_OFFSET);
    const int2 r = tiles_full_row(*ap, row);
    ok = r.x;
    tok = r.y;
  }
  if (t == 0) {
    if (a.rows_only) {
      a.rres[2 * row] = ok;
      a.rres[2 * row + 1] = tok;
    } else {
      finish_decide(a, row, ok, tok);
    }
  }
}

// ---------------------------------------------------------------- full-vocabulary scores (Sampler.scores)

// out[row, j] for part p of the row: greedy - the penalised logit; sampling -
// z - c_0 - log(S) on the kept set (z >= cutoff), -inf elsewhere, where
// (c_0, S, cutoff) are the row's filter record, or for an unfiltered row
// c_0 = max z and S = sum exp(z - c_0) combined from the part statistics in the
// accept kernels' order (engine/sampler.py:30-52).
__global__ __launch_bounds__(NT) void spec_scores_kernel(SpecArgs a, float* __restrict__ out) {
  const int p = blockIdx.x, row = blockIdx.y;
  const int t = threadIdx.x;
  const void* src = row_ptr(a, row, 0);
  float c0 = 0.0f, lS = 0.0f, cut = -__builtin_inff();
  if (!a.greedy) {
    if (a.filt) {
      const float* fr = a.frow + (long)row * 4;
      c0 = fr[0];
      lS = logf(fr[1]);
      cut = fr[2];
    } else {
      const float* w = a.ws + (long)row * a.P * 2;
      float m = -__builtin_inff();
      for (int q = 0; q < a.P; ++q) m = fmaxf(m, w[2 * q]);
      float S = 0.0f;
      for (int q = 0; q < a.P; ++q) S = S + w[2 * q + 1] * qx_expf(w[2 * q] - m);
      c0 = m;
      lS = logf(S);
    }
  }
  const int base = p * PART, end = min(a.V, base + PART);
  float* o = out + (long)row * a.V;
  for (int j = base + t; j < end; j += NT) {
    const float x = pen_x(a.seen, a.pen, lg(src, j, a.bf), j, nullptr, 0);
    if (a.greedy) {
      o[j] = x;
    } else {
      const float z = x * a.inv_temp;
      o[j] = z >= cut ? (z - c0) - lS : -__builtin_inff();
    }
  }
}

int nparts(int V) { return (V + PART - 1) / PART; }

}  // namespace

uint64_t ws_floats(int S, int rps, int P) {
  return (uint64_t)S * rps * P * 2 + (uint64_t)S * P * NT + (uint64_t)S * P + (uint64_t)S * 8;
}

// list-form part lists (1 <= top_k <= 64) and the per-row (c_0, S_p, cutoff),
// which every filtered call needs (the wide form keeps no lists)
uint64_t filter_floats(int S, int k, int P, int top_k) {
  const uint64_t lists = (top_k >= 1 && top_k <= 64) ? (uint64_t)S * (k + 1) * P * (top_k + 1) : 0;
  return lists + (uint64_t)S * (k + 1) * 4;
}

// list form without draft logits: per target row and part CAND_CAP candidate
// indices and their count, then one finished-filter counter per step and each
// row's (accept flag, draw)
bool cand_fits(int P) { return P * CAND_CAP <= NT * CAND_IT; }
uint64_t cand_ints(int S, int k, int P, int top_k, int has_draft) {
  return (top_k >= 1 && top_k <= 64 && !has_draft && cand_fits(P))
             ? (uint64_t)S * (k + 1) * P * (2 * CAND_CAP + 2) + S + (uint64_t)S * (k + 1) * 2
             : 0;
}

extern "C" uint64_t qvex_spec_accept_filtered_workspace_bytes(int S, int k, int V, int has_draft, int top_k) {
  if (S < 1 || k < 0 || V < 1 || top_k < 0) return 0;
  const int rps = (k + 1) + (has_draft ? k : 0);
  const int P = nparts(V);
  const int tk = top_k < V ? top_k : 0;
  return (ws_floats(S, rps, P) + filter_floats(S, k, P, top_k) + cand_ints(S, k, P, tk, has_draft)) * sizeof(float);
}

extern "C" uint64_t qvex_spec_accept_workspace_bytes(int S, int k, int V, int has_draft) {
  return qvex_spec_accept_filtered_workspace_bytes(S, k, V, has_draft, 0);
}

static int spec_accept_impl(const void* target, const void* draft, int bf, const int32_t* draft_ids,
                            const float* u_accept, const float* u_sample, float inv_temp, const float* seen,
                            float presence_penalty, int top_k, float top_p, int32_t* n_accept, int32_t* out_token,
                            int S, int k, int V, void* workspace, uint64_t workspace_bytes, void* stream) {
  QVEX_CHECK_ARG(S >= 1 && k >= 0 && k <= 32, "qvex_spec_accept: S=%d k=%d (need S >= 1, 0 <= k <= 32)", S, k);
  QVEX_CHECK_ARG(V >= 4 && V % 4 == 0, "qvex_spec_accept: V=%d must be a positive multiple of 4", V);
  QVEX_CHECK_ARG(target && n_accept && out_token && workspace, "qvex_spec_accept: null pointer");
  QVEX_CHECK_ARG(k == 0 || (draft_ids && u_accept), "qvex_spec_accept: draft_ids/u_accept required for k > 0");
  QVEX_CHECK_ARG(qvex_aligned(target, 16) && (!draft || qvex_aligned(draft, 16)),
                 "qvex_spec_accept: logits must be 16-byte aligned");
  const int greedy = !(inv_temp > 0.0f);
  QVEX_CHECK_ARG(greedy || u_sample, "qvex_spec_accept: u_sample required when sampling");
  QVEX_CHECK_ARG(top_k >= 0, "qvex_spec_accept: top_k=%d must be >= 0", top_k);
  QVEX_CHECK_ARG(presence_penalty == presence_penalty, "qvex_spec_accept: presence_penalty is NaN");
  QVEX_CHECK_ARG(top_p == top_p, "qvex_spec_accept: top_p is NaN");
  const bool use_p = top_p > 0.0f && top_p < 1.0f;
  const int P = nparts(V);
  // engine/sampler.py:44-47: top-k only when 0 < top_k < V; greedy scores are not filtered
  const int tk = (top_k > 0 && top_k < V) ? top_k : 0;
  const int filt = greedy ? 0 : (tk >= 1 && tk <= 64 ? 1 : ((tk > 64 || use_p) ? 2 : 0));
  const int kf = filt == 1 ? tk : 0;           // list-form top-k
  QVEX_CHECK_ARG(kf == 0 || P * kf <= 64 * 64, "qvex_spec_accept: V=%d too large for top_k=%d", V, kf);
  const int rps = (k + 1) + (draft ? k : 0);
  const bool fast = filt == 1 && !draft && cand_fits(P);
  const uint64_t base = ws_floats(S, rps, P);
  const uint64_t need =
      (base + (filt ? filter_floats(S, k, P, kf) : 0) + (fast ? cand_ints(S, k, P, kf, 0) : 0)) * sizeof(float);
  QVEX_CHECK_ARG(workspace_bytes >= need, "qvex_spec_accept: workspace %llu bytes < %llu needed",
                 (unsigned long long)workspace_bytes, (unsigned long long)need);
  const size_t lds = ((size_t)P * NT + P + 2 * rps) * sizeof(float);
  QVEX_CHECK_ARG(lds <= 150 * 1024, "qvex_spec_accept: V=%d too large for the LDS sampling table", V);
  QVEX_CHECK_ARG((long)S * rps <= 65535, "qvex_spec_accept: S*rows=%ld exceeds the grid limit", (long)S * rps);
  QVEX_CHECK_ARG(rps <= 80, "qvex_spec_accept: k=%d too large", k);
  float* fws = (float*)workspace + base;
  float* frow = fws + (kf > 0 ? (uint64_t)S * (k + 1) * P * (kf + 1) : 0);
  int32_t* cand = reinterpret_cast<int32_t*>(frow + (uint64_t)S * (k + 1) * 4);
  float* cand_z = reinterpret_cast<float*>(cand + (uint64_t)S * (k + 1) * P * CAND_CAP);
  int32_t* ncand = reinterpret_cast<int32_t*>(cand_z + (uint64_t)S * (k + 1) * P * CAND_CAP);
  int32_t* ctr = ncand + (uint64_t)S * (k + 1) * P * 2;
  int32_t* rres = ctr + S;
  SpecArgs a{target, draft, draft_ids, u_accept, u_sample, inv_temp, greedy, n_accept, out_token,
             (float*)workspace, S, k, V, P, rps, seen, presence_penalty, kf, use_p ? top_p : 1.0f, fws, frow, bf,
             filt, filt == 2 ? tk : 0, fast ? 1 : 0, fast ? cand : nullptr, fast ? cand_z : nullptr,
             fast ? ncand : nullptr, fast ? ctr : nullptr, fast ? rres : nullptr};
  hipStream_t st = (hipStream_t)stream;
  if (a.bf)
    hipLaunchKernelGGL(spec_rowstats_kernel<true>, dim3(P, S * rps), dim3(NT), 0, st, a);
  else
    hipLaunchKernelGGL(spec_rowstats_kernel<false>, dim3(P, S * rps), dim3(NT), 0, st, a);
  QVEX_CHECK_LAUNCH("qvex_spec_accept/rowstats");
  if (fast) {
    hipLaunchKernelGGL(spec_finish_kernel, dim3(S * (k + 1)), dim3(NT), lds, st, a);
    QVEX_CHECK_LAUNCH("qvex_spec_accept/finish");
    return QVEX_OK;
  }
  if (filt == 1) {
    hipLaunchKernelGGL(spec_filter_kernel, dim3(S * (k + 1)), dim3(NT), 0, st, a);
    QVEX_CHECK_LAUNCH("qvex_spec_accept/filter");
  } else if (filt == 2) {
    hipLaunchKernelGGL(spec_wide_filter_kernel, dim3(S * (k + 1)), dim3(WT), 0, st, a);
    QVEX_CHECK_LAUNCH("qvex_spec_accept/wide_filter");
  }
  hipLaunchKernelGGL(spec_decide_kernel, dim3(P, S), dim3(NT), 0, st, a);
  QVEX_CHECK_LAUNCH("qvex_spec_accept/decide");
  if (!greedy) {
    hipLaunchKernelGGL(spec_sample_kernel, dim3(S), dim3(NT), lds, st, a);
    QVEX_CHECK_LAUNCH("qvex_spec_accept/sample");
  }
  return QVEX_OK;
}

extern "C" int qvex_spec_accept_filtered(const float* target, const float* draft, const int32_t* draft_ids,
                                         const float* u_accept, const float* u_sample, float inv_temp,
                                         const float* seen, float presence_penalty, int top_k, float top_p,
                                         int32_t* n_accept, int32_t* out_token, int S, int k, int V,
                                         void* workspace, uint64_t workspace_bytes, void* stream) {
  return spec_accept_impl(target, draft, 0, draft_ids, u_accept, u_sample, inv_temp, seen, presence_penalty, top_k,
                          top_p, n_accept, out_token, S, k, V, workspace, workspace_bytes, stream);
}

extern "C" int qvex_spec_accept_filtered_bf16(const uint16_t* target, const uint16_t* draft,
                                              const int32_t* draft_ids, const float* u_accept,
                                              const float* u_sample, float inv_temp, const float* seen,
                                              float presence_penalty, int top_k, float top_p, int32_t* n_accept,
                                              int32_t* out_token, int S, int k, int V, void* workspace,
                                              uint64_t workspace_bytes, void* stream) {
  return spec_accept_impl(target, draft, 1, draft_ids, u_accept, u_sample, inv_temp, seen, presence_penalty, top_k,
                          top_p, n_accept, out_token, S, k, V, workspace, workspace_bytes, stream);
}


// Whether the one-kernel list form runs for a call with these arguments (tile
// maxima given): bf16 logits without draft logits, sampling with 1 <= top_k <= 64
// and no presence penalty, V a multiple of 128 whose tiles and parts fit.
static bool tiles_form_applies(int S, int k, int V, float inv_temp, int top_k, float presence_penalty) {
  const int tk = (top_k > 0 && top_k < V) ? top_k : 0;
  return inv_temp > 0.0f && tk >= 1 && tk <= 64 && presence_penalty == 0.0f && V % 128 == 0 && V >= 128 &&
         V / 16 <= NT * 8 * TM_PER && cand_fits(nparts(V)) && S >= 1 && k >= 0 && k <= 32 &&
         (long)S * (k + 1) <= 65535;
}

extern "C" int qvex_spec_accept_tiles_applies(int S, int k, int V, float inv_temp, int top_k,
                                              float presence_penalty) {
  return tiles_form_applies(S, k, V, inv_temp, top_k, presence_penalty) ? 1 : 0;
}

// The one-kernel list form. rows == nullptr: the last row of each step decides
// (n_accept, out_token); otherwise each row leaves its (accept flag, draw) in
// rows [S * (k+1)][2] and nothing decides.
static int spec_tiles_launch(const uint16_t* target, const uint16_t* tile_max, const int32_t* draft_ids,
                             const float* u_accept, const float* u_sample, float inv_temp, const float* seen,
                             int top_k, float top_p, int32_t* n_accept, int32_t* out_token, int32_t* rows, int S,
                             int k, int V, void* workspace, uint64_t workspace_bytes, void* stream) {
  const int tk = (top_k > 0 && top_k < V) ? top_k : 0;
  const int P = nparts(V);
  const int tiles = V / 16;
  QVEX_CHECK_ARG(target && workspace && u_sample && (rows || (n_accept && out_token)),
                 "qvex_spec_accept_tiles: null pointer");
  QVEX_CHECK_ARG(k == 0 || (draft_ids && u_accept), "qvex_spec_accept_tiles: draft_ids/u_accept required for k > 0");
  QVEX_CHECK_ARG(qvex_aligned(target, 16) && qvex_aligned(tile_max, 16),
                 "qvex_spec_accept_tiles: logits and tile maxima must be 16-byte aligned");
  QVEX_CHECK_ARG(top_p == top_p, "qvex_spec_accept_tiles: top_p is NaN");
  const bool use_p = top_p > 0.0f && top_p < 1.0f;
  const int rps = k + 1;
  const uint64_t base = ws_floats(S, rps, P);
  const uint64_t need = (base + filter_floats(S, k, P, tk) + cand_ints(S, k, P, tk, 0)) * sizeof(float);
  QVEX_CHECK_ARG(workspace_bytes >= need, "qvex_spec_accept_tiles: workspace %llu bytes < %llu needed",
                 (unsigned long long)workspace_bytes, (unsigned long long)need);
  const size_t lds = ((size_t)P * NT + P + 2 * rps) * sizeof(float);
  float* fws = (float*)workspace + base;
  float* frow = fws + (uint64_t)S * (k + 1) * P * (tk + 1);
  int32_t* cand = reinterpret_cast<int32_t*>(frow + (uint64_t)S * (k + 1) * 4);
  float* cand_z = reinterpret_cast<float*>(cand + (uint64_t)S * (k + 1) * P * CAND_CAP);
  int32_t* ncand = reinterpret_cast<int32_t*>(cand_z + (uint64_t)S * (k + 1) * P * CAND_CAP);
  int32_t* ctr = ncand + (uint64_t)S * (k + 1) * P * 2;
  int32_t* rres = rows ? rows : ctr + S;
  SpecArgs a{target, nullptr, draft_ids, u_accept, u_sample, inv_temp, 0, n_accept, out_token,
             (float*)workspace, S, k, V, P, rps, seen, 0.0f, tk, use_p ? top_p : 1.0f, fws, frow, 1,
             1, 0, 1, cand, cand_z, ncand, ctr, rres, rows ? 1 : 0};
  hipLaunchKernelGGL(spec_tiles_kernel, dim3(S * rps), dim3(NT), lds, (hipStream_t)stream, tile_max, tiles, a);
  QVEX_CHECK_LAUNCH("qvex_spec_accept_tiles");
  return QVEX_OK;
}

extern "C" int qvex_spec_accept_tiles_bf16(const uint16_t* target, const uint16_t* tile_max, const int32_t* draft_ids,
                                           const float* u_accept, const float* u_sample, float inv_temp,
                                           const float* seen, float presence_penalty, int top_k, float top_p,
                                           int32_t* n_accept, int32_t* out_token, int S, int k, int V,
                                           void* workspace, uint64_t workspace_bytes, void* stream) {
  if (!tile_max || !tiles_form_applies(S, k, V, inv_temp, top_k, presence_penalty))
    return spec_accept_impl(target, nullptr, 1, draft_ids, u_accept, u_sample, inv_temp, seen, presence_penalty,
                            top_k, top_p, n_accept, out_token, S, k, V, workspace, workspace_bytes, stream);
  return spec_tiles_launch(target, tile_max, draft_ids, u_accept, u_sample, inv_temp, seen, top_k, top_p, n_accept,
                           out_token, nullptr, S, k, V, workspace, workspace_bytes, stream);
}

extern "C" int qvex_spec_accept_tiles_rows_bf16(const uint16_t* target, const uint16_t* tile_max,
                                                const int32_t* draft_ids, const float* u_accept,
                                                const float* u_sample, float inv_temp, const float* seen,
                                                float presence_penalty, int top_k, float top_p, int32_t* rows, int S,
                                                int k, int V, void* workspace, uint64_t workspace_bytes,
                                                void* stream) {
  QVEX_CHECK_ARG(tile_max && rows, "qvex_spec_accept_tiles_rows: tile_max and rows are required");
  QVEX_CHECK_ARG(tiles_form_applies(S, k, V, inv_temp, top_k, presence_penalty),
                 "qvex_spec_accept_tiles_rows: the one-kernel form does not apply to this call (see "
                 "qvex_spec_accept_tiles_applies)");
  return spec_tiles_launch(target, tile_max, draft_ids, u_accept, u_sample, inv_temp, seen, top_k, top_p, nullptr,
                           nullptr, rows, S, k, V, workspace, workspace_bytes, stream);
}

// tile_max[r][t] = the largest of x[r][16 t .. 16 t + 15] (bf16; -inf for no value)
__global__ void tile_max_kernel(const uint16_t* __restrict__ x, int rows, int V, uint16_t* __restrict__ out) {
  const int tiles = (V + 15) / 16;
  const long g = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (g >= (long)rows * tiles) return;
  const int r = (int)(g / tiles), tt = (int)(g - (long)r * tiles);
  const uint16_t* xr = x + (long)r * V + 16 * tt;
  float m = -__builtin_inff();
  for (int e = 0; e < 16 && 16 * tt + e < V; ++e) m = fmaxf(m, bf16_to_f32(xr[e]));
  out[g] = f32_to_bf16(m);
}

extern "C" int qvex_tile_max_bf16(const uint16_t* x, int rows, int V, uint16_t* out, void* stream) {
  QVEX_CHECK_ARG(x && out && rows >= 1 && V >= 1, "qvex_tile_max_bf16: bad arguments (rows=%d V=%d)", rows, V);
  const long n = (long)rows * ((V + 15) / 16);
  hipLaunchKernelGGL(tile_max_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, (hipStream_t)stream, x, rows,
                     V, out);
  QVEX_CHECK_LAUNCH("qvex_tile_max_bf16");
  return QVEX_OK;
}

extern "C" uint64_t qvex_sampler_scores_workspace_bytes(int R, int V, int top_k) {
  return qvex_spec_accept_filtered_workspace_bytes(R, 0, V, 0, top_k);
}

extern "C" int qvex_sampler_scores(const void* logits, int logits_bf16, int R, int V, const float* seen,
                                   float presence_penalty, float inv_temp, int top_k, float top_p, float* out,
                                   void* workspace, uint64_t workspace_bytes, void* stream) {
  QVEX_CHECK_ARG(logits && out && workspace, "qvex_sampler_scores: null pointer");
  QVEX_CHECK_ARG(R >= 1 && R <= 65535 && V >= 4 && V % 4 == 0 && top_k >= 0,
                 "qvex_sampler_scores: R=%d V=%d top_k=%d (V a positive multiple of 4)", R, V, top_k);
  QVEX_CHECK_ARG(qvex_aligned(logits, 16), "qvex_sampler_scores: logits must be 16-byte aligned");
  QVEX_CHECK_ARG(presence_penalty == presence_penalty && top_p == top_p, "qvex_sampler_scores: NaN argument");
  const int greedy = !(inv_temp > 0.0f);
  const bool use_p = top_p > 0.0f && top_p < 1.0f;
  const int P = nparts(V);
  const int tk = (top_k > 0 && top_k < V) ? top_k : 0;
  const int filt = greedy ? 0 : (tk >= 1 && tk <= 64 ? 1 : ((tk > 64 || use_p) ? 2 : 0));
  const int kf = filt == 1 ? tk : 0;
  QVEX_CHECK_ARG(kf == 0 || P * kf <= 64 * 64, "qvex_sampler_scores: V=%d too large for top_k=%d", V, kf);
  const uint64_t base = ws_floats(R, 1, P);
  const uint64_t need = (base + (filt ? filter_floats(R, 0, P, kf) : 0)) * sizeof(float);
  QVEX_CHECK_ARG(workspace_bytes >= need, "qvex_sampler_scores: workspace %llu bytes < %llu needed",
                 (unsigned long long)workspace_bytes, (unsigned long long)need);
  float* fws = (float*)workspace + base;
  float* frow = fws + (kf > 0 ? (uint64_t)R * P * (kf + 1) : 0);
  SpecArgs a{logits, nullptr, nullptr, nullptr, nullptr, inv_temp, greedy, nullptr, nullptr, (float*)workspace,
             R, 0, V, P, 1, seen, presence_penalty, kf, use_p ? top_p : 1.0f, fws, frow, logits_bf16 ? 1 : 0,
             filt, filt == 2 ? tk : 0};
  hipStream_t st = (hipStream_t)stream;
  if (!greedy) {
    if (a.bf)
      hipLaunchKernelGGL(spec_rowstats_kernel<true>, dim3(P, R), dim3(NT), 0, st, a);
    else
      hipLaunchKernelGGL(spec_rowstats_kernel<false>, dim3(P, R), dim3(NT), 0, st, a);
    QVEX_CHECK_LAUNCH("qvex_sampler_scores/rowstats");
    if (filt == 1) {
      hipLaunchKernelGGL(spec_filter_kernel, dim3(R), dim3(NT), 0, st, a);
      QVEX_CHECK_LAUNCH("qvex_sampler_scores/filter");
    } else if (filt == 2) {
      hipLaunchKernelGGL(spec_wide_filter_kernel, dim3(R), dim3(WT), 0, st, a);
      QVEX_CHECK_LAUNCH("qvex_sampler_scores/wide_filter");
    }
  }
  hipLaunchKernelGGL(spec_scores_kernel, dim3(P, R), dim3(NT), 0, st, a, out);
  QVEX_CHECK_LAUNCH("qvex_sampler_scores/scores");
  return QVEX_OK;
}

extern "C" int qvex_spec_accept(const float* target, const float* draft, const int32_t* draft_ids,
                                const float* u_accept, const float* u_sample, float inv_temp,
                                int32_t* n_accept, int32_t* out_token, int S, int k, int V,
                                void* workspace, uint64_t workspace_bytes, void* stream) {
  return qvex_spec_accept_filtered(target, draft, draft_ids, u_accept, u_sample, inv_temp, nullptr, 0.0f, 0, 1.0f,
                                   n_accept, out_token, S, k, V, workspace, workspace_bytes, stream);
}

// Device address of `scratch` on the current device, looked up on the first
// call there (hipGetSymbolAddress with that device current); nullptr on error.
static void* scratch_ptr(int* err_dev) {
  static std::mutex mu;
  static void* ptrs[64] = {nullptr};
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) {
    *err_dev = dev;
    return nullptr;
  }
  std::lock_guard<std::mutex> lock(mu);
  if (!ptrs[dev]) {
    void* p = nullptr;
    if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) != hipSuccess || !p) {
      *err_dev = dev;
      return nullptr;
    }
    ptrs[dev] = p;
  }
  return ptrs[dev];
}

extern "C" int qvex_spec_accept_filtered_bf16_noalloc(const uint16_t* target, const uint16_t* draft,
                                                      const int32_t* draft_ids, const float* u_accept,
                                                      const float* u_sample, float inv_temp, const float* seen,
                                                      float presence_penalty, int top_k, float top_p,
                                                      int32_t* n_accept, int32_t* out_token, int S, int k, int V,
                                                      void* stream) {
  QVEX_CHECK_ARG(S >= 1 && k >= 0 && V >= 1 && top_k >= 0, "qvex_spec_accept_noalloc: S=%d k=%d V=%d top_k=%d", S, k,
                 V, top_k);
  const uint64_t need = qvex_spec_accept_filtered_workspace_bytes(S, k, V, draft != nullptr, top_k);
  QVEX_CHECK_ARG(need <= QVEX_SPEC_SCRATCH_BYTES,
                 "qvex_spec_accept_noalloc: S=%d k=%d V=%d top_k=%d need %llu workspace bytes, more than the %u-byte "
                 "static scratch; use qvex_spec_accept_filtered_bf16 with a workspace",
                 S, k, V, top_k, (unsigned long long)need, (unsigned)QVEX_SPEC_SCRATCH_BYTES);
  int dev = -1;
  void* ws = scratch_ptr(&dev);
  if (!ws) return qvex::fail(QVEX_EHIP, "qvex_spec_accept_noalloc: no scratch address on device %d", dev);
  return spec_accept_impl(target, draft, 1, draft_ids, u_accept, u_sample, inv_temp, seen, presence_penalty, top_k,
                          top_p, n_accept, out_token, S, k, V, ws, QVEX_SPEC_SCRATCH_BYTES, stream);
}
