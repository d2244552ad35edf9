// Gated DeltaNet recurrence (verify form) with a state snapshot per token.
//
// Reference: engine/kernels.py:11-116 (gated_delta, keep_mid). Per value head hv
// and value row dv, for each token t:
//   g = exp(-exp(A_log) * softplus(a + dt_bias)),  beta = sigmoid(b)
//   S *= g;  kv = S.k;  delta = (v - kv) * beta;  S += k * delta;  y = S.q
// with GQA key head hk = hv / (Hv / Hk). The reference keeps only the state
// before the last token (k = 1 rollback); here the state after every token is
// written, so rolling back to any accepted length is a choice of slot.
//
// MI355X mapping: one 16-lane DPP row owns one 128-float state row (8 fp32 per
// lane, two 16-byte loads); a wave holds 4 rows, a block 16 rows of one head.
// The row's dot products reduce inside the 16-lane row with quad_perm/row_ror
// DPP (no LDS). All T tokens' q/k/v/gates are prefetched before the sequential
// loop. The state never leaves registers between tokens; each snapshot is two
// 16-byte stores per lane.
#include "qvex_common.h"

namespace {

constexpr int DK = 128;
constexpr int ROWS_PER_BLOCK = 16;
constexpr int TMAX_PREFETCH = 8;

struct GdnArgs {
  const uint16_t* q;
  const uint16_t* k;
  const uint16_t* v;
  const uint16_t* a;
  const uint16_t* b;
  const float* A_log;
  const uint16_t* dt_bias;
  const float* s_in;     // state source (slot base when slot_ptr != nullptr)
  float* s_out;          // snapshot destination base
  const int* slot_ptr;   // device-side current slot (ring mode) or nullptr
  long slot_stride;      // floats per state slot = B*Hv*Dv*Dk
  int n_slots;           // ring slots (ring mode)
  int snap_every;        // plain mode: 1 = slot t gets the state after token t, 0 = final only
  uint16_t* y;
  int B, T, Hk, Hv, Dv;
};

__global__ __launch_bounds__(256) void gdn_recurrent_kernel(GdnArgs p) {
  const int rows_per_head = p.Dv / ROWS_PER_BLOCK;
  const int n = blockIdx.x / rows_per_head;            // b * Hv + hv
  const int bi = n / p.Hv, hv = n % p.Hv;
  const int hk = hv / (p.Hv / p.Hk);
  const int grp = threadIdx.x >> 4, l16 = threadIdx.x & 15;
  const int dv = (blockIdx.x % rows_per_head) * ROWS_PER_BLOCK + grp;
  const int T = p.T;

  int cur = 0;
  const float* s_in = p.s_in;
  if (p.slot_ptr) {
    cur = *p.slot_ptr;
    cur = ((cur % p.n_slots) + p.n_slots) % p.n_slots;   // never index outside the ring
    s_in += (long)cur * p.slot_stride;
  }
  const long row_off = ((long)n * p.Dv + dv) * DK + l16 * 8;

  float st[8];
  {
    const u32x4 s0 = load16(s_in + row_off);
    const u32x4 s1 = load16(s_in + row_off + 4);
    st[0] = __uint_as_float(s0.x); st[1] = __uint_as_float(s0.y);
    st[2] = __uint_as_float(s0.z); st[3] = __uint_as_float(s0.w);
    st[4] = __uint_as_float(s1.x); st[5] = __uint_as_float(s1.y);
    st[6] = __uint_as_float(s1.z); st[7] = __uint_as_float(s1.w);
  }
  // the gate inputs as raw values, converted after the first block's token
  // loads are out (converting here would wait for them first)
  float a_log = p.A_log[hv];
  uint32_t dt_raw = p.dt_bias[hv];
  // one block of up to TMAX_PREFETCH tokens; the first is peeled out of the
  // loop so that its loads are not held behind a loop-carried wait
  auto block = [&](const int t0) {
    const int tn = min(TMAX_PREFETCH, T - t0);
    // every token's inputs requested at once, as raw words (tokens past tn
    // re-read token t0 + tn - 1, never used): converting inside a per-token
    // branch would wait for each token's loads before issuing the next's
    u32x4 kr[TMAX_PREFETCH], qr[TMAX_PREFETCH];
    uint16_t vr[TMAX_PREFETCH];
#pragma unroll
    for (int j = 0; j < TMAX_PREFETCH; ++j) {
      const int t = t0 + min(j, tn - 1);
      const long qk = (((long)bi * T + t) * p.Hk + hk) * DK + l16 * 8;
      kr[j] = load16(p.k + qk);
      qr[j] = load16(p.q + qk);
      vr[j] = p.v[(((long)bi * T + t) * p.Hv + hv) * p.Dv + dv];
    }
    // the decay and beta of token t0 + l in lane l, all tokens at once (the
    // same value in every row of the head), each token's read back with a
    // readlane in the chain: one gate latency per block instead of one per token
    const int tl = t0 + min(threadIdx.x & 63, tn - 1);
    uint32_t a_raw = p.a[((long)bi * T + tl) * p.Hv + hv];
    uint32_t b_raw = p.b[((long)bi * T + tl) * p.Hv + hv];
    asm volatile("" : "+v"(a_log), "+v"(dt_raw));
    const float A = expf(a_log);
    const float dt = bf16_to_f32((uint16_t)dt_raw);
    const float xl = bf16_to_f32((uint16_t)a_raw) + dt;
    const float spl = xl > 20.0f ? xl : log1pf(expf(xl));
    const float g_l = expf(-A * spl);
    const float beta_l = 1.0f / (1.0f + expf(-bf16_to_f32((uint16_t)b_raw)));
#pragma unroll
    for (int j = 0; j < TMAX_PREFETCH; ++j) {
      if (j < tn) {
        const int t = t0 + j;
        float kk[8], qq[8];
        const uint32_t kw[4] = {kr[j].x, kr[j].y, kr[j].z, kr[j].w};
        const uint32_t qw[4] = {qr[j].x, qr[j].y, qr[j].z, qr[j].w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          kk[2 * i] = bf16_lo(kw[i]);
          kk[2 * i + 1] = bf16_hi(kw[i]);
          qq[2 * i] = bf16_lo(qw[i]);
          qq[2 * i + 1] = bf16_hi(qw[i]);
        }
        const float g = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(g_l), j));
        const float beta = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(beta_l), j));
        float kv = 0.0f;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          st[i] *= g;
          kv = fmaf(st[i], kk[i], kv);
        }
        kv = row16_allsum(kv);
        const float delta = (bf16_to_f32(vr[j]) - kv) * beta;
        float o = 0.0f;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          st[i] = fmaf(kk[i], delta, st[i]);
          o = fmaf(st[i], qq[i], o);
        }
        o = row16_allsum(o);
        if (l16 == 0) p.y[(((long)bi * T + t) * p.Hv + hv) * p.Dv + dv] = f32_to_bf16(o);

        long slot = -1;
        if (p.slot_ptr) {
          if (p.snap_every || t == T - 1) slot = (cur + 1 + t) % p.n_slots;
        } else if (p.snap_every) {
          slot = t;
        } else if (t == T - 1) {
          slot = 0;
        }
        if (slot >= 0) {
          float* dst = p.s_out + slot * p.slot_stride + row_off;
          u32x4 o0, o1;
          o0.x = __float_as_uint(st[0]); o0.y = __float_as_uint(st[1]);
          o0.z = __float_as_uint(st[2]); o0.w = __float_as_uint(st[3]);
          o1.x = __float_as_uint(st[4]); o1.y = __float_as_uint(st[5]);
          o1.z = __float_as_uint(st[6]); o1.w = __float_as_uint(st[7]);
          // nontemporal: the snapshots are read back by a later call at most
          // once, and dirty lines left in L2 slow the next kernels' reads
          __builtin_nontemporal_store(o0, reinterpret_cast<u32x4*>(dst));
          __builtin_nontemporal_store(o1, reinterpret_cast<u32x4*>(dst + 4));
        }
      }
    }
  };
  block(0);
  for (int t0 = TMAX_PREFETCH; t0 < T; t0 += TMAX_PREFETCH) block(t0);
}

// ---------------------------------------------------------------- fused decode layer
//
// One block of 1024 threads per value head runs the whole GDN mixer between
// the input and output projections for T <= 8 tokens (engine/model.py:235-291):
//   1. depthwise conv over the ring window + silu for the head's 128 q, 128 k
//      and 128 v channels, q/k weightless RMSNorm and scales, and the new
//      projection rows stored into the conv ring (each channel by one block);
//   2. the recurrence with a snapshot per token (as gdn_recurrent_kernel);
//   3. the gated RMSNorm of the head's output rows.
// Every step keeps the arithmetic and reduction order of conv_silu_qk_kernel,
// gdn_recurrent_kernel and gated_rmsnorm_kernel (one wave per 128-channel head
// with 2 channels per lane; one 16-lane DPP row per state row, here two rows
// per 16 lanes), so the outputs, the conv ring and the state ring are
// bitwise those of the three-kernel path.
constexpr int FUSED_TMAX = 8;
constexpr int FUSED_THREADS = 1024;
constexpr int FUSED_KC = 4;   // conv taps (Qwen3.5: linear_conv_kernel_dim = 4)

// (base + d) mod m for 0 <= base < m and -m <= d < m: a 64-bit modulo is a long
// instruction sequence, so the token count is reduced once per kernel (the ring
// offsets -3 .. T-1 lie within that range since ring_rows >= T + 3)
__device__ __forceinline__ int wrap_add(int base, int d, int m) {
  int r = base + d;
  r = r < 0 ? r + m : r;
  return r >= m ? r - m : r;
}

struct GdnFusedArgs {
  const uint16_t* proj;    // [T, p_stride]: conv channels | z | b | a
  long p_stride;
  uint16_t* ring;          // [R, C] conv input history
  int R;
  const int32_t* counter;  // the layer's token count (conv ring row and state slot)
  const uint16_t* cw;      // [C, FUSED_KC]
  int C, key_dim;
  float q_scale, k_scale, qk_eps;
  const float* A_log;
  const uint16_t* dt_bias;
  int z_off, ab_off;
  float* state;            // [n_slots, Hv, 128, 128]
  int n_slots, snap_every;
  const uint16_t* norm_w;  // [128]
  float norm_eps;
  uint16_t* out;           // [T, Hv * 128]
  int T, Hk, Hv;
};

__global__ __launch_bounds__(FUSED_THREADS) void gdn_decode_fused_kernel(GdnFusedArgs p) {
  __shared__ float qs[FUSED_TMAX][DK], ks[FUSED_TMAX][DK], vs[FUSED_TMAX][DK], ys[FUSED_TMAX][DK];
  const int hv = blockIdx.x;
  const int hk = hv / (p.Hv / p.Hk);
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int grp = threadIdx.x >> 4, l16 = threadIdx.x & 15;
  const int T = p.T;
  const long p0 = *p.counter;
  const int cur = (int)(((p0 % p.n_slots) + p.n_slots) % p.n_slots);
  const int rbase = (int)(((p0 % p.R) + p.R) % p.R);
  const long slot_stride = (long)p.Hv * DK * DK;

  // state rows grp and grp + 64 of this head, 8 columns per lane
  long row_off[2];
  float st[2][8];
#pragma unroll
  for (int r = 0; r < 2; ++r) {
    row_off[r] = ((long)hv * DK + grp + 64 * r) * DK + l16 * 8;
    const float* src = p.state + cur * slot_stride + row_off[r];
    const u32x4 s0 = load16(src);
    const u32x4 s1 = load16(src + 4);
    st[r][0] = __uint_as_float(s0.x); st[r][1] = __uint_as_float(s0.y);
    st[r][2] = __uint_as_float(s0.z); st[r][3] = __uint_as_float(s0.w);
    st[r][4] = __uint_as_float(s1.x); st[r][5] = __uint_as_float(s1.y);
    st[r][6] = __uint_as_float(s1.z); st[r][7] = __uint_as_float(s1.w);
  }

  // the gate inputs b, a of every token, and this wave's token of z and the
  // norm weight for step 3, all requested before any of them is needed
  // per-token decay g and write strength beta, once per block
  __shared__ float gb_s[2][FUSED_TMAX];
  if (threadIdx.x < T) {
    const int t = threadIdx.x;
    const float A = expf(p.A_log[hv]);
    const float dt = bf16_to_f32(p.dt_bias[hv]);
    const float aa = bf16_to_f32(p.proj[(size_t)t * p.p_stride + p.ab_off + p.Hv + hv]);
    const float bb = bf16_to_f32(p.proj[(size_t)t * p.p_stride + p.ab_off + hv]);
    const float x = aa + dt;
    const float sp = x > 20.0f ? x : log1pf(expf(x));
    gb_s[0][t] = expf(-A * sp);
    gb_s[1][t] = 1.0f / (1.0f + expf(-bb));
  }
  uint32_t zp = 0, wp = 0;
  if (wave < T) {
    zp = *reinterpret_cast<const uint32_t*>(p.proj + (size_t)wave * p.p_stride + p.z_off + hv * DK + 2 * lane);
    wp = *reinterpret_cast<const uint32_t*>(p.norm_w + 2 * lane);
  }

  // 1. conv + silu (+ q/k norm): one wave per (token, q | k | v head); the
  // KC = 4 window rows and the lane's two channels' taps (16 bytes) load at once
  constexpr int W = FUSED_KC - 1;
  const bool ring_qk = hv % (p.Hv / p.Hk) == 0;
  for (int task = wave; task < 3 * T; task += FUSED_THREADS / 64) {
    const int t = task / 3, part = task - 3 * (task / 3);
    const int cb = part == 0 ? hk * DK : part == 1 ? p.key_dim + hk * DK : 2 * p.key_dim + hv * DK;
    const int c0 = cb + 2 * lane;
    uint32_t win[FUSED_KC];
#pragma unroll
    for (int j = 0; j < FUSED_KC; ++j) {
      const int r = t + j;
      if (r < W) {
        const long rr = wrap_add(rbase, r - W, p.R);
        win[j] = *reinterpret_cast<const uint32_t*>(p.ring + rr * p.C + c0);
      } else {
        win[j] = *reinterpret_cast<const uint32_t*>(p.proj + (size_t)(r - W) * p.p_stride + c0);
      }
    }
    const u32x4 taps = load16(p.cw + (size_t)c0 * FUSED_KC);   // c0: x0 x1 x2 x3 | c0+1: x0 x1 x2 x3
    const float w0[4] = {bf16_lo(taps.x), bf16_hi(taps.x), bf16_lo(taps.y), bf16_hi(taps.y)};
    const float w1[4] = {bf16_lo(taps.z), bf16_hi(taps.z), bf16_lo(taps.w), bf16_hi(taps.w)};
    float acc0 = 0.0f, acc1 = 0.0f;
#pragma unroll
    for (int j = 0; j < FUSED_KC; ++j) {
      acc0 = fmaf(bf16_lo(win[j]), w0[j], acc0);
      acc1 = fmaf(bf16_hi(win[j]), w1[j], acc1);
    }
    if (part == 2 || ring_qk) {
      const long rr = wrap_add(rbase, t, p.R);
      *reinterpret_cast<uint32_t*>(p.ring + rr * p.C + c0) = win[W];
    }
    float s0 = silu(acc0), s1 = silu(acc1);
    float* dst = part == 0 ? qs[t] : part == 1 ? ks[t] : vs[t];
    if (part < 2) {
      const float ss = wave_allsum(fmaf(s0, s0, s1 * s1));
      const float inv = rsqrtf(ss / 128.0f + p.qk_eps);
      const float sc = part == 0 ? p.q_scale : p.k_scale;
      s0 = s0 * inv * sc;
      s1 = s1 * inv * sc;
    }
    const uint32_t pk = pack_bf16x2(s0, s1);
    dst[2 * lane] = bf16_lo(pk);
    dst[2 * lane + 1] = bf16_hi(pk);
  }
  __syncthreads();

  // 2. recurrence
  for (int t = 0; t < T; ++t) {
    const float g = gb_s[0][t];
    const float beta = gb_s[1][t];
    float kk[8], qq[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      kk[i] = ks[t][l16 * 8 + i];
      qq[i] = qs[t][l16 * 8 + i];
    }
    long slot = -1;
    if (p.snap_every || t == T - 1) slot = wrap_add(cur, (1 + t) % p.n_slots, p.n_slots);
#pragma unroll
    for (int r = 0; r < 2; ++r) {
      const int dv = grp + 64 * r;
      float kv = 0.0f;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        st[r][i] *= g;
        kv = fmaf(st[r][i], kk[i], kv);
      }
      kv = row16_allsum(kv);
      const float delta = (vs[t][dv] - kv) * beta;
      float o = 0.0f;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        st[r][i] = fmaf(kk[i], delta, st[r][i]);
        o = fmaf(st[r][i], qq[i], o);
      }
      o = row16_allsum(o);
      if (l16 == 0) ys[t][dv] = bf16_to_f32(f32_to_bf16(o));
      if (slot >= 0) {
        float* dstp = p.state + slot * slot_stride + row_off[r];
        u32x4 o0, o1;
        o0.x = __float_as_uint(st[r][0]); o0.y = __float_as_uint(st[r][1]);
        o0.z = __float_as_uint(st[r][2]); o0.w = __float_as_uint(st[r][3]);
        o1.x = __float_as_uint(st[r][4]); o1.y = __float_as_uint(st[r][5]);
        o1.z = __float_as_uint(st[r][6]); o1.w = __float_as_uint(st[r][7]);
        __builtin_nontemporal_store(o0, reinterpret_cast<u32x4*>(dstp));
        __builtin_nontemporal_store(o1, reinterpret_cast<u32x4*>(dstp + 4));
      }
    }
  }
  __syncthreads();

  // 3. gated RMSNorm: one wave per token (T <= 8 < 16 waves), 2 channels per lane
  if (wave < T) {
    const int t = wave;
    const float y0 = ys[t][2 * lane], y1 = ys[t][2 * lane + 1];
    float ss = 0.0f;
    ss = fmaf(y0, y0, fmaf(y1, y1, ss));
    ss = wave_allsum(ss);
    const float inv = rsqrtf(ss / (float)DK + p.norm_eps);
    const float n0 = bf16_to_f32(f32_to_bf16(bf16_lo(wp) * (y0 * inv)));
    const float n1 = bf16_to_f32(f32_to_bf16(bf16_hi(wp) * (y1 * inv)));
    const float z0 = bf16_lo(zp), z1 = bf16_hi(zp);
    *reinterpret_cast<uint32_t*>(p.out + (size_t)t * p.Hv * DK + hv * DK + 2 * lane) =
        pack_bf16x2(silu(z0) * n0, silu(z1) * n1);
  }
}

// The mixer with each value head split over NB blocks of 128 / NB state rows
// (one row per 16-lane DPP row, the arithmetic of gdn_recurrent_kernel), so the
// recurrence fills NB * Hv CUs. The gated RMSNorm's per-(token, head) scale
// rsqrt(mean(y^2) + eps) would need all 128 rows of a head; it commutes with the
// out_proj product, so each block writes instead
//   u = bf16(silu(z) * (w * y))            (y the bf16 recurrence output)
//   ss_parts[(t * Hv + head) * NB + b] = the sum of y^2 over its rows,
// and the out_proj applies the scale to each 128-column segment of its input
// as it stages it (qvex_qmv_w4g64_packed_resid with a segment scale). The conv
// ring and state ring are bitwise those of the other forms.
// TT: the token count (p.T == TT, 1..FUSED_TMAX) as a compile-time constant:
// the token loop is unrolled into one branch-free block, so one token's output
// dot, gated-norm input and snapshot overlap the next token's state update (the
// same operations in the same order as a loop: the same bits).
// What the first loads need - the token-count pointer, the state, projection,
// conv-ring and conv-weight pointers and the shape, small values packed in
// pairs of 16 bits - is passed as scalar arguments ahead of the argument struct
// (an aggregate is never preloaded into SGPRs: 14 dwords are), so the count's
// load and the count-independent loads go out at wave start instead of after a
// chain of waits for struct fields, the count, then more fields.
//   dims0 = p_stride | R << 16, dims1 = n_slots | Hv << 8 | Hk << 16,
//   dims2 = z_off | ab_off << 16, dims3 = C | key_dim << 16.
// Blocks have at least 8 waves: with 8 blocks per head the 4 waves past the
// 16 state rows only run conv tasks (a 4-token verify's T + 1 tasks stay one
// round), while the state rows get one wave per SIMD.
template <int NB>
constexpr int split_threads() { return 16 * (DK / NB) < 512 ? 512 : 16 * (DK / NB); }

template <int NB, int TT>
__global__ __launch_bounds__(split_threads<NB>()) void gdn_decode_split_kernel(
    const int32_t* __restrict__ counter, float* __restrict__ state_, const uint16_t* __restrict__ proj_,
    uint16_t* __restrict__ ring_, const uint16_t* __restrict__ cw_, uint32_t dims0, uint32_t dims1, uint32_t dims2,
    uint32_t dims3, GdnFusedArgs p, float* ss_parts) {
  const int p_stride_ = (int)(dims0 & 0xffffu), R_ = (int)(dims0 >> 16);
  const int n_slots_ = (int)(dims1 & 0xffu), Hv_ = (int)((dims1 >> 8) & 0xffu), Hk_ = (int)(dims1 >> 16);
  const int z_off_ = (int)(dims2 & 0xffffu), ab_off_ = (int)(dims2 >> 16);
  const int C_ = (int)(dims3 & 0xffffu), key_dim_ = (int)(dims3 >> 16);
  constexpr int RB = DK / NB;            // rows per block
  constexpr int NREC = 16 * RB;          // threads on state rows (the first NREC / 64 waves)
  constexpr int NW = split_threads<NB>() / 64;   // waves
  __shared__ float qs[FUSED_TMAX][DK], ks[FUSED_TMAX][DK], vs[FUSED_TMAX][RB], ys[FUSED_TMAX][RB];
  __shared__ float gb_s[2][FUSED_TMAX];
  const int hv = blockIdx.x / NB, b = blockIdx.x % NB;
  const int hk = hv / (Hv_ / Hk_);
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int grp = threadIdx.x >> 4, l16 = threadIdx.x & 15;
  const bool rec = threadIdx.x < NREC;   // uniform per wave
  const int dv = b * RB + (rec ? grp : 0);   // conv-only waves: a valid row, never used
  constexpr int T = TT;
  const long p0 = *counter;
  const int cur = (int)(((p0 % n_slots_) + n_slots_) % n_slots_);
  const int rbase = (int)(((p0 % R_) + R_) % R_);
  const long slot_stride = (long)Hv_ * DK * DK;
  // this block's state row first (it waits on the token count)
  const long row_off = ((long)hv * DK + dv) * DK + l16 * 8;
  float st[8] = {};
  if (rec) {
    const float* src = state_ + cur * slot_stride + row_off;
    const u32x4 s0 = load16(src);
    const u32x4 s1 = load16(src + 4);
    st[0] = __uint_as_float(s0.x); st[1] = __uint_as_float(s0.y);
    st[2] = __uint_as_float(s0.z); st[3] = __uint_as_float(s0.w);
    st[4] = __uint_as_float(s1.x); st[5] = __uint_as_float(s1.y);
    st[6] = __uint_as_float(s1.z); st[7] = __uint_as_float(s1.w);
  }
  // the tokens' decay and beta inputs: lanes t < T of the first wave without a
  // conv task below (the last wave when every wave has one), so that their
  // transcendentals do not lengthen a conv task's wave; converted after the
  // conv tasks so that no wave waits on them before issuing its conv loads
  constexpr int GATE_WAVE = T + (T + 2 * 64 / RB - 1) / (2 * 64 / RB) < NW ? T + (T + 2 * 64 / RB - 1) / (2 * 64 / RB)
                                                                            : NW - 1;
  const bool gate_lane = wave == GATE_WAVE && lane < T;
  float a_log = 0.0f;
  uint32_t dt_raw = 0, aa_raw = 0, bb_raw = 0;
  if (gate_lane) {
    const int t = lane;
    a_log = p.A_log[hv];
    dt_raw = p.dt_bias[hv];
    aa_raw = proj_[(size_t)t * p_stride_ + ab_off_ + Hv_ + hv];
    bb_raw = proj_[(size_t)t * p_stride_ + ab_off_ + hv];
  }
  // lane t of a row: the row's z of token t (lanes past T re-read token T - 1)
  // and its norm weight, both first waited for after the recurrence, where
  // lane t writes token t's output
  const uint32_t z_own = proj_[(size_t)min(l16, T - 1) * p_stride_ + z_off_ + hv * DK + dv];
  const uint32_t wr_raw = p.norm_w[dv];
  // 1. conv + silu. Two kinds of task, each one wave with all of its loads
  // issued in its own iteration: a token's q and k heads (lane: channels 2l,
  // 2l+1 of both, each head normed by its own wave sum as in
  // conv_silu_qk_kernel), and this block's RB v channels for VTOK tokens at
  // once (lane: one token and channel pair). T + ceil(T / VTOK) tasks, so a
  // 4-token verify is one round of loads on 8 waves. The q / k ring rows are
  // written by one block per k head.
  constexpr int W = FUSED_KC - 1;
  constexpr int VPT = RB / 2;          // v channel pairs per token
  constexpr int VTOK = 64 / VPT;       // tokens per v task
  const bool ring_qk = hv % (Hv_ / Hk_) == 0 && b == 0;
  auto conv_pair = [&](const uint32_t (&win)[FUSED_KC], const u32x4 taps, float& s0, float& s1) {
    const float w0[4] = {bf16_lo(taps.x), bf16_hi(taps.x), bf16_lo(taps.y), bf16_hi(taps.y)};
    const float w1[4] = {bf16_lo(taps.z), bf16_hi(taps.z), bf16_lo(taps.w), bf16_hi(taps.w)};
    float acc0 = 0.0f, acc1 = 0.0f;
#pragma unroll
    for (int j = 0; j < FUSED_KC; ++j) {
      acc0 = fmaf(bf16_lo(win[j]), w0[j], acc0);
      acc1 = fmaf(bf16_hi(win[j]), w1[j], acc1);
    }
    s0 = silu(acc0);
    s1 = silu(acc1);
  };
  const int n_vt = (T + VTOK - 1) / VTOK;
  static_assert(VTOK == 2 * 64 / RB, "gate wave placement assumes this v-task width");
  for (int task = wave; task < T + n_vt; task += NW) {
    if (task < T) {                       // uniform over the wave
      const int t = task;
      const int cq = hk * DK + 2 * lane, ck = key_dim_ + hk * DK + 2 * lane;
      uint32_t wq[FUSED_KC], wk[FUSED_KC];
#pragma unroll
      for (int j = 0; j < FUSED_KC; ++j) {
        const int r = t + j;
        if (r < W) {
          const long rr = wrap_add(rbase, r - W, R_);
          wq[j] = *reinterpret_cast<const uint32_t*>(ring_ + rr * C_ + cq);
          wk[j] = *reinterpret_cast<const uint32_t*>(ring_ + rr * C_ + ck);
        } else {
          wq[j] = *reinterpret_cast<const uint32_t*>(proj_ + (size_t)(r - W) * p_stride_ + cq);
          wk[j] = *reinterpret_cast<const uint32_t*>(proj_ + (size_t)(r - W) * p_stride_ + ck);
        }
      }
      const u32x4 tq = load16(cw_ + (size_t)cq * FUSED_KC);
      const u32x4 tk = load16(cw_ + (size_t)ck * FUSED_KC);
      if (ring_qk) {
        const long rr = wrap_add(rbase, t, R_);
        *reinterpret_cast<uint32_t*>(ring_ + rr * C_ + cq) = wq[W];
        *reinterpret_cast<uint32_t*>(ring_ + rr * C_ + ck) = wk[W];
      }
      float q0, q1, k0, k1;
      conv_pair(wq, tq, q0, q1);
      conv_pair(wk, tk, k0, k1);
      const float iq = rsqrtf(wave_allsum(fmaf(q0, q0, q1 * q1)) / 128.0f + p.qk_eps);
      const float ik = rsqrtf(wave_allsum(fmaf(k0, k0, k1 * k1)) / 128.0f + p.qk_eps);
      const uint32_t pq = pack_bf16x2(q0 * iq * p.q_scale, q1 * iq * p.q_scale);
      const uint32_t pk = pack_bf16x2(k0 * ik * p.k_scale, k1 * ik * p.k_scale);
      qs[t][2 * lane] = bf16_lo(pq);
      qs[t][2 * lane + 1] = bf16_hi(pq);
      ks[t][2 * lane] = bf16_lo(pk);
      ks[t][2 * lane + 1] = bf16_hi(pk);
    } else {
      const int t = (task - T) * VTOK + lane / VPT, cp = lane % VPT;
      if (t < T) {
        const int c0 = 2 * key_dim_ + hv * DK + b * RB + 2 * cp;
        uint32_t win[FUSED_KC];
#pragma unroll
        for (int j = 0; j < FUSED_KC; ++j) {
          const int r = t + j;
          if (r < W) {
            const long rr = wrap_add(rbase, r - W, R_);
            win[j] = *reinterpret_cast<const uint32_t*>(ring_ + rr * C_ + c0);
          } else {
            win[j] = *reinterpret_cast<const uint32_t*>(proj_ + (size_t)(r - W) * p_stride_ + c0);
          }
        }
        const u32x4 taps = load16(cw_ + (size_t)c0 * FUSED_KC);
        const long rr = wrap_add(rbase, t, R_);
        *reinterpret_cast<uint32_t*>(ring_ + rr * C_ + c0) = win[W];
        float v0, v1;
        conv_pair(win, taps, v0, v1);
        const uint32_t pv = pack_bf16x2(v0, v1);
        vs[t][2 * cp] = bf16_lo(pv);
        vs[t][2 * cp + 1] = bf16_hi(pv);
      }
    }
  }
  if (gate_lane) {
    const int t = lane;
    // empty asm: keeps the compiler from hoisting these conversions (and the
    // wait for their loads) back above the conv tasks
    asm volatile("" : "+v"(a_log), "+v"(dt_raw), "+v"(aa_raw), "+v"(bb_raw));
    const float A = expf(a_log);
    const float x = bf16_to_f32((uint16_t)aa_raw) + bf16_to_f32((uint16_t)dt_raw);
    const float sp = x > 20.0f ? x : log1pf(expf(x));
    gb_s[0][t] = expf(-A * sp);
    gb_s[1][t] = 1.0f / (1.0f + expf(-bf16_to_f32((uint16_t)bb_raw)));
  }
  __syncthreads();

  // 2. recurrence; u of this block's rows to `out`, y to LDS for the sums.
  // Each token's snapshot address, computed once in scalar registers (without
  // per-token snapshots every token stores to the final slot: the last store
  // wins, no branch in the unrolled form).
  float* snap[TT];
#pragma unroll
  for (int t = 0; t < TT; ++t) {
    int s = cur + (p.snap_every ? 1 + t : T);
    while (s >= n_slots_) s -= n_slots_;
    snap[t] = state_ + s * slot_stride + row_off;
  }
  if (rec) {
    float ot[TT];
    auto token = [&](int t) {
      const float g = gb_s[0][t];
      const float beta = gb_s[1][t];
      float kk[8], qq[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        kk[i] = ks[t][l16 * 8 + i];
        qq[i] = qs[t][l16 * 8 + i];
      }
      float kv = 0.0f;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        st[i] *= g;
        kv = fmaf(st[i], kk[i], kv);
      }
      kv = row16_allsum(kv);
      const float delta = (vs[t][grp] - kv) * beta;
      float o = 0.0f;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        st[i] = fmaf(kk[i], delta, st[i]);
        o = fmaf(st[i], qq[i], o);
      }
      ot[t] = row16_allsum(o);
      u32x4 o0, o1;
      o0.x = __float_as_uint(st[0]); o0.y = __float_as_uint(st[1]);
      o0.z = __float_as_uint(st[2]); o0.w = __float_as_uint(st[3]);
      o1.x = __float_as_uint(st[4]); o1.y = __float_as_uint(st[5]);
      o1.z = __float_as_uint(st[6]); o1.w = __float_as_uint(st[7]);
      __builtin_nontemporal_store(o0, reinterpret_cast<u32x4*>(snap[t]));
      __builtin_nontemporal_store(o1, reinterpret_cast<u32x4*>(snap[t] + 4));
    };
#pragma unroll
    for (int t = 0; t < TT; ++t) token(t);
    // the outputs, one lane per token: lane t of a row takes lane 0's sum of
    // token t (the lanes' sums may differ in the last bit) by a row shift, then
    // rounds it, gates it and stores it: once per (row, token) instead of in all
    // 16 lanes inside the state chain
    float orow = ot[0];
#pragma unroll
    for (int t = 1; t < TT; ++t) {
      const float sh = row_shr_n(ot[t], t);
      orow = l16 == t ? sh : orow;
    }
    if (l16 < T) {
      const int t = l16;
      const float y = bf16_to_f32(f32_to_bf16(orow));
      ys[t][grp] = y;
      const float zt = bf16_to_f32((uint16_t)z_own);
      p.out[(size_t)t * Hv_ * DK + hv * DK + dv] = f32_to_bf16(silu(zt) * (bf16_to_f32((uint16_t)wr_raw) * y));
    }
  }
  __syncthreads();
  // 3. per token, the sum of y^2 over this block's rows: one wave per token,
  // lane r < RB squares row r, a DPP sum over the wave
  for (int t = wave; t < T; t += NW) {
    const float y = lane < RB ? ys[t][lane] : 0.0f;
    const float ss = wave_allsum(y * y);
    if (lane == 0) ss_parts[((size_t)t * Hv_ + hv) * NB + b] = ss;
  }
}

int check_common(const char* fn, int B, int T, int Hk, int Hv, int Dk, int Dv) {
  QVEX_CHECK_ARG(B >= 1 && T >= 1, "%s: B=%d T=%d must be >= 1", fn, B, T);
  QVEX_CHECK_ARG(Hk >= 1 && Hv >= Hk && Hv % Hk == 0, "%s: Hv=%d must be a multiple of Hk=%d", fn, Hv, Hk);
  if (Dk != DK || Dv % ROWS_PER_BLOCK != 0)
    return qvex::fail(QVEX_ENOTSUP, "%s: needs Dk=128 and Dv %% 16 == 0 (got Dk=%d Dv=%d)", fn, Dk, Dv);
  return QVEX_OK;
}

int launch(const GdnArgs& p, hipStream_t stream) {
  const int blocks = p.B * p.Hv * (p.Dv / ROWS_PER_BLOCK);
  hipLaunchKernelGGL(gdn_recurrent_kernel, dim3(blocks), dim3(256), 0, stream, p);
  QVEX_CHECK_LAUNCH("qvex_gdn_recurrent");
  return QVEX_OK;
}

}  // namespace

extern "C" int qvex_gdn_recurrent(const uint16_t* q, const uint16_t* k, const uint16_t* v,
                                  const uint16_t* a, const uint16_t* b, const float* A_log,
                                  const uint16_t* dt_bias, const float* state_in, float* snapshots,
                                  int snap_every, uint16_t* y, int B, int T, int Hk, int Hv, int Dk,
                                  int Dv, void* stream) {
  if (int rc = check_common("qvex_gdn_recurrent", B, T, Hk, Hv, Dk, Dv)) return rc;
  QVEX_CHECK_ARG(q && k && v && a && b && A_log && dt_bias && state_in && snapshots && y,
                 "qvex_gdn_recurrent: null pointer");
  QVEX_CHECK_ARG(qvex_aligned(q, 16) && qvex_aligned(k, 16) && qvex_aligned(state_in, 16) &&
                     qvex_aligned(snapshots, 16),
                 "qvex_gdn_recurrent: q, k, state_in, snapshots must be 16-byte aligned");
  GdnArgs p{q, k, v, a, b, A_log, dt_bias, state_in, snapshots, nullptr,
            (long)B * Hv * Dv * Dk, 0, snap_every ? 1 : 0, y, B, T, Hk, Hv, Dv};
  return launch(p, (hipStream_t)stream);
}

extern "C" int qvex_gdn_recurrent_ring(const uint16_t* q, const uint16_t* k, const uint16_t* v,
                                       const uint16_t* a, const uint16_t* b, const float* A_log,
                                       const uint16_t* dt_bias, float* ring, int n_slots,
                                       const int32_t* cur_slot, int snap_every, uint16_t* y, int B, int T,
                                       int Hk, int Hv, int Dk, int Dv, void* stream) {
  if (int rc = check_common("qvex_gdn_recurrent_ring", B, T, Hk, Hv, Dk, Dv)) return rc;
  QVEX_CHECK_ARG(q && k && v && a && b && A_log && dt_bias && ring && cur_slot && y,
                 "qvex_gdn_recurrent_ring: null pointer");
  QVEX_CHECK_ARG(n_slots >= 2 && (!snap_every || n_slots >= T + 1),
                 "qvex_gdn_recurrent_ring: n_slots=%d must be >= T+1=%d with snapshots (>= 2 without)", n_slots, T + 1);
  QVEX_CHECK_ARG(qvex_aligned(q, 16) && qvex_aligned(k, 16) && qvex_aligned(ring, 16),
                 "qvex_gdn_recurrent_ring: q, k, ring must be 16-byte aligned");
  GdnArgs p{q, k, v, a, b, A_log, dt_bias, ring, ring, cur_slot,
            (long)B * Hv * Dv * Dk, n_slots, snap_every ? 1 : 0, y, B, T, Hk, Hv, Dv};
  return launch(p, (hipStream_t)stream);
}

extern "C" int qvex_gdn_decode_fused(const uint16_t* proj, long p_stride, uint16_t* conv_ring, int ring_rows,
                                     const int32_t* counter, const uint16_t* conv_w, int kernel_size, int conv_dim,
                                     int key_dim, float q_scale, float k_scale, float qk_eps, const float* A_log,
                                     const uint16_t* dt_bias, int z_offset, int ab_offset, float* state_ring,
                                     int n_slots, int snap_every, const uint16_t* norm_w, float norm_eps,
                                     uint16_t* out, int T, int Hk, int Hv, int Dk, int Dv, void* stream) {
  QVEX_CHECK_ARG(proj && conv_ring && counter && conv_w && A_log && dt_bias && state_ring && norm_w && out,
                 "qvex_gdn_decode_fused: null pointer");
  QVEX_CHECK_ARG(T >= 1 && T <= FUSED_TMAX, "qvex_gdn_decode_fused: T=%d must be in 1..%d", T, FUSED_TMAX);
  if (Dk != DK || Dv != DK)
    return qvex::fail(QVEX_ENOTSUP, "qvex_gdn_decode_fused: needs Dk = Dv = 128 (got %d, %d)", Dk, Dv);
  QVEX_CHECK_ARG(Hk >= 1 && Hv >= Hk && Hv % Hk == 0, "qvex_gdn_decode_fused: Hv=%d must be a multiple of Hk=%d",
                 Hv, Hk);
  QVEX_CHECK_ARG(key_dim == Hk * DK && conv_dim == 2 * key_dim + Hv * DK,
                 "qvex_gdn_decode_fused: conv_dim=%d key_dim=%d do not match Hk=%d Hv=%d", conv_dim, key_dim, Hk, Hv);
  if (kernel_size != FUSED_KC)
    return qvex::fail(QVEX_ENOTSUP, "qvex_gdn_decode_fused: needs kernel_size = %d (got %d)", FUSED_KC, kernel_size);
  QVEX_CHECK_ARG(ring_rows >= T + kernel_size - 1, "qvex_gdn_decode_fused: ring_rows=%d < T + K - 1 = %d",
                 ring_rows, T + kernel_size - 1);
  QVEX_CHECK_ARG(n_slots >= 2 && (!snap_every || n_slots >= T + 1),
                 "qvex_gdn_decode_fused: n_slots=%d must be >= T+1=%d with snapshots (>= 2 without)", n_slots, T + 1);
  QVEX_CHECK_ARG(p_stride % 2 == 0 && conv_dim <= p_stride && z_offset % 2 == 0 && z_offset + Hv * DK <= p_stride &&
                     ab_offset >= 0 && ab_offset + 2 * Hv <= p_stride,
                 "qvex_gdn_decode_fused: p_stride=%ld z_offset=%d ab_offset=%d do not fit the projection row",
                 p_stride, z_offset, ab_offset);
  QVEX_CHECK_ARG(qvex_aligned(proj, 4) && qvex_aligned(conv_ring, 4) && qvex_aligned(norm_w, 4) &&
                     qvex_aligned(out, 4) && qvex_aligned(state_ring, 16) && qvex_aligned(conv_w, 16),
                 "qvex_gdn_decode_fused: proj, conv_ring, norm_w, out need 4-byte and state_ring, conv_w 16-byte "
                 "alignment");
  GdnFusedArgs p{proj, p_stride, conv_ring, ring_rows, counter, conv_w, conv_dim, key_dim,
                 q_scale, k_scale, qk_eps, A_log, dt_bias, z_offset, ab_offset, state_ring, n_slots,
                 snap_every ? 1 : 0, norm_w, norm_eps, out, T, Hk, Hv};
  hipLaunchKernelGGL(gdn_decode_fused_kernel, dim3(Hv), dim3(FUSED_THREADS), 0, (hipStream_t)stream, p);
  QVEX_CHECK_LAUNCH("qvex_gdn_decode_fused");
  return QVEX_OK;
}

template <int NB, int TT>
void launch_split_t(dim3 grid, hipStream_t st, const GdnFusedArgs& p, float* ss_parts) {
  const uint32_t d0 = (uint32_t)p.p_stride | ((uint32_t)p.R << 16);
  const uint32_t d1 = (uint32_t)p.n_slots | ((uint32_t)p.Hv << 8) | ((uint32_t)p.Hk << 16);
  const uint32_t d2 = (uint32_t)p.z_off | ((uint32_t)p.ab_off << 16);
  const uint32_t d3 = (uint32_t)p.C | ((uint32_t)p.key_dim << 16);
  hipLaunchKernelGGL((gdn_decode_split_kernel<NB, TT>), grid, dim3(split_threads<NB>()), 0, st, p.counter, p.state, p.proj,
                     p.ring, p.cw, d0, d1, d2, d3, p, ss_parts);
}

template <int NB>
void launch_split(dim3 grid, int T, hipStream_t st, const GdnFusedArgs& p, float* ss_parts) {
  static_assert(FUSED_TMAX == 8, "one instantiation per token count");
  switch (T) {
    case 1: launch_split_t<NB, 1>(grid, st, p, ss_parts); break;
    case 2: launch_split_t<NB, 2>(grid, st, p, ss_parts); break;
    case 3: launch_split_t<NB, 3>(grid, st, p, ss_parts); break;
    case 4: launch_split_t<NB, 4>(grid, st, p, ss_parts); break;
    case 5: launch_split_t<NB, 5>(grid, st, p, ss_parts); break;
    case 6: launch_split_t<NB, 6>(grid, st, p, ss_parts); break;
    case 7: launch_split_t<NB, 7>(grid, st, p, ss_parts); break;
    case 8: launch_split_t<NB, 8>(grid, st, p, ss_parts); break;
  }
}

extern "C" int qvex_gdn_decode_split(const uint16_t* proj, long p_stride, uint16_t* conv_ring, int ring_rows,
                                     const int32_t* counter, const uint16_t* conv_w, int kernel_size, int conv_dim,
                                     int key_dim, float q_scale, float k_scale, float qk_eps, const float* A_log,
                                     const uint16_t* dt_bias, int z_offset, int ab_offset, float* state_ring,
                                     int n_slots, int snap_every, const uint16_t* norm_w, uint16_t* u_out,
                                     float* ss_parts, int T, int Hk, int Hv, int Dk, int Dv, int blocks_per_head,
                                     void* stream) {
  const char* fn = "qvex_gdn_decode_split";
  QVEX_CHECK_ARG(proj && conv_ring && counter && conv_w && A_log && dt_bias && state_ring && norm_w && u_out &&
                     ss_parts,
                 "%s: null pointer", fn);
  QVEX_CHECK_ARG(blocks_per_head == 2 || blocks_per_head == 4 || blocks_per_head == 8,
                 "%s: blocks_per_head=%d must be 2, 4 or 8", fn, blocks_per_head);
  QVEX_CHECK_ARG(T >= 1 && T <= FUSED_TMAX, "%s: T=%d must be in 1..%d", fn, T, FUSED_TMAX);
  if (Dk != DK || Dv != DK) return qvex::fail(QVEX_ENOTSUP, "%s: needs Dk = Dv = 128 (got %d, %d)", fn, Dk, Dv);
  QVEX_CHECK_ARG(Hk >= 1 && Hv >= Hk && Hv % Hk == 0, "%s: Hv=%d must be a multiple of Hk=%d", fn, Hv, Hk);
  QVEX_CHECK_ARG(key_dim == Hk * DK && conv_dim == 2 * key_dim + Hv * DK,
                 "%s: conv_dim=%d key_dim=%d do not match Hk=%d Hv=%d", fn, conv_dim, key_dim, Hk, Hv);
  if (kernel_size != FUSED_KC)
    return qvex::fail(QVEX_ENOTSUP, "%s: needs kernel_size = %d (got %d)", fn, FUSED_KC, kernel_size);
  QVEX_CHECK_ARG(ring_rows >= T + kernel_size - 1, "%s: ring_rows=%d < T + K - 1 = %d", fn, ring_rows,
                 T + kernel_size - 1);
  QVEX_CHECK_ARG(n_slots >= 2 && (!snap_every || n_slots >= T + 1),
                 "%s: n_slots=%d must be >= T+1=%d with snapshots (>= 2 without)", fn, n_slots, T + 1);
  QVEX_CHECK_ARG(p_stride % 2 == 0 && conv_dim <= p_stride && z_offset + Hv * DK <= p_stride && ab_offset >= 0 &&
                     ab_offset + 2 * Hv <= p_stride,
                 "%s: p_stride=%ld z_offset=%d ab_offset=%d do not fit the projection row", fn, p_stride, z_offset,
                 ab_offset);
  QVEX_CHECK_ARG(qvex_aligned(proj, 4) && qvex_aligned(conv_ring, 4) && qvex_aligned(state_ring, 16) &&
                     qvex_aligned(conv_w, 16),
                 "%s: proj, conv_ring need 4-byte and state_ring, conv_w 16-byte alignment", fn);
  QVEX_CHECK_ARG(p_stride < 65536 && ring_rows < 65536 && n_slots < 256 && Hv < 256 && Hk < 65536 &&
                     z_offset < 65536 && ab_offset < 65536 && conv_dim < 65536 && key_dim < 65536,
                 "%s: p_stride, ring_rows, offsets and dims must be below 65536 (n_slots, Hv below 256)", fn);
  GdnFusedArgs p{proj, p_stride, conv_ring, ring_rows, counter, conv_w, conv_dim, key_dim,
                 q_scale, k_scale, qk_eps, A_log, dt_bias, z_offset, ab_offset, state_ring, n_slots,
                 snap_every ? 1 : 0, norm_w, 0.0f, u_out, T, Hk, Hv};
  const dim3 grid(Hv * blocks_per_head);
  switch (blocks_per_head) {
    case 2: launch_split<2>(grid, T, (hipStream_t)stream, p, ss_parts); break;
    case 4: launch_split<4>(grid, T, (hipStream_t)stream, p, ss_parts); break;
    case 8: launch_split<8>(grid, T, (hipStream_t)stream, p, ss_parts); break;
  }
  QVEX_CHECK_LAUNCH(fn);
  return QVEX_OK;
}
