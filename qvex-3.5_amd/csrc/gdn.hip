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

template <int CTRL>
__device__ __forceinline__ float dpp_row(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xf, 0xf, false));
}

// Sum over the 16 lanes of a DPP row, broadcast to all 16.
__device__ __forceinline__ float row16_allsum(float v) {
  v += dpp_row<0xB1>(v);   // quad_perm [1,0,3,2]
  v += dpp_row<0x4E>(v);   // quad_perm [2,3,0,1]
  v += dpp_row<0x124>(v);  // row_ror 4
  v += dpp_row<0x128>(v);  // row_ror 8
  return v;
}

__device__ __forceinline__ void load8_bf16(const uint16_t* p, float* o) {
  const u32x4 v = load16(p);
  o[0] = bf16_lo(v.x); o[1] = bf16_hi(v.x);
  o[2] = bf16_lo(v.y); o[3] = bf16_hi(v.y);
  o[4] = bf16_lo(v.z); o[5] = bf16_hi(v.z);
  o[6] = bf16_lo(v.w); o[7] = bf16_hi(v.w);
}

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
  const float A = expf(p.A_log[hv]);
  const float dt = bf16_to_f32(p.dt_bias[hv]);

  for (int t0 = 0; t0 < T; t0 += TMAX_PREFETCH) {
    const int tn = min(TMAX_PREFETCH, T - t0);
    float kk[TMAX_PREFETCH][8], qq[TMAX_PREFETCH][8], vv[TMAX_PREFETCH], aa[TMAX_PREFETCH], bb[TMAX_PREFETCH];
#pragma unroll
    for (int j = 0; j < TMAX_PREFETCH; ++j) {
      if (j < tn) {
        const int t = t0 + j;
        const long qk = (((long)bi * T + t) * p.Hk + hk) * DK + l16 * 8;
        load8_bf16(p.k + qk, kk[j]);
        load8_bf16(p.q + qk, qq[j]);
        vv[j] = bf16_to_f32(p.v[(((long)bi * T + t) * p.Hv + hv) * p.Dv + dv]);
        aa[j] = bf16_to_f32(p.a[((long)bi * T + t) * p.Hv + hv]);
        bb[j] = bf16_to_f32(p.b[((long)bi * T + t) * p.Hv + hv]);
      }
    }
#pragma unroll
    for (int j = 0; j < TMAX_PREFETCH; ++j) {
      if (j < tn) {
        const int t = t0 + j;
        const float x = aa[j] + dt;
        const float sp = x > 20.0f ? x : log1pf(expf(x));
        const float g = expf(-A * sp);
        const float beta = 1.0f / (1.0f + expf(-bb[j]));
        float kv = 0.0f;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          st[i] *= g;
          kv = fmaf(st[i], kk[j][i], kv);
        }
        kv = row16_allsum(kv);
        const float delta = (vv[j] - kv) * beta;
        float o = 0.0f;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          st[i] = fmaf(kk[j][i], delta, st[i]);
          o = fmaf(st[i], qq[j][i], o);
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
          *reinterpret_cast<u32x4*>(dst) = o0;
          *reinterpret_cast<u32x4*>(dst + 4) = o1;
        }
      }
    }
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
