// Generic decode kernel (VALU): every page dtype (f32, f16, Q8A), head_dim
// 64/128/256, 1..8 query heads per kv head.  The f16 / head_dim 128 case has
// a faster MFMA kernel (lnskv_decode_mfma.hip); this one covers the rest.
//
// Grid (kv head, partition, sequence); 256 threads = 4 waves.  The block's
// token range [ta, tb) is its partition of `split` tokens intersected with the
// window [p_start, kv_len) (minus the newest token when the append is fused).
// Pages of the range go round-robin to the 4 waves.  kv heads vary fastest in
// the launch order, so the blocks reading the same slot-major pages run at the
// same time and the DRAM pages they share are opened once.
//
// Lane layout for a page (rows of D*ES bytes, one per token and kv head):
//   LPR = D*ES/16 lanes cover one row with 16-byte loads, RPL = 64/LPR rows
//   per wave load, NLOAD = 16/RPL loads per page.  Lane (r, c) = (lane/LPR,
//   lane%LPR) holds elements [c*EPL, (c+1)*EPL) of token j*RPL + r for load j.
// Query heads of the group live in registers in the same column layout, so a
// score is a per-lane partial dot plus a DPP sum over the row's LPR lanes, and
// the P.V update needs no data exchange at all: acc[h][e] accumulates per row
// and rows are summed once at the end.
#include "lnskv_device.h"

namespace lnskv {
namespace {

// Element (un)packing from a 16-byte lane chunk.
template <int DT>
__device__ __forceinline__ float elem(const uint4& raw, int e) {
  const uint32_t w = (&raw.x)[(e * Storage<DT>::kBytes) / 4];
  if constexpr (DT == LNSKV_DTYPE_F32) {
    return __builtin_bit_cast(float, w);
  } else if constexpr (DT == LNSKV_DTYPE_F16) {
    const uint16_t h = (uint16_t)(w >> (16 * (e & 1)));
    return (float)__builtin_bit_cast(_Float16, h);
  } else {
    return (float)(int8_t)(w >> (8 * (e & 3)));
  }
}

template <int DT, int D, int REP>
struct Geo {
  static constexpr int ES = Storage<DT>::kBytes;
  static constexpr int EPL = 16 / ES;        // elements per lane per load
  static constexpr int LPR = D * ES / 16;    // lanes per row
  static constexpr int RPL = kWave / LPR;    // rows per load
  static constexpr int NLOAD = kPage / RPL;  // loads per page
  static_assert(LPR >= 4 && LPR <= 64, "row must span 4..64 lanes");
};

// Loads one page (K and V chunks of this lane, plus Q8A per-token scales).
template <int DT, int D, int REP>
struct PageRegs {
  using G = Geo<DT, D, REP>;
  uint4 k[G::NLOAD];
  uint4 v[G::NLOAD];
  float ks[G::NLOAD];
  float vs[G::NLOAD];
};

template <int DT, int D, int REP>
__device__ __forceinline__ void load_page(const DecodeArgs& a, uint32_t phys, int kvh, int r, int c,
                                          PageRegs<DT, D, REP>& pr) {
  using G = Geo<DT, D, REP>;
#pragma unroll
  for (int j = 0; j < G::NLOAD; ++j) {
    const size_t slot = (size_t)phys * kPage + (size_t)(j * G::RPL + r);
    const size_t off = ((slot * a.n_kv + kvh) * D) * G::ES + (size_t)c * 16;
    pr.k[j] = *reinterpret_cast<const uint4*>(a.k_pages + off);
    pr.v[j] = *reinterpret_cast<const uint4*>(a.v_pages + off);
    if constexpr (DT == LNSKV_DTYPE_Q8A) {
      pr.ks[j] = a.k_scales[slot * a.n_kv + kvh];
      pr.vs[j] = a.v_scales[slot * a.n_kv + kvh];
    }
  }
}

template <int DT, int D, int REP>
struct WaveState {
  using G = Geo<DT, D, REP>;
  float q[REP][G::EPL];
  float acc[REP][G::EPL];
  float m[REP];
  float l[REP];
};

// One page through the online softmax.  `full` means every token of the page
// is inside [ta, tb) and the page is valid; otherwise token validity is
// checked per row and masked V chunks are zeroed (unwritten slots may hold any
// bits, NaN included).
template <int DT, int D, int REP>
__device__ __forceinline__ void consume_page(WaveState<DT, D, REP>& st, const PageRegs<DT, D, REP>& pr,
                                             bool full, bool valid, int tok0, int ta, int tb, int r) {
  using G = Geo<DT, D, REP>;
  float s[G::NLOAD][REP];
#pragma unroll
  for (int j = 0; j < G::NLOAD; ++j) {
#pragma unroll
    for (int h = 0; h < REP; ++h) {
      float part = 0.0f;
#pragma unroll
      for (int e = 0; e < G::EPL; ++e) part = fmaf(elem<DT>(pr.k[j], e), st.q[h][e], part);
      s[j][h] = group_sum<G::LPR>(part);
      if constexpr (DT == LNSKV_DTYPE_Q8A) s[j][h] *= pr.ks[j];
    }
  }
  bool tok_ok[G::NLOAD];
#pragma unroll
  for (int j = 0; j < G::NLOAD; ++j) {
    const int t = tok0 + j * G::RPL + r;
    tok_ok[j] = full || (valid && t >= ta && t < tb);
    if (!tok_ok[j]) {
#pragma unroll
      for (int h = 0; h < REP; ++h) s[j][h] = -INFINITY;
    }
  }
  float alpha[REP];
#pragma unroll
  for (int h = 0; h < REP; ++h) {
    float mx = s[0][h];
#pragma unroll
    for (int j = 1; j < G::NLOAD; ++j) mx = fmaxf(mx, s[j][h]);
    mx = cross_max<G::LPR>(mx);
    const float m_new = fmaxf(st.m[h], mx);
    alpha[h] = fast_exp2(st.m[h] - m_new);
    st.m[h] = m_new;
    float lsum = 0.0f;
#pragma unroll
    for (int j = 0; j < G::NLOAD; ++j) {
      s[j][h] = fast_exp2(s[j][h] - m_new);  // now p
      lsum += s[j][h];
    }
    st.l[h] = fmaf(alpha[h], st.l[h], lsum);
#pragma unroll
    for (int e = 0; e < G::EPL; ++e) st.acc[h][e] *= alpha[h];
  }
#pragma unroll
  for (int j = 0; j < G::NLOAD; ++j) {
    float pj[REP];
#pragma unroll
    for (int h = 0; h < REP; ++h) {
      pj[h] = s[j][h];
      if constexpr (DT == LNSKV_DTYPE_Q8A) pj[h] *= pr.vs[j];
    }
#pragma unroll
    for (int e = 0; e < G::EPL; ++e) {
      float ve = elem<DT>(pr.v[j], e);
      if (!full) ve = tok_ok[j] ? ve : 0.0f;
#pragma unroll
      for (int h = 0; h < REP; ++h) st.acc[h][e] = fmaf(pj[h], ve, st.acc[h][e]);
    }
  }
}

// The newest token (fused append): lanes of row 0 convert k_new/v_new to the
// page dtype, store them to the token's slot, and feed the stored values to
// the online softmax.  All lanes run the cross-lane steps; only row 0 loads,
// stores and accumulates.
template <int DT, int D, int REP>
__device__ __forceinline__ void fused_new_token(const DecodeArgs& a, WaveState<DT, D, REP>& st, int s,
                                                int kvh, int pos, bool attend, int lane) {
  using G = Geo<DT, D, REP>;
  const int r = lane / G::LPR, c = lane % G::LPR;
  const bool row0 = r == 0;
  const int lp = pos / kPage;
  const uint32_t phys = a.bt[(size_t)s * a.bt_stride + lp];
  const bool valid = phys < a.num_pages;
  const size_t slot = (size_t)phys * kPage + (size_t)(pos % kPage);
  const size_t src = ((size_t)s * a.n_kv + kvh) * D + (size_t)c * G::EPL;
  float kx[G::EPL], vx[G::EPL];
#pragma unroll
  for (int e = 0; e < G::EPL; ++e) {
    kx[e] = row0 ? a.k_new[src + e] : 0.0f;
    vx[e] = row0 ? a.v_new[src + e] : 0.0f;
  }
  // Convert to stored values, keep them as floats for the attention update.
  float kst[G::EPL], vst[G::EPL];
  float ksc = 1.0f, vsc = 1.0f;
  uint32_t kw[4] = {0, 0, 0, 0}, vw[4] = {0, 0, 0, 0};
  if constexpr (DT == LNSKV_DTYPE_F32) {
#pragma unroll
    for (int e = 0; e < G::EPL; ++e) {
      kst[e] = kx[e];
      vst[e] = vx[e];
      kw[e] = __builtin_bit_cast(uint32_t, kx[e]);
      vw[e] = __builtin_bit_cast(uint32_t, vx[e]);
    }
  } else if constexpr (DT == LNSKV_DTYPE_F16) {
#pragma unroll
    for (int e = 0; e < G::EPL; ++e) {
      const uint32_t hk = to_f16_bits(kx[e]), hv = to_f16_bits(vx[e]);
      kst[e] = (float)__builtin_bit_cast(_Float16, (uint16_t)hk);
      vst[e] = (float)__builtin_bit_cast(_Float16, (uint16_t)hv);
      kw[e / 2] |= hk << (16 * (e & 1));
      vw[e / 2] |= hv << (16 * (e & 1));
    }
  } else {
    float ka = 0.0f, va = 0.0f;
#pragma unroll
    for (int e = 0; e < G::EPL; ++e) {
      ka = fmaxf(ka, fabsf(kx[e]));
      va = fmaxf(va, fabsf(vx[e]));
    }
    ka = group_max<G::LPR>(ka);
    va = group_max<G::LPR>(va);
    ksc = ka == 0.0f ? 1.0f : ka / 127.0f;
    vsc = va == 0.0f ? 1.0f : va / 127.0f;
#pragma unroll
    for (int e = 0; e < G::EPL; ++e) {
      const int32_t kq = to_q8(kx[e], ksc), vq = to_q8(vx[e], vsc);
      kst[e] = (float)kq;
      vst[e] = (float)vq;
      kw[e / 4] |= ((uint32_t)kq & 0xFFu) << (8 * (e & 3));
      vw[e / 4] |= ((uint32_t)vq & 0xFFu) << (8 * (e & 3));
    }
  }
  if (row0 && valid) {
    const size_t off = ((slot * a.n_kv + kvh) * D) * G::ES + (size_t)c * 16;
    *reinterpret_cast<uint4*>(a.k_pages_w + off) = make_uint4(kw[0], kw[1], kw[2], kw[3]);
    *reinterpret_cast<uint4*>(a.v_pages_w + off) = make_uint4(vw[0], vw[1], vw[2], vw[3]);
    if constexpr (DT == LNSKV_DTYPE_Q8A) {
      if (c == 0) {
        a.k_scales_w[slot * a.n_kv + kvh] = ksc;
        a.v_scales_w[slot * a.n_kv + kvh] = vsc;
      }
    }
  }
  if (!(attend && valid)) return;  // wave-uniform
#pragma unroll
  for (int h = 0; h < REP; ++h) {
    float part = 0.0f;
#pragma unroll
    for (int e = 0; e < G::EPL; ++e) part = fmaf(kst[e], st.q[h][e], part);
    float sc = group_sum<G::LPR>(part);
    if constexpr (DT == LNSKV_DTYPE_Q8A) sc *= ksc;
    sc = __shfl(sc, 0);  // row 0's score, wave-uniform
    const float m_new = fmaxf(st.m[h], sc);
    const float alpha = fast_exp2(st.m[h] - m_new);
    const float p = fast_exp2(sc - m_new);
    st.m[h] = m_new;
    const float pv = (DT == LNSKV_DTYPE_Q8A) ? p * vsc : p;
    st.l[h] = alpha * st.l[h] + (row0 ? p : 0.0f);
#pragma unroll
    for (int e = 0; e < G::EPL; ++e) st.acc[h][e] = alpha * st.acc[h][e] + (row0 ? pv * vst[e] : 0.0f);
  }
}

template <int DT, int D, int REP, bool FUSED>
__global__ __launch_bounds__(kBlock) void decode_valu_kernel(DecodeArgs a) {
  using G = Geo<DT, D, REP>;
  __shared__ EpilogueLds<REP, D> sm;

  const int kvh = blockIdx.x, part = blockIdx.y, s = blockIdx.z;
  const SeqWindow w = seq_window<FUSED>(a, s);
  if (part >= w.nparts) return;  // block-uniform
  const int j = w.jf + part;
  const int tread_end = FUSED ? max(w.L - 1, 0) : w.L;  // newest token comes from registers
  const int ta = max(w.p0, j * a.split);
  const int tb = min(tread_end, (j + 1) * a.split);

  const int lane = threadIdx.x % kWave, wave = threadIdx.x / kWave;
  const int r = lane / G::LPR, c = lane % G::LPR;

  WaveState<DT, D, REP> st;
  const int h0 = kvh * REP;
#pragma unroll
  for (int h = 0; h < REP; ++h) {
    const float* qh = a.q + ((size_t)s * a.n_heads + h0 + h) * D + (size_t)c * G::EPL;
#pragma unroll
    for (int e = 0; e < G::EPL; ++e) {
      st.q[h][e] = qh[e] * a.scale_log2;
      st.acc[h][e] = 0.0f;
    }
    st.m[h] = kMInit;
    st.l[h] = 0.0f;
  }

  const uint32_t* bt_row = a.bt + (size_t)s * a.bt_stride;
  if (ta < tb) {
    const int pg_first = ta / kPage, pg_last = (tb - 1) / kPage;
    int pg = pg_first + wave;
    if (pg <= pg_last) {
      auto page_phys = [&](int p, bool& valid) {
        const uint32_t ph = bt_row[p];
        valid = ph < a.num_pages;
        return valid ? ph : 0u;  // in-bounds dummy for missing pages, fully masked
      };
      bool valid;
      uint32_t phys = page_phys(pg, valid);
      PageRegs<DT, D, REP> cur;
      load_page<DT, D, REP>(a, phys, kvh, r, c, cur);
      // The next page is loaded while this one is consumed, except at
      // head_dim 256 with 8 query heads on f32 or Q8A pages, where two pages
      // in flight beside the state (and the Q8A element conversions) exceed
      // the 512 registers and spilled; the block's other waves then cover
      // the load latency.
      constexpr bool kAhead = !(D == 256 && REP == 8 && DT != LNSKV_DTYPE_F16);
      for (; pg <= pg_last; pg += kWavesPerBlock) {
        const int nxt = pg + kWavesPerBlock;
        PageRegs<DT, D, REP> nx;
        bool nvalid = false;
        if (kAhead && nxt <= pg_last) {
          const uint32_t nphys = page_phys(nxt, nvalid);
          load_page<DT, D, REP>(a, nphys, kvh, r, c, nx);
        }
        const int tok0 = pg * kPage;
        const bool full = valid && tok0 >= ta && tok0 + kPage <= tb;
        consume_page<DT, D, REP>(st, cur, full, valid, tok0, ta, tb, r);
        if (!kAhead && nxt <= pg_last) {
          const uint32_t nphys = page_phys(nxt, nvalid);
          load_page<DT, D, REP>(a, nphys, kvh, r, c, nx);
        }
        cur = nx;
        valid = nvalid;
      }
    }
  }

  if constexpr (FUSED) {
    if (wave == 0 && w.L > 0 && part == w.nparts - 1) {
      const int pos = w.L - 1;
      fused_new_token<DT, D, REP>(a, st, s, kvh, pos, pos >= w.p0, lane);
    }
  }

  // Rows -> wave totals (every row holds the same m).
#pragma unroll
  for (int h = 0; h < REP; ++h) {
    st.l[h] = cross_sum<G::LPR>(st.l[h]);
#pragma unroll
    for (int e = 0; e < G::EPL; ++e) st.acc[h][e] = cross_sum<G::LPR>(st.acc[h][e]);
  }
  if (r == 0) {
#pragma unroll
    for (int h = 0; h < REP; ++h)
#pragma unroll
      for (int e = 0; e < G::EPL; ++e) sm.acc[wave][h][c * G::EPL + e] = st.acc[h][e];
  }
  if (lane == 0) {
#pragma unroll
    for (int h = 0; h < REP; ++h) {
      sm.m[wave][h] = st.m[h];
      sm.l[wave][h] = st.l[h];
    }
  }
  __syncthreads();
  finish_block<REP, D>(a, sm, w, s, kvh, part);
}

}  // namespace

template <int DT, int D, int REP, bool FUSED>
static void launch_t(const DecodeArgs& a, int n_seq, hipStream_t st) {
  const dim3 grid((unsigned)a.n_kv, (unsigned)a.max_parts, (unsigned)n_seq);
  decode_valu_kernel<DT, D, REP, FUSED><<<grid, kBlock, 0, st>>>(a);
  launch_combine<REP, D, FUSED>(a, n_seq, st);
}

template <int DT, int D, bool FUSED>
static int launch_rep(const DecodeArgs& a, int rep, int n_seq, hipStream_t st) {
  switch (rep) {
    case 1: launch_t<DT, D, 1, FUSED>(a, n_seq, st); break;
    case 2: launch_t<DT, D, 2, FUSED>(a, n_seq, st); break;
    case 4: launch_t<DT, D, 4, FUSED>(a, n_seq, st); break;
    case 8: launch_t<DT, D, 8, FUSED>(a, n_seq, st); break;
    default: return fail(LNSKV_ERR_UNSUPPORTED, "n_heads/n_kv_heads = %d not supported (1, 2, 4, 8)", rep);
  }
  return hip_check("decode kernel launch");
}

template <int DT, bool FUSED>
int launch_decode_valu(const DecodeArgs& a, int d, int rep, int n_seq, hipStream_t st) {
  switch (d) {
    case 64: return launch_rep<DT, 64, FUSED>(a, rep, n_seq, st);
    case 128: return launch_rep<DT, 128, FUSED>(a, rep, n_seq, st);
    case 256: return launch_rep<DT, 256, FUSED>(a, rep, n_seq, st);
    default: return fail(LNSKV_ERR_UNSUPPORTED, "head_dim %d", d);
  }
}

template int launch_decode_valu<LNSKV_DTYPE_F32, false>(const DecodeArgs&, int, int, int, hipStream_t);
template int launch_decode_valu<LNSKV_DTYPE_F32, true>(const DecodeArgs&, int, int, int, hipStream_t);
template int launch_decode_valu<LNSKV_DTYPE_F16, false>(const DecodeArgs&, int, int, int, hipStream_t);
template int launch_decode_valu<LNSKV_DTYPE_F16, true>(const DecodeArgs&, int, int, int, hipStream_t);
template int launch_decode_valu<LNSKV_DTYPE_Q8A, false>(const DecodeArgs&, int, int, int, hipStream_t);
template int launch_decode_valu<LNSKV_DTYPE_Q8A, true>(const DecodeArgs&, int, int, int, hipStream_t);

}  // namespace lnskv
