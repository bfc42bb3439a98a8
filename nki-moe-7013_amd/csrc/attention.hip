// GQA attention pieces for head_dim 128:
//
//  qkv_norm_rope  -- QKV projection on the MFMA tile engine with a 128-column
//                    tile = exactly one head, so the per-head RMSNorm and the
//                    RoPE pairs (i, i+64) are tile-local.  The fp32 tile goes
//                    through LDS; two threads per token row finish the head.
//                    K and V rows go straight into the contiguous cache.
//  attn_prefill   -- causal flash attention on MFMA.  Scores are computed
//                    transposed, S^T = K . Q^T, so each lane owns one query
//                    column: row max / row sum are lane-local plus one
//                    exchange with lane^32, and the probabilities already sit
//                    in the B-operand layout of O^T = V^T . P^T (the key order
//                    inside each 16-key MFMA step is permuted to match; V is
//                    stored transposed in LDS in that order).
//  attn_decode    -- split-KV flash decoding: a workgroup owns one (batch, kv
//                    head, 256-key split) and all q heads of that GQA group,
//                    so each K/V row is read from HBM once; a second kernel
//                    merges the splits.
#include "mfma_tile.hpp"

namespace qmoe {

constexpr int HD = 128;  // head_dim

// ====================================================================== QKV
__global__ __launch_bounds__(256) void qkv_norm_rope_kernel(
    const uint16_t* __restrict__ x, const uint16_t* __restrict__ wqkv,
    const uint16_t* __restrict__ qn_w, const uint16_t* __restrict__ kn_w,
    const float* __restrict__ rope_cos, const float* __restrict__ rope_sin,
    const int32_t* __restrict__ positions, int T, int S, int H, int Hq, int Hkv, int S_max,
    int max_pos, float eps, uint16_t* __restrict__ q_out, uint16_t* __restrict__ k_cache,
    uint16_t* __restrict__ v_cache) {
  __shared__ __attribute__((aligned(16))) uint16_t smem[tile::SMEM_BYTES / 2];
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const int head = blockIdx.x;  // 0..Hq+2Hkv-1
  const int m0 = blockIdx.y * tile::BM;
  const int n0 = head * HD;
  const int kc = (t & 7) * 8;
  const uint16_t* ap[4];
  const uint16_t* bp[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int r = tile::stage_row(t, j);
    ap[j] = (m0 + r < T) ? x + int64_t(m0 + r) * H + kc : nullptr;
    bp[j] = wqkv + int64_t(n0 + r) * H + kc;
  }
  tile::Acc acc;
  tile::mma_128x128(ap, bp, H, smem, acc);  // ends with a barrier

  constexpr int LDC = HD + 4;
  float* ct = reinterpret_cast<float*>(smem);  // [128][LDC] fp32 (66 KB)
#pragma unroll
  for (int mi = 0; mi < 2; ++mi)
#pragma unroll
    for (int ni = 0; ni < 2; ++ni) {
      const int col = tile::acc_col(wave, lane, ni);
#pragma unroll
      for (int i = 0; i < 16; ++i) ct[tile::acc_row(wave, lane, mi, i) * LDC + col] = acc.c[mi][ni][i];
    }
  __syncthreads();

  const int row = t >> 1, half = t & 1;
  const int tok = m0 + row;
  // thread owns elements [32h, 32h+32) and their RoPE partners +64
  float lo[32], hi[32];
#pragma unroll
  for (int i = 0; i < 32; ++i) {
    lo[i] = ct[row * LDC + half * 32 + i];
    hi[i] = ct[row * LDC + 64 + half * 32 + i];
  }
  if (tok >= T) return;
  const int pos = positions[tok];
  if (pos < 0 || pos >= S_max || pos >= max_pos) return;  // rejected: nothing written
  const int b = tok / S;
  uint16_t* dst;
  if (head < Hq + Hkv) {
    const uint16_t* nw = head < Hq ? qn_w : kn_w;
    float ss = 0.0f;
#pragma unroll
    for (int i = 0; i < 32; ++i) ss += lo[i] * lo[i] + hi[i] * hi[i];
    ss += __shfl_xor(ss, 1, 64);
    const float r = rsqrtf(ss / float(HD) + eps);
    const float* cs = rope_cos + int64_t(pos) * (HD / 2) + half * 32;
    const float* sn = rope_sin + int64_t(pos) * (HD / 2) + half * 32;
#pragma unroll
    for (int i = 0; i < 32; ++i) {
      const float a = bf16_to_f32(nw[half * 32 + i]) * (lo[i] * r);
      const float bb = bf16_to_f32(nw[64 + half * 32 + i]) * (hi[i] * r);
      const float c = cs[i], s = sn[i];
      lo[i] = a * c - bb * s;
      hi[i] = bb * c + a * s;
    }
    if (head < Hq)
      dst = q_out + (int64_t(tok) * Hq + head) * HD;
    else
      dst = k_cache + ((int64_t(b) * Hkv + (head - Hq)) * S_max + pos) * HD;
  } else {
    dst = v_cache + ((int64_t(b) * Hkv + (head - Hq - Hkv)) * S_max + pos) * HD;
  }
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    u32x4 v0, v1;
    v0.x = pack_bf16x2(lo[c * 8 + 0], lo[c * 8 + 1]);
    v0.y = pack_bf16x2(lo[c * 8 + 2], lo[c * 8 + 3]);
    v0.z = pack_bf16x2(lo[c * 8 + 4], lo[c * 8 + 5]);
    v0.w = pack_bf16x2(lo[c * 8 + 6], lo[c * 8 + 7]);
    v1.x = pack_bf16x2(hi[c * 8 + 0], hi[c * 8 + 1]);
    v1.y = pack_bf16x2(hi[c * 8 + 2], hi[c * 8 + 3]);
    v1.z = pack_bf16x2(hi[c * 8 + 4], hi[c * 8 + 5]);
    v1.w = pack_bf16x2(hi[c * 8 + 6], hi[c * 8 + 7]);
    *reinterpret_cast<u32x4*>(dst + half * 32 + c * 8) = v0;
    *reinterpret_cast<u32x4*>(dst + 64 + half * 32 + c * 8) = v1;
  }
}

// ====================================================================== prefill
constexpr int AP_QT = 128;      // query rows per workgroup (4 waves x 32)
constexpr int AP_KT = 64;       // keys per step
constexpr int AP_LDK = HD + 8;  // K tile row stride (bf16)
constexpr int AP_LDV = AP_KT + 8;

// position of key r (0..63) inside the permuted, transposed V tile row
__device__ __forceinline__ int vt_slot(int key) {
  const int s = key >> 4, r = key & 15;
  const int h = (r >> 2) & 1, jj = (r >> 3) * 4 + (r & 3);
  return s * 16 + h * 8 + jj;
}

__global__ __launch_bounds__(256) void attn_prefill_kernel(
    const uint16_t* __restrict__ q, const uint16_t* __restrict__ k_cache,
    const uint16_t* __restrict__ v_cache, int S, int Hq, int Hkv, int S_max, int start,
    float scale_log2, uint16_t* __restrict__ out) {
  __shared__ __attribute__((aligned(16))) uint16_t Ks[AP_KT * AP_LDK];
  __shared__ __attribute__((aligned(16))) uint16_t Vt[HD * AP_LDV];
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const int qt = gridDim.x - 1 - blockIdx.x;  // heavy (late) query tiles first
  const int h = blockIdx.y, b = blockIdx.z;
  const int kvh = h / (Hq / Hkv);
  const int q0 = qt * AP_QT;
  const int qrow = q0 + wave * 32 + (lane & 31);  // this lane's query (column of S^T)
  const int hl = lane >> 5;
  const int64_t kv_base = (int64_t(b) * Hkv + kvh) * S_max * HD;

  // Q fragments (B operand of S^T = K Q^T): d = ks*16 + hl*8 + [0,8)
  bf16x8 qf[HD / 16];
  {
    const bool ok = qrow < S;
    const uint16_t* qp = q + ((int64_t(b) * S + (ok ? qrow : 0)) * Hq + h) * HD + hl * 8;
#pragma unroll
    for (int ks = 0; ks < HD / 16; ++ks) {
      u32x4 v = ok ? ld16(qp + ks * 16) : u32x4{0u, 0u, 0u, 0u};
      qf[ks] = *reinterpret_cast<bf16x8*>(&v);
    }
  }
  f32x16 o[4];
#pragma unroll
  for (int db = 0; db < 4; ++db)
#pragma unroll
    for (int i = 0; i < 16; ++i) o[db][i] = 0.0f;
  float m_run = -INFINITY, l_run = 0.0f;
  const int q_idx = start + qrow;               // cache index of this query
  const int kv_end = start + min(q0 + AP_QT, S);  // keys [0, kv_end) can be visible
  const int n_kt = (kv_end + AP_KT - 1) / AP_KT;

  for (int kt = 0; kt < n_kt; ++kt) {
    const int kv0 = kt * AP_KT;
    __syncthreads();
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int c = t + 256 * j;
      const int key = c >> 4, dc = (c & 15) * 8;
      const bool ok = kv0 + key < kv_end;
      const int64_t off = kv_base + int64_t(kv0 + key) * HD + dc;
      const u32x4 kv = ok ? ld16(k_cache + off) : u32x4{0u, 0u, 0u, 0u};
      const u32x4 vv = ok ? ld16(v_cache + off) : u32x4{0u, 0u, 0u, 0u};
      *reinterpret_cast<u32x4*>(Ks + key * AP_LDK + dc) = kv;
      const int vs = vt_slot(key);
      const uint32_t w4[4] = {vv.x, vv.y, vv.z, vv.w};
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        Vt[(dc + 2 * u) * AP_LDV + vs] = uint16_t(w4[u] & 0xffffu);
        Vt[(dc + 2 * u + 1) * AP_LDV + vs] = uint16_t(w4[u] >> 16);
      }
    }
    __syncthreads();
    // S^T blocks: keys [0,32) and [32,64) x this wave's 32 queries
    f32x16 st[2];
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
#pragma unroll
      for (int i = 0; i < 16; ++i) st[kb][i] = 0.0f;
      const uint16_t* kp = Ks + (kb * 32 + (lane & 31)) * AP_LDK + hl * 8;
#pragma unroll
      for (int ks = 0; ks < HD / 16; ++ks) {
        const bf16x8 a = *reinterpret_cast<const bf16x8*>(kp + ks * 16);
        st[kb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, qf[ks], st[kb], 0, 0, 0);
      }
    }
    // scale (log2 domain), causal mask, online softmax
    float mloc = -INFINITY;
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int key = kv0 + kb * 32 + (i >> 2) * 8 + hl * 4 + (i & 3);
        float s = st[kb][i] * scale_log2;
        if (key > q_idx || key >= kv_end) s = -INFINITY;
        st[kb][i] = s;
        mloc = fmaxf(mloc, s);
      }
    mloc = fmaxf(mloc, __shfl_xor(mloc, 32, 64));
    const float m_new = fmaxf(m_run, mloc);
    const float alpha = (m_new == -INFINITY) ? 1.0f : exp2f(m_run - m_new);
    float lsum = 0.0f;
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const float p = (m_new == -INFINITY) ? 0.0f : exp2f(st[kb][i] - m_new);
        st[kb][i] = p;
        lsum += p;
      }
    lsum += __shfl_xor(lsum, 32, 64);
    l_run = l_run * alpha + lsum;
    m_run = m_new;
#pragma unroll
    for (int db = 0; db < 4; ++db)
#pragma unroll
      for (int i = 0; i < 16; ++i) o[db][i] *= alpha;
    // O^T += V^T P^T over 4 steps of 16 keys
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      bf16x8 pb;
#pragma unroll
      for (int jj = 0; jj < 8; ++jj) pb[jj] = static_cast<__bf16>(st[s >> 1][(s & 1) * 8 + jj]);
#pragma unroll
      for (int db = 0; db < 4; ++db) {
        const bf16x8 a =
            *reinterpret_cast<const bf16x8*>(Vt + (db * 32 + (lane & 31)) * AP_LDV + s * 16 + hl * 8);
        o[db] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, pb, o[db], 0, 0, 0);
      }
    }
  }
  if (qrow >= S) return;
  const float inv = 1.0f / l_run;
  uint16_t* op = out + ((int64_t(b) * S + qrow) * Hq + h) * HD;
#pragma unroll
  for (int db = 0; db < 4; ++db)
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const int d = db * 32 + g * 8 + hl * 4;
      u32x2 v;
      v.x = pack_bf16x2(o[db][g * 4 + 0] * inv, o[db][g * 4 + 1] * inv);
      v.y = pack_bf16x2(o[db][g * 4 + 2] * inv, o[db][g * 4 + 3] * inv);
      *reinterpret_cast<u32x2*>(op + d) = v;
    }
}

// ====================================================================== decode
constexpr int AD_SPLIT = 256;  // keys per workgroup
constexpr int AD_MAX_G = 16;   // q heads per kv head

__global__ __launch_bounds__(256) void attn_decode_split_kernel(
    const uint16_t* __restrict__ q, const uint16_t* __restrict__ k_cache,
    const uint16_t* __restrict__ v_cache, const int32_t* __restrict__ ctx_len, int Hq, int Hkv,
    int S_max, int nsplit, float scale, float* __restrict__ partial) {
  __shared__ float qs[AD_MAX_G][HD];
  __shared__ float ps[AD_MAX_G][AD_SPLIT];
  __shared__ float red[AD_MAX_G][4];
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const int split = blockIdx.x, kvh = blockIdx.y, b = blockIdx.z;
  const int G = Hq / Hkv;
  const int ctx = min(ctx_len[b], S_max);
  const int k0 = split * AD_SPLIT;
  const int nk = min(AD_SPLIT, ctx - k0);
  float* pout = partial + ((int64_t(b) * Hq + kvh * G) * nsplit + split) * (HD + 2);
  // partial layout per (b, q head, split): [m, l, o[0..127]]
  if (nk <= 0) {
    for (int i = t; i < G * (HD + 2); i += 256) {
      const int g = i / (HD + 2), r = i - g * (HD + 2);
      pout[int64_t(g) * nsplit * (HD + 2) + r] = (r == 0) ? -INFINITY : 0.0f;
    }
    return;
  }
  for (int i = t; i < G * HD; i += 256) {
    const int g = i / HD, d = i - g * HD;
    qs[g][d] = bf16_to_f32(q[(int64_t(b) * Hq + kvh * G + g) * HD + d]);
  }
  __syncthreads();
  const int64_t kv_base = (int64_t(b) * Hkv + kvh) * S_max * HD;
  // scores: thread t owns key k0 + t
  float sc[AD_MAX_G];
#pragma unroll
  for (int g = 0; g < AD_MAX_G; ++g) sc[g] = 0.0f;
  if (t < nk) {
    const uint16_t* kp = k_cache + kv_base + int64_t(k0 + t) * HD;
#pragma unroll
    for (int c = 0; c < HD / 8; ++c) {
      const u32x4 kv = ld16(kp + c * 8);
      const float k8[8] = {bf16_lo(kv.x), bf16_hi(kv.x), bf16_lo(kv.y), bf16_hi(kv.y),
                           bf16_lo(kv.z), bf16_hi(kv.z), bf16_lo(kv.w), bf16_hi(kv.w)};
#pragma unroll
      for (int g = 0; g < AD_MAX_G; ++g) {
        if (g < G) {
#pragma unroll
          for (int u = 0; u < 8; ++u) sc[g] = fmaf(k8[u], qs[g][c * 8 + u], sc[g]);
        }
      }
    }
  }
  // max per head
#pragma unroll
  for (int g = 0; g < AD_MAX_G; ++g) {
    if (g < G) {
      const float s = (t < nk) ? sc[g] * scale : -INFINITY;
      sc[g] = s;
      const float m = wave_max(s);
      if (lane == 0) red[g][wave] = m;
    }
  }
  __syncthreads();
  float mg[AD_MAX_G];
#pragma unroll
  for (int g = 0; g < AD_MAX_G; ++g)
    mg[g] = (g < G) ? fmaxf(fmaxf(red[g][0], red[g][1]), fmaxf(red[g][2], red[g][3])) : 0.0f;
  __syncthreads();
#pragma unroll
  for (int g = 0; g < AD_MAX_G; ++g) {
    if (g < G) {
      const float p = (t < nk) ? __expf(sc[g] - mg[g]) : 0.0f;
      ps[g][t] = p;
      const float l = wave_sum(p);
      if (lane == 0) red[g][wave] = l;
    }
  }
  __syncthreads();
  // O[g][d] = sum_k p[g][k] V[k][d]; thread: d pair (t % 64) * 2, heads g = t/64 + 4*jg
  const int d2 = (t & 63) * 2;
  float oa[AD_MAX_G / 4][2];
#pragma unroll
  for (int jg = 0; jg < AD_MAX_G / 4; ++jg) oa[jg][0] = oa[jg][1] = 0.0f;
  const uint16_t* vp = v_cache + kv_base + int64_t(k0) * HD + d2;
  for (int kk = 0; kk < nk; ++kk) {
    const uint32_t vv = *reinterpret_cast<const uint32_t*>(vp + int64_t(kk) * HD);
    const float v0 = bf16_lo(vv), v1 = bf16_hi(vv);
#pragma unroll
    for (int jg = 0; jg < AD_MAX_G / 4; ++jg) {
      const int g = wave + 4 * jg;
      if (g < G) {
        const float p = ps[g][kk];
        oa[jg][0] = fmaf(p, v0, oa[jg][0]);
        oa[jg][1] = fmaf(p, v1, oa[jg][1]);
      }
    }
  }
#pragma unroll
  for (int jg = 0; jg < AD_MAX_G / 4; ++jg) {
    const int g = wave + 4 * jg;
    if (g < G) {
      float* pg = pout + int64_t(g) * nsplit * (HD + 2);
      if ((t & 63) == 0) {
        pg[0] = mg[g];
        pg[1] = red[g][0] + red[g][1] + red[g][2] + red[g][3];
      }
      pg[2 + d2] = oa[jg][0];
      pg[2 + d2 + 1] = oa[jg][1];
    }
  }
}

__global__ __launch_bounds__(HD) void attn_decode_merge_kernel(const float* __restrict__ partial,
                                                               int nsplit,
                                                               uint16_t* __restrict__ out) {
  const int bh = blockIdx.x;  // b * Hq + h
  const int d = threadIdx.x;
  const float* p = partial + int64_t(bh) * nsplit * (HD + 2);
  float M = -INFINITY;
  for (int s = 0; s < nsplit; ++s) M = fmaxf(M, p[int64_t(s) * (HD + 2)]);
  float L = 0.0f, O = 0.0f;
  for (int s = 0; s < nsplit; ++s) {
    const float* ps = p + int64_t(s) * (HD + 2);
    const float m = ps[0];
    if (m == -INFINITY) continue;
    const float w = __expf(m - M);
    L += ps[1] * w;
    O += ps[2 + d] * w;
  }
  out[int64_t(bh) * HD + d] = f32_to_bf16(O / L);
}

}  // namespace qmoe

using namespace qmoe;

extern "C" int qmoe_qkv_norm_rope(const qmoe_bf16* x, const qmoe_bf16* wqkv,
                                  const qmoe_bf16* q_norm_w, const qmoe_bf16* k_norm_w,
                                  const float* rope_cos, const float* rope_sin, int64_t max_pos,
                                  const int32_t* positions, int64_t B, int64_t S, int64_t H,
                                  int64_t Hq, int64_t Hkv, int64_t D, int64_t S_max, float eps,
                                  qmoe_bf16* q_out, qmoe_bf16* k_cache, qmoe_bf16* v_cache,
                                  qmoe_stream_t stream) {
  QMOE_REQUIRE(x && wqkv && q_norm_w && k_norm_w && rope_cos && rope_sin && positions && q_out &&
                   k_cache && v_cache,
               "qmoe_qkv_norm_rope: null pointer");
  QMOE_REQUIRE(D == HD, "qmoe_qkv_norm_rope: head_dim must be 128 (D=%lld)", (long long)D);
  QMOE_REQUIRE(H > 0 && H % 64 == 0, "qmoe_qkv_norm_rope: H %% 64 != 0");
  QMOE_REQUIRE(Hq > 0 && Hkv > 0 && Hq % Hkv == 0 && Hq + 2 * Hkv < 65536,
               "qmoe_qkv_norm_rope: bad head counts");
  QMOE_REQUIRE(B >= 0 && S >= 0 && B * S < (1ll << 31), "qmoe_qkv_norm_rope: bad B/S");
  QMOE_REQUIRE(S_max > 0 && max_pos > 0, "qmoe_qkv_norm_rope: bad S_max/max_pos");
  const int64_t T = B * S;
  if (T == 0) return QMOE_OK;
  dim3 grid(unsigned(Hq + 2 * Hkv), unsigned((T + tile::BM - 1) / tile::BM));
  hipLaunchKernelGGL(qkv_norm_rope_kernel, grid, dim3(256), 0, as_stream(stream), x, wqkv, q_norm_w,
                     k_norm_w, rope_cos, rope_sin, positions, int(T), int(S), int(H), int(Hq),
                     int(Hkv), int(S_max), int(std::min<int64_t>(max_pos, 1ll << 30)), eps, q_out,
                     k_cache, v_cache);
  return hip_status("qmoe_qkv_norm_rope");
}

extern "C" int qmoe_attn_prefill(const qmoe_bf16* q, const qmoe_bf16* k_cache,
                                 const qmoe_bf16* v_cache, int64_t B, int64_t S, int64_t Hq,
                                 int64_t Hkv, int64_t D, int64_t S_max, int64_t start, float scale,
                                 qmoe_bf16* out, qmoe_stream_t stream) {
  QMOE_REQUIRE(q && k_cache && v_cache && out, "qmoe_attn_prefill: null pointer");
  QMOE_REQUIRE(D == HD, "qmoe_attn_prefill: head_dim must be 128");
  QMOE_REQUIRE(Hq > 0 && Hkv > 0 && Hq % Hkv == 0 && Hq < 65536, "qmoe_attn_prefill: bad heads");
  QMOE_REQUIRE(B >= 0 && B < 65536 && S >= 0 && start >= 0 && start + S <= S_max,
               "qmoe_attn_prefill: need 0 <= start and start + S <= S_max");
  if (B == 0 || S == 0) return QMOE_OK;
  dim3 grid(unsigned((S + AP_QT - 1) / AP_QT), unsigned(Hq), unsigned(B));
  const float scale_log2 = scale * 1.4426950408889634f;
  hipLaunchKernelGGL(attn_prefill_kernel, grid, dim3(256), 0, as_stream(stream), q, k_cache, v_cache,
                     int(S), int(Hq), int(Hkv), int(S_max), int(start), scale_log2, out);
  return hip_status("qmoe_attn_prefill");
}

extern "C" int64_t qmoe_attn_decode_workspace(int64_t B, int64_t Hq, int64_t D, int64_t S_max) {
  const int64_t nsplit = (S_max + AD_SPLIT - 1) / AD_SPLIT;
  return B * Hq * nsplit * (D + 2);
}

extern "C" int qmoe_attn_decode(const qmoe_bf16* q, const qmoe_bf16* k_cache,
                                const qmoe_bf16* v_cache, const int32_t* ctx_len, int64_t B,
                                int64_t Hq, int64_t Hkv, int64_t D, int64_t S_max, float scale,
                                float* partial, qmoe_bf16* out, qmoe_stream_t stream) {
  QMOE_REQUIRE(q && k_cache && v_cache && ctx_len && partial && out, "qmoe_attn_decode: null pointer");
  QMOE_REQUIRE(D == HD, "qmoe_attn_decode: head_dim must be 128");
  QMOE_REQUIRE(Hq > 0 && Hkv > 0 && Hq % Hkv == 0 && Hq / Hkv <= AD_MAX_G && Hkv < 65536,
               "qmoe_attn_decode: need Hq %% Hkv == 0 and Hq / Hkv <= 16");
  QMOE_REQUIRE(B >= 0 && B < 65536 && S_max > 0, "qmoe_attn_decode: bad B/S_max");
  if (B == 0) return QMOE_OK;
  const int nsplit = int((S_max + AD_SPLIT - 1) / AD_SPLIT);
  hipStream_t s = as_stream(stream);
  hipLaunchKernelGGL(attn_decode_split_kernel, dim3(unsigned(nsplit), unsigned(Hkv), unsigned(B)),
                     dim3(256), 0, s, q, k_cache, v_cache, ctx_len, int(Hq), int(Hkv), int(S_max),
                     nsplit, scale, partial);
  int rc = hip_status("qmoe_attn_decode(split)");
  if (rc) return rc;
  hipLaunchKernelGGL(attn_decode_merge_kernel, dim3(unsigned(B * Hq)), dim3(HD), 0, s, partial, nsplit,
                     out);
  return hip_status("qmoe_attn_decode(merge)");
}
