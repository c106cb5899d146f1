// Jeff (Qwen3.5) full attention on gfx950 matrix cores.
//
// Arithmetic follows cpu-kernels jeff_full_attention_into
// (crates/cpu-kernels/src/lib.rs:609-763): per head, centered RMSNorm of q and
// k with x * (scale * (1 + w)) (676-691), partial RoPE on channel pairs
// (i, i + rot/2) with angle t * theta^(-2i/rot) (692-709, table built on the
// host with the same f32 libm calls), keys with key > query or mask == 0 are
// dropped (716), s = (q.k)/sqrt(hd), softmax, o = sum p*v skipping p == 0 and
// o = 0 when nothing is kept (731-754), out = o * 1/(1 + exp(-gate)) (755-758).
//
// Layout: every (L, W) tensor is token-contiguous (element t + L*f), so a
// wavefront's 32 queries or a tile's 32 keys are one 128-byte run per
// feature.
//
// One workgroup = 4 wavefronts sharing one kv head. With G = heads/kv_heads
// query heads per kv head, a workgroup holds hg = gcd(G, 4) heads x (4/hg)
// query sub-tiles of 16, so each K/V tile staged in LDS is used by every
// query head of the group (native GQA). K is RMS-normalized and rotated while
// it is staged; Q is normalized and rotated once per wave into registers.
// Key tiles outside [first active key, last query] are never visited.
//
// Each wavefront owns 16 queries and walks 32-key tiles on the 16x16x4 f32
// MFMA: S^T = K Q^T as two 16-key blocks, then O^T += V^T P^T. At hd = 256
// this keeps Q (hd/4 registers) and O^T (hd/4) within one wave's registers.
#include "tfd_device.hpp"
#include "tfd_internal.hpp"

namespace tfd {

// x * (scale * (1 + w)) with the reference's rounding (no contraction).
__device__ __forceinline__ float rms_apply(float x, float scale, float w) {
#pragma clang fp contract(off)
  return x * (scale * (1.0f + w));
}

__device__ __forceinline__ float rope_lo(float a, float b, float c, float s) {
#pragma clang fp contract(off)
  return a * c - b * s;
}

__device__ __forceinline__ float rope_hi(float a, float b, float c, float s) {
#pragma clang fp contract(off)
  return a * s + b * c;
}

// 1 / sqrt(mean + eps) with mean = sumsq / hd, in the reference's order.
__device__ __forceinline__ float rms_scale(float sumsq, int hd, float eps) {
#pragma clang fp contract(off)
  const float mean = sumsq / (float)hd;
  return 1.0f / sqrtf(mean + eps);
}

// Scans one row's key mask: first and last active key (mask != 0).
__device__ __forceinline__ void scan_active(const float *maskr, int L, int tid, int lane,
                                            int *s_span) {
  int lo = 0x7fffffff, hi = -1;
  for (int k = tid; k < L; k += 256) {
    if (maskr[k] != 0.0f) {
      lo = min(lo, k);
      hi = max(hi, k);
    }
  }
  lo = wave_min(lo);
  hi = wave_max(hi);
  if (lane == 0) {
    atomicMin(&s_span[0], lo);
    atomicMax(&s_span[1], hi);
  }
}

template <int HDP>
__global__ __launch_bounds__(256, 2) void jeff_attention_f32_kernel(const JeffArgs a) {
  constexpr int QS = HDP / 4;   // Q registers per lane (4 lane groups split hd)
  constexpr int NB = HDP / 16;  // 16-row blocks of O^T
  constexpr int DP = HDP / 8;   // dims per staging thread (8 threads per key)
  constexpr int KS = HDP + 4;   // K and V stored [key][d]
  __shared__ __attribute__((aligned(16))) float Ks[kKeyTile * KS];
  __shared__ __attribute__((aligned(16))) float Vs[kKeyTile * KS];
  __shared__ float s_red[8 * kKeyTile];
  __shared__ float Ps[kWavesPerGroup * kKeyTile * kJeffWaveQueries];
  __shared__ int s_span[2];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int col = lane & 15, grp = lane >> 4;
  const int hg = a.heads_per_group, qsubs = kWavesPerGroup / hg;
  const int row = blockIdx.z;
  const int head = blockIdx.y * hg + wave % hg;
  const int kvh = min(head / a.groups, a.kv_heads - 1);
  const int L = a.L, hd = a.hd, rh = a.rot_half;
  const int QT = kJeffWaveQueries * qsubs;
  const int qa = blockIdx.x * QT;
  const int q = qa + (wave / hg) * kJeffWaveQueries + col;
  const bool qin = q < L;
  const float *maskr = a.mask + (size_t)row * L;
  const float *Q = static_cast<const float *>(a.q) + row * a.q_row + (size_t)head * hd * L;
  const float *Gt = static_cast<const float *>(a.gate) + row * a.q_row + (size_t)head * hd * L;
  const float *K = static_cast<const float *>(a.k) + row * a.kv_row + (size_t)kvh * hd * L;
  const float *V = static_cast<const float *>(a.v) + row * a.kv_row + (size_t)kvh * hd * L;
  float *OUT = a.out + row * a.q_row + (size_t)head * hd * L;
  const bool rope = a.cos_t != nullptr && rh > 0;

  // -------- active-key span; RoPE positions restart at `start` when trimming
  if (tid == 0) {
    s_span[0] = 0x7fffffff;
    s_span[1] = -1;
  }
  __syncthreads();
  scan_active(maskr, L, tid, lane, s_span);
  __syncthreads();
  const int first = s_span[0], last = s_span[1];
  const int start = (a.trim && last >= 0) ? first : 0;
  int kt_begin = 0, kt_end = 0;
  {
    const int kl = min(last, min(qa + QT, L) - 1);
    if (last >= 0 && first <= kl) {
      kt_begin = first / kKeyTile;
      kt_end = kl / kKeyTile + 1;
    }
  }

  // -------- Q: RMSNorm + partial RoPE into registers.
  // Lane (col, grp) holds Qn[q][grp*QS + s], the B operand of step s.
  float qreg[QS];
  const bool q_live = qin && q >= start;
  {
    float ss = 0.0f;
#pragma unroll
    for (int s = 0; s < QS; ++s) {
      const int d = grp * QS + s;
      const float x = (q_live && d < hd) ? Q[q + (size_t)L * d] : 0.0f;
      qreg[s] = x;
      ss += x * x;
    }
    ss += __shfl_xor(ss, 16);
    ss += __shfl_xor(ss, 32);
    const float scale = rms_scale(ss, hd, a.eps);
    const int pos = q_live ? q - start : 0;
#pragma unroll
    for (int s = 0; s < QS; ++s) {
      const int d = grp * QS + s;
      float y = 0.0f;
      if (q_live && d < hd) {
        y = rms_apply(qreg[s], scale, a.q_norm[d]);
        if (rope && d < 2 * rh) {
          const int p = d < rh ? d + rh : d - rh;
          const int i = d < rh ? d : d - rh;
          const float yp = rms_apply(Q[q + (size_t)L * p], scale, a.q_norm[p]);
          const float c = a.cos_t[(size_t)pos * rh + i], sn = a.sin_t[(size_t)pos * rh + i];
          y = d < rh ? rope_lo(y, yp, c, sn) : rope_hi(yp, y, c, sn);
        }
      }
      qreg[s] = y;
    }
  }

  f32x4 O[NB];
#pragma unroll
  for (int j = 0; j < NB; ++j)
#pragma unroll
    for (int r = 0; r < 4; ++r) O[j][r] = 0.0f;
  float m = -INFINITY, l = 0.0f;

  const int kk = tid & 31, part = tid >> 5;
  for (int kt = kt_begin; kt < kt_end; ++kt) {
    const int k0 = kt * kKeyTile;
    const int key = k0 + kk;
    const bool kin = key < L;
    // -------- stage in three light phases so little is live beside Q and O:
    // (1) raw K and V slices to LDS with partial sums of squares; V goes as
    // is, the MFMA product only runs on tiles whose V is all finite;
    // (2) RMSNorm of this thread's K slice in place; (3) RoPE on the pairs.
    float ss = 0.0f;
    int nonfinite = 0;
    {
      const float *kp = K + key;
      const float *vp = V + key;
#pragma unroll 4
      for (int i = 0; i < DP; ++i) {
        const int d = part * DP + i;
        float x = 0.0f, vv = 0.0f;
        if (kin && d < hd) {
          x = kp[(size_t)L * d];
          vv = vp[(size_t)L * d];
        }
        ss += x * x;
        nonfinite |= !__builtin_isfinite(vv);
        Ks[kk * KS + d] = x;
        Vs[kk * KS + d] = vv;
      }
    }
    s_red[part * kKeyTile + kk] = ss;
    __syncthreads();
    {
      float tot = 0.0f;
#pragma unroll
      for (int p = 0; p < 8; ++p) tot += s_red[p * kKeyTile + kk];
      const float scale = rms_scale(tot, hd, a.eps);
#pragma unroll 4
      for (int i = 0; i < DP; ++i) {
        const int d = part * DP + i;
        if (kin && d < hd) Ks[kk * KS + d] = rms_apply(Ks[kk * KS + d], scale, a.k_norm[d]);
      }
    }
    if (rope) {
      __syncthreads();
      for (int e = tid; e < kKeyTile * rh; e += 256) {
        const int k2 = e / rh, i = e - k2 * rh;
        const int pos = max(k0 + k2 - start, 0);
        if (k0 + k2 < L) {
          const float c = a.cos_t[(size_t)pos * rh + i], sn = a.sin_t[(size_t)pos * rh + i];
          const float x = Ks[k2 * KS + i], y = Ks[k2 * KS + i + rh];
          Ks[k2 * KS + i] = rope_lo(x, y, c, sn);
          Ks[k2 * KS + i + rh] = rope_hi(x, y, c, sn);
        }
      }
    }
    // -------- keep word: active key, key >= start, causal key <= query
    uint32_t w = 0u;
    {
      const int kc = k0 + (lane & 31);
      const bool act = kc < L && kc >= start && maskr[kc] != 0.0f;
      const uint32_t abits = (uint32_t)__ballot(act);
      if (q_live) w = abits & range_bits(0, q - k0);
    }
    const int nf = __syncthreads_or(nonfinite);

    if (__ballot(w != 0u) != 0) {
      f32x4 s0, s1;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        s0[r] = 0.0f;
        s1[r] = 0.0f;
      }
      // K operands are double-buffered one step ahead; the scheduling fences
      // keep the compiler from hoisting every LDS read (and its registers) to
      // the top of the loop.
      const f32x4 *k0row = reinterpret_cast<const f32x4 *>(&Ks[col * KS + grp * QS]);
      const f32x4 *k1row = reinterpret_cast<const f32x4 *>(&Ks[(16 + col) * KS + grp * QS]);
      f32x4 ka = k0row[0], kb = k1row[0];
#pragma unroll
      for (int c = 0; c < QS / 4; ++c) {
        f32x4 na = ka, nb = kb;
        if (c + 1 < QS / 4) {
          na = k0row[c + 1];
          nb = k1row[c + 1];
        }
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          s0 = mfma_16x16x4(ka[e], qreg[4 * c + e], s0);
          s1 = mfma_16x16x4(kb[e], qreg[4 * c + e], s1);
        }
        __builtin_amdgcn_sched_barrier(0);
        ka = na;
        kb = nb;
      }
      const float alpha = softmax_tile16(s0, s1, w, grp, a.c1, m, l);
      if (alpha != 1.0f) {
#pragma unroll
        for (int j = 0; j < NB; ++j) O[j] *= alpha;
      }
      if (!nf) {
        const float *v0 = &Vs[(4 * grp) * KS + col];
        const float *v1 = &Vs[(16 + 4 * grp) * KS + col];
        float va[4], vb[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          va[r] = v0[r * KS];
          vb[r] = v1[r * KS];
        }
#pragma unroll
        for (int j = 0; j < NB; ++j) {
          float na[4], nb[4];
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            na[r] = va[r];
            nb[r] = vb[r];
            if (j + 1 < NB) {
              na[r] = v0[r * KS + (j + 1) * 16];
              nb[r] = v1[r * KS + (j + 1) * 16];
            }
          }
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            O[j] = mfma_16x16x4(va[r], s0[r], O[j]);
            O[j] = mfma_16x16x4(vb[r], s1[r], O[j]);
          }
          __builtin_amdgcn_sched_barrier(0);
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            va[r] = na[r];
            vb[r] = nb[r];
          }
        }
      } else {
        // Non-finite value in the tile: accumulate key by key, skipping p == 0
        // (lib.rs:746-748), so masked NaN/inf values never leak. The wave's
        // probabilities go through its own LDS slice (wave-local, in order).
        float *pw = Ps + wave * (kKeyTile * kJeffWaveQueries);
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          pw[(4 * grp + r) * kJeffWaveQueries + col] = s0[r];
          pw[(16 + 4 * grp + r) * kJeffWaveQueries + col] = s1[r];
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma nounroll
        for (int kx = 0; kx < kKeyTile; ++kx) {
          const float p = pw[kx * kJeffWaveQueries + col];
          if (p == 0.0f) continue;
          const float *vrow = &Vs[kx * KS + 4 * grp];
#pragma unroll
          for (int j = 0; j < NB; ++j) {
#pragma unroll
            for (int r = 0; r < 4; ++r) O[j][r] += p * vrow[j * 16 + r];
            if ((j & 3) == 3) __builtin_amdgcn_sched_barrier(0);
          }
        }
      }
    }
    __syncthreads();
  }

  // -------- o / sum (0 when nothing was kept), sigmoid gate, store
  float lt = l + __shfl_xor(l, 16);
  lt += __shfl_xor(lt, 32);
  if (qin) {
    const bool dropped = a.trim && q < start;
#pragma unroll
    for (int j = 0; j < NB; ++j)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int d = j * 16 + 4 * grp + r;
        if (d < hd) {
          const size_t at = q + (size_t)L * d;
          const float o = lt > 0.0f ? O[j][r] / lt : 0.0f;
          const float g = Gt[at];
          const float sig = 1.0f / (1.0f + expf(-g));
          OUT[at] = dropped ? 0.0f : o * sig;
        }
      }
  }
}

// ----------------------------------------------------------------- launchers

template <int HDP>
static hipError_t launch_jeff_f32_hd(const JeffArgs &a, int rows, hipStream_t stream) {
  const int qsubs = kWavesPerGroup / a.heads_per_group;
  const int qt = kJeffWaveQueries * qsubs;
  dim3 grid((a.L + qt - 1) / qt, a.heads / a.heads_per_group, rows);
  hipLaunchKernelGGL((jeff_attention_f32_kernel<HDP>), grid, dim3(256), 0, stream, a);
  return hipGetLastError();
}

hipError_t launch_jeff_attention_f32(const JeffArgs &a, int rows, int hd_pad,
                                     hipStream_t stream) {
  switch (hd_pad) {
    case 32: return launch_jeff_f32_hd<32>(a, rows, stream);
    case 64: return launch_jeff_f32_hd<64>(a, rows, stream);
    case 128: return launch_jeff_f32_hd<128>(a, rows, stream);
    case 256: return launch_jeff_f32_hd<256>(a, rows, stream);
    default: return hipErrorInvalidValue;
  }
}

hipError_t launch_jeff_attention_bf16(const JeffArgs &, int, int, hipStream_t) {
  return hipErrorNotSupported;
}

}  // namespace tfd
