// reforder.hip — the decode step in the reference's floating-point order.
//
// The fast kernels (matvec.hip, attn_decode.hip) sum across lanes and
// chunks, so their fp32 sums round in another order than the reference's
// left-to-right loops.  On deep models the reference re-quantizes every
// matmul input to Q8_0, and an ulp moved anywhere moves an activation code
// now and then and cascades, so those kernels sit at the reference builds'
// own noise floor.  With EHIP_ORDER=reference a state runs these kernels
// instead: every fp32 operation is the reference's, in its order, and expf
// is its libm's, so the step reproduces the reference's deterministic build
// bit for bit.  They are slow by construction (sequential sums over
// thousands of terms) and serve parity, not speed.
//
//   k_matvec_ref   one thread per output: rmsnorm (model.c:50-55) with one
//                  thread summing the squares in order, Q8_0 quantization
//                  (kernels.c:73-92), then per output the block sums of
//                  vecdot_q8 / vecdot_q4 / dot_f32 (kernels.c:120-182)
//                  added block after block, and the bias / residual /
//                  SwiGLU epilogues of ember_forward (model.c:382-408)
//   k_attn_ref     one workgroup per query head: the head's QK-norm
//                  (model.c:386-389), RoPE (model.c:66-80), the cache store
//                  (model.c:39-48) and attn_heads + softmax (model.c:57-64,
//                  207-278): scores summed over the head dims in order, the
//                  softmax sum and every output dim summed over positions in
//                  order
#include "kernels.h"
#include "libm_expf.h"

namespace ehip {

// expf: the reference's libm's (libm_expf.h)
__device__ __forceinline__ float ref_expf(float x) { return libm_expf(x); }

template <int DT, int PRO, int EPI>
__global__ __launch_bounds__(WG) void k_matvec_ref(MatvecArgs a) {
    extern __shared__ __align__(16) uint8_t smem[];
    __shared__ float sscale;
    __shared__ float am_v[NWAVE];
    __shared__ int am_i[NWAVE];
    const int K = a.W.cols, nb = K / QB;
    float *xs = reinterpret_cast<float *>(smem);              // [K] the activation (normed)
    float *dxs = xs + K;                                       // [nb] fp16-rounded block scales
    int8_t *qx = reinterpret_cast<int8_t *>(dxs + nb);         // [K] codes
    const int tid = threadIdx.x;

    for (int i = tid; i < K; i += WG) {
        float v;
        if (PRO == PRO_EMBED_NORM) {   // embed_row / dequant_q8_row (model.c:83-100)
            const int tok = a.tokpos[0];
            if (a.emb.dtype == DT_F32) {
                v = reinterpret_cast<const float *>(a.emb.q)[(size_t)tok * K + i];
            } else {
                v = (float)reinterpret_cast<const int8_t *>(a.emb.q)[(size_t)tok * K + i] *
                    h2f(a.emb.d[(size_t)tok * nb + i / QB]);
            }
            if (blockIdx.x == 0) a.x_out[i] = v;
        } else {
            v = a.in[i];
        }
        xs[i] = v;
    }
    __syncthreads();
    if (PRO != PRO_PLAIN) {   // rmsnorm, the squares summed in order by one thread
        if (tid == 0) {
            float ss = 0.0f;
            for (int i = 0; i < K; i++) ss += xs[i] * xs[i];
            sscale = 1.0f / sqrtf(ss / (float)K + a.eps);
        }
        __syncthreads();
        const float scale = sscale;
        for (int i = tid; i < K; i += WG) xs[i] = xs[i] * scale * a.norm_w[i];
        __syncthreads();
    }
    if (DT != DT_F32) {   // ember_quantize_q8_0, one thread per block
        for (int bk = tid; bk < nb; bk += WG) {
            const float *xb = xs + bk * QB;
            float amax = 0.0f;
            for (int i = 0; i < QB; i++) {
                const float v = fabsf(xb[i]);
                if (v > amax) amax = v;
            }
            const float d = amax / 127.0f;
            const float id = d > 0.0f ? 1.0f / d : 0.0f;
            for (int i = 0; i < QB; i++) {
                int q = (int)roundf(xb[i] * id);
                if (q > 127) q = 127;
                if (q < -127) q = -127;
                qx[bk * QB + i] = (int8_t)q;
            }
            dxs[bk] = h2f(f2h(d));
        }
        __syncthreads();
    }

    constexpr int NR = EPI == EPI_SWIGLU ? 2 : 1;
    const int u = blockIdx.x * WG + tid;
    float best_v = -INFINITY;
    int best_i = 0x7fffffff;
    if (u < a.units) {
        float r[NR];
#pragma unroll
        for (int k = 0; k < NR; k++) {
            const size_t row = (size_t)u + (size_t)k * a.pair_off;
            float sum = 0.0f;
            if (DT == DT_F32) {   // dot_f32, products added in order
                const float *w = reinterpret_cast<const float *>(a.W.q) + row * K;
                for (int i = 0; i < K; i++) sum += w[i] * xs[i];
            } else {
                const uint16_t *dw = a.W.d + row * nb;
                for (int bk = 0; bk < nb; bk++) {
                    int acc = 0;
                    const int *xq = reinterpret_cast<const int *>(qx + bk * QB);
                    if (DT == DT_Q8) {
                        const int *w = reinterpret_cast<const int *>(a.W.q + row * K + (size_t)bk * QB);
#pragma unroll
                        for (int j = 0; j < QB / 4; j++) acc = sdot4(w[j], xq[j], acc);
                    } else {   // byte i: weight i (low nibble), weight i + 16 (high nibble), both - 8
                        const uint8_t *w = a.W.q + row * (K / 2) + (size_t)bk * (QB / 2);
                        const int8_t *xb = qx + bk * QB;
                        for (int i = 0; i < QB / 2; i++)
                            acc += ((int)(w[i] & 0x0f) - 8) * (int)xb[i] + ((int)(w[i] >> 4) - 8) * (int)xb[i + QB / 2];
                    }
                    sum += (float)acc * h2f(dw[bk]) * dxs[bk];
                }
            }
            r[k] = sum;
        }
        float o;
        if (EPI == EPI_STORE) {
            o = a.bias ? r[0] + a.bias[u] : r[0];
        } else if (EPI == EPI_RESID) {
            o = a.out[u] + r[0];
        } else {
            const float g = r[0];
            o = g / (1.0f + ref_expf(-g)) * r[NR - 1];
        }
        a.out[u] = o;
        best_v = o;
        best_i = u;
    }
    if (EPI != EPI_STORE || !a.am_val) return;
    // this workgroup's first maximum (the argmax merge takes the first over workgroups)
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
        const float v2 = __shfl_xor(best_v, off);
        const int i2 = __shfl_xor(best_i, off);
        if (v2 > best_v || (v2 == best_v && i2 < best_i)) { best_v = v2; best_i = i2; }
    }
    const int w = tid >> 6;
    if ((tid & 63) == 0) { am_v[w] = best_v; am_i[w] = best_i; }
    __syncthreads();
    if (tid == 0) {
        float v = am_v[0];
        int i = am_i[0];
        for (int k = 1; k < NWAVE; k++)
            if (am_v[k] > v || (am_v[k] == v && am_i[k] < i)) { v = am_v[k]; i = am_i[k]; }
        a.am_val[blockIdx.x] = v;
        a.am_idx[blockIdx.x] = i;
    }
}

template <int DT, int PRO, int EPI>
static int ref_go(hipStream_t st, const MatvecArgs &a) {
    const int K = a.W.cols;
    const size_t lds = (size_t)K * 4 + (size_t)(K / QB) * 4 + (size_t)K;
    if (lds > 64 * 1024) return -1;
    const int grid = (a.units + WG - 1) / WG;
    if (a.am_val && grid > MATVEC_MAX_GRID) return -1;
    hipLaunchKernelGGL((k_matvec_ref<DT, PRO, EPI>), dim3(grid), dim3(WG), lds, st, a);
    return grid;
}

template <int PRO, int EPI>
static int ref_dt(hipStream_t st, const MatvecArgs &a) {
    switch (a.W.dtype) {
        case DT_Q8: return ref_go<DT_Q8, PRO, EPI>(st, a);
        case DT_Q4: return ref_go<DT_Q4, PRO, EPI>(st, a);
        case DT_F32: return ref_go<DT_F32, PRO, EPI>(st, a);
    }
    return -1;
}

int launch_matvec_ref(hipStream_t st, int pro, int epi, const MatvecArgs &a) {
    const int K = a.W.cols;
    if (K % QB != 0 || K <= 0 || a.units <= 0) return -1;
    if (a.am_val && epi != EPI_STORE) return -1;
    int grid = -1;
    if (pro == PRO_NORM && epi == EPI_STORE) grid = ref_dt<PRO_NORM, EPI_STORE>(st, a);
    else if (pro == PRO_EMBED_NORM && epi == EPI_STORE) grid = ref_dt<PRO_EMBED_NORM, EPI_STORE>(st, a);
    else if (pro == PRO_NORM && epi == EPI_SWIGLU) grid = ref_dt<PRO_NORM, EPI_SWIGLU>(st, a);
    else if (pro == PRO_PLAIN && epi == EPI_RESID) grid = ref_dt<PRO_PLAIN, EPI_RESID>(st, a);
    if (grid <= 0) return -1;
    if (a.am_val) return launch_argmax_merge(st, a.am_val, a.am_idx, grid, a.units, a.am_tokpos, a.am_out, a.am_cap);
    return 0;
}

// One workgroup per query head h (kv head g = h / (n_heads / n_kv)).  The
// token's raw q|k|v row is a.q; att is [n_heads][ctx] scratch.  The first
// query head of each kv group writes the cache row at pos; every workgroup
// attends to its own copy of that row for t = pos (the same values).
template <bool F16>
__global__ __launch_bounds__(WG) void k_attn_ref(AttnArgs a, float *att_all) {
    __shared__ float qv[256], kn[256], vn[256];
    __shared__ float red[NWAVE], sh[2];
    const int tid = threadIdx.x, h = blockIdx.x, HD = a.hd;
    const int G = a.n_heads / a.n_kv, g = h / G;
    const int qd = a.n_heads * HD;
    const int pos = a.tokpos[1];
    float *att = att_all + (size_t)h * a.ctx;
    for (int i = tid; i < HD; i += WG) {
        qv[i] = a.q[(size_t)h * HD + i];
        kn[i] = a.q[qd + (size_t)g * HD + i];
        vn[i] = a.q[qd + a.kv_dim + (size_t)g * HD + i];
    }
    __syncthreads();
    if (a.q_norm) {   // rmsnorm of the head rows (model.c:386-389)
        if (tid == 0) {
            float sq = 0.0f, sk = 0.0f;
            for (int i = 0; i < HD; i++) sq += qv[i] * qv[i];
            for (int i = 0; i < HD; i++) sk += kn[i] * kn[i];
            sh[0] = 1.0f / sqrtf(sq / (float)HD + a.eps);
            sh[1] = 1.0f / sqrtf(sk / (float)HD + a.eps);
        }
        __syncthreads();
        for (int i = tid; i < HD; i += WG) {
            qv[i] = qv[i] * sh[0] * a.q_norm[i];
            kn[i] = kn[i] * sh[1] * a.k_norm[i];
        }
        __syncthreads();
    }
    // rope (model.c:66-80): (v0, v1) -> (v0 c - v1 s, v0 s + v1 c), (c, s) of pos * freq_i
    const float2 *rp = a.rope + (size_t)pos * (HD / 2);
    float nq[2] = {0.0f, 0.0f}, nk[2] = {0.0f, 0.0f};
    int ia = 0, ib = 0;
    const bool pair = tid < HD / 2;
    if (pair) {
        ia = a.rope_style == ROPE_NEOX ? tid : 2 * tid;
        ib = a.rope_style == ROPE_NEOX ? tid + HD / 2 : 2 * tid + 1;
        const float2 cs = rp[tid];
        float v0 = qv[ia], v1 = qv[ib];
        nq[0] = v0 * cs.x - v1 * cs.y; nq[1] = v0 * cs.y + v1 * cs.x;
        v0 = kn[ia]; v1 = kn[ib];
        nk[0] = v0 * cs.x - v1 * cs.y; nk[1] = v0 * cs.y + v1 * cs.x;
    }
    __syncthreads();
    if (pair) { qv[ia] = nq[0]; qv[ib] = nq[1]; kn[ia] = nk[0]; kn[ib] = nk[1]; }
    __syncthreads();
    // the cache row at pos (model.c:39-48); an fp16 cache holds (and is read as) the rounded values
    const size_t rowoff = (size_t)pos * a.kv_dim + (size_t)g * HD;
    for (int i = tid; i < HD; i += WG) {
        if (F16) {
            const uint16_t hk = f2h(kn[i]), hv = f2h(vn[i]);
            if (h % G == 0) {
                reinterpret_cast<uint16_t *>(a.kc)[rowoff + i] = hk;
                reinterpret_cast<uint16_t *>(a.vc)[rowoff + i] = hv;
            }
            kn[i] = h2f(hk); vn[i] = h2f(hv);
        } else if (h % G == 0) {
            reinterpret_cast<float *>(a.kc)[rowoff + i] = kn[i];
            reinterpret_cast<float *>(a.vc)[rowoff + i] = vn[i];
        }
    }
    __syncthreads();
    auto kval = [&](int t, int i) -> float {
        if (t == pos) return kn[i];
        const size_t off = (size_t)t * a.kv_dim + (size_t)g * HD + i;
        return F16 ? h2f(reinterpret_cast<const uint16_t *>(a.kc)[off]) : reinterpret_cast<const float *>(a.kc)[off];
    };
    auto vval = [&](int t, int i) -> float {
        if (t == pos) return vn[i];
        const size_t off = (size_t)t * a.kv_dim + (size_t)g * HD + i;
        return F16 ? h2f(reinterpret_cast<const uint16_t *>(a.vc)[off]) : reinterpret_cast<const float *>(a.vc)[off];
    };
    // scores: the head dims summed in order, then times 1/sqrt(hd)
    float mx = -INFINITY;
    for (int t = tid; t <= pos; t += WG) {
        float sc = 0.0f;
        for (int i = 0; i < HD; i++) sc += qv[i] * kval(t, i);
        const float s = sc * a.inv_sqrt;
        att[t] = s;
        mx = fmaxf(mx, s);
    }
    // softmax (model.c:57-64): the maximum, expf(s - max), their sum in order, times 1/sum
    mx = wave_max(mx);
    if ((tid & 63) == 0) red[tid >> 6] = mx;
    __syncthreads();
    float M = red[0];
    for (int w = 1; w < NWAVE; w++) M = fmaxf(M, red[w]);
    for (int t = tid; t <= pos; t += WG) att[t] = ref_expf(att[t] - M);
    __syncthreads();
    if (tid == 0) {
        float sum = 0.0f;
        for (int t = 0; t <= pos; t++) sum += att[t];
        sh[0] = 1.0f / sum;
    }
    __syncthreads();
    const float inv = sh[0];
    for (int t = tid; t <= pos; t += WG) att[t] *= inv;
    __syncthreads();
    // out[i] = sum over positions in order of p_t v_t[i]
    for (int i = tid; i < HD; i += WG) {
        float o = 0.0f;
        for (int t = 0; t <= pos; t++) o += att[t] * vval(t, i);
        a.out[(size_t)h * HD + i] = o;
    }
}

int launch_attn_ref(hipStream_t st, bool f16kv, const AttnArgs &a, float *att) {
    if (a.n_kv <= 0 || a.n_heads % a.n_kv != 0 || a.hd > 256 || a.hd % 2 || !att || !a.tokpos) return -1;
    if (f16kv) hipLaunchKernelGGL((k_attn_ref<true>), dim3(a.n_heads), dim3(WG), 0, st, a, att);
    else hipLaunchKernelGGL((k_attn_ref<false>), dim3(a.n_heads), dim3(WG), 0, st, a, att);
    return 0;
}

}  // namespace ehip
