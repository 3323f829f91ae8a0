// Batched prompt processing for the Llama runner: the kernels between the
// prefill GEMMs (S prompt rows at once, rusty-graph/src/lib.rs:364-378 over
// every position of the prompt):
//   k_embed_rows        x[s] = embed[tokens[p0 + s]] (f32 residual rows)
//   k_add_rmsnorm_rows  x[s] += y[s] (the residual add of the previous
//                       projection), then xn[s] = fp16((x * inv) * w),
//                       inv = 1 / sqrt(mean(x^2) + eps) (kernels.wgsl:87-102)
//   k_rope_scatter      RoPE (kernels.wgsl:60-79) on q and k of every row;
//                       q to an fp16 [S][n_heads][hd] buffer, k and v (fp16)
//                       into the KV cache at positions p0..p0+S-1
//   k_attn_prefill      causal GQA attention of the S queries over cache
//                       positions 0..p0+S-1 on the matrix cores
//
// Attention (flash-style, four waves per (query tile of 32, head)):
// the scores of a key tile are computed transposed, S^T = K . Q^T, with
// v_mfma_f32_32x32x16_f16: A = 32 cache rows of K (lane l: row l % 32, the
// 8 halves 16 s + 8 (l / 32) of k-step s -- one 16-byte load), B = Q^T (the
// same halves of the lane's query row, loaded once).  The accumulator puts
// the scores of one query in one lane column (lane l holds keys
// 8 (r / 4) + 4 (l / 32) + r % 4, r < 16, of query l % 32), so the online
// softmax is in-lane plus one exchange with lane l ^ 32 for the running max.
// P . V is computed as O^T = V^T . P^T: the P values a lane holds are its
// B operand as they stand, once the 16 keys of a k-step are taken in the
// order the accumulator gives them (keys 4h..4h+3, 8+4h..8+4h+3 of the step
// for lane half h); V^T is staged in LDS per key tile (each lane loads 4 keys
// x 8 dims and writes 8 four-key pieces), and each lane reads its two 8-byte
// pieces of a row of V^T in that key order.  Scores, softmax and the
// accumulators are f32 (exponentials as 2^x on scores scaled by log2 e);
// q, k, v and p enter the matrix cores as fp16.
#include "common.hpp"

namespace rq {
namespace {

constexpr int NT = 256;
constexpr uint32_t kOOB = 0x80000000u;  // any offset past a buffer resource reads zero

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float floatx16 __attribute__((ext_vector_type(16)));
typedef unsigned u32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void *p, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(p), 0, bytes, 0x00020000);
}
__device__ __forceinline__ uint4 bload(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    const u32x4 v = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0));
    return make_uint4(v.x, v.y, v.z, v.w);
}

__device__ __forceinline__ uint32_t word(const uint4 v, int i) {
    return i == 0 ? v.x : (i == 1 ? v.y : (i == 2 ? v.z : v.w));
}

__global__ __launch_bounds__(NT) void k_embed_rows(const int *__restrict__ tokens, const _Float16 *__restrict__ embed,
                                                   int H, float *__restrict__ x) {
    const _Float16 *row = embed + (size_t)tokens[blockIdx.x] * H;
    float *xr = x + (size_t)blockIdx.x * H;
    for (int i = threadIdx.x; i < H; i += NT) xr[i] = (float)row[i];
}

// One block per row.  y null: no add; nw null: add only.  The row stays in
// registers between the sum of squares and the normalisation: float4 pieces,
// piece i by thread i % NT (H % 4 == 0, H <= 4 * NT * NV).
template <int NV>
__global__ __launch_bounds__(NT) void k_add_rmsnorm_rows(float *__restrict__ x, const float *__restrict__ y,
                                                         const _Float16 *__restrict__ nw, float eps,
                                                         _Float16 *__restrict__ xn, int H) {
    __shared__ float red[NT / 64];
    const int t = threadIdx.x, h4 = H / 4;
    float4 *xr = reinterpret_cast<float4 *>(x + (size_t)blockIdx.x * H);
    const float4 *yr = y ? reinterpret_cast<const float4 *>(y + (size_t)blockIdx.x * H) : nullptr;
    typedef _Float16 half4 __attribute__((ext_vector_type(4)));
    const half4 *w4 = reinterpret_cast<const half4 *>(nw);
    // every load of the row -- x, y and the norm weight -- requested before the
    // first use: one memory round trip (the weight had been a second one, after
    // the reduction)
    float4 v[NV], a[NV];
    half4 w[NV];
#pragma unroll
    for (int j = 0; j < NV; ++j) {
        const int i = t + NT * j;
        if (i < h4) {
            v[j] = xr[i];
            if (y) a[j] = yr[i];
            if (nw) w[j] = w4[i];
        }
    }
    float ss = 0.0f;
#pragma unroll
    for (int j = 0; j < NV; ++j) {
        const int i = t + NT * j;
        if (i >= h4) break;
        if (y) {
            v[j].x += a[j].x;
            v[j].y += a[j].y;
            v[j].z += a[j].z;
            v[j].w += a[j].w;
            xr[i] = v[j];
        }
        ss = fmaf(v[j].x, v[j].x, fmaf(v[j].y, v[j].y, fmaf(v[j].z, v[j].z, fmaf(v[j].w, v[j].w, ss))));
    }
    if (!nw) return;
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) ss += __shfl_xor(ss, o);
    if ((t & 63) == 0) red[t >> 6] = ss;
    __syncthreads();
    ss = (red[0] + red[1]) + (red[2] + red[3]);
    const float inv = 1.0f / sqrtf(ss / (float)H + eps);
    half4 *o4 = reinterpret_cast<half4 *>(xn + (size_t)blockIdx.x * H);
#pragma unroll
    for (int j = 0; j < NV; ++j) {
        const int i = t + NT * j;
        if (i >= h4) break;
        const half4 r = {(_Float16)((v[j].x * inv) * (float)w[j].x), (_Float16)((v[j].y * inv) * (float)w[j].y),
                         (_Float16)((v[j].z * inv) * (float)w[j].z), (_Float16)((v[j].w * inv) * (float)w[j].w)};
        o4[i] = r;
    }
}

// One block per row s (position p0 + s): qkv f32 [S][(n_heads + 2 n_kv) hd].
__global__ __launch_bounds__(NT) void k_rope_scatter(const float *__restrict__ qkv, const float2 *__restrict__ rope,
                                                     int p0, int n_heads, int n_kv, int hd, int max_seq,
                                                     _Float16 *__restrict__ q, _Float16 *__restrict__ kc,
                                                     _Float16 *__restrict__ vc) {
    const int s = blockIdx.x, pos = p0 + s, half = hd / 2, t = threadIdx.x;
    const float *row = qkv + (size_t)s * (n_heads + 2 * n_kv) * hd;
    const float2 *cs = rope + (size_t)pos * half;
    for (int i = t; i < n_heads * half; i += NT) {
        const int h = i / half, d = i % half;
        const float2 c = cs[d];
        const float a = row[h * hd + d], b = row[h * hd + d + half];
        _Float16 *o = q + ((size_t)s * n_heads + h) * hd;
        o[d] = (_Float16)(a * c.x - b * c.y);
        o[d + half] = (_Float16)(a * c.y + b * c.x);
    }
    const float *kr = row + (size_t)n_heads * hd, *vr = kr + (size_t)n_kv * hd;
    for (int i = t; i < n_kv * half; i += NT) {
        const int g = i / half, d = i % half;
        const float2 c = cs[d];
        const float a = kr[g * hd + d], b = kr[g * hd + d + half];
        _Float16 *o = kc + ((size_t)g * max_seq + pos) * hd;
        o[d] = (_Float16)(a * c.x - b * c.y);
        o[d + half] = (_Float16)(a * c.y + b * c.x);
    }
    for (int i = t; i < n_kv * hd; i += NT) {
        const int g = i / hd, d = i % hd;
        vc[((size_t)g * max_seq + pos) * hd + d] = (_Float16)vr[i];
    }
}

// Grid: n_heads x ceil(n / 32) blocks of NW waves, the longest query tiles
// first.  q: fp16 [n][n_heads][HD]; kc/vc: this layer's cache,
// [n_kv][max_seq][HD], positions 0..p0+n-1 written; out: fp16
// [n][n_heads * HD].  The NW waves of a block share one (head, query tile)
// and take its key tiles in turn (wave w: tiles w, w + NW, ...), each with
// the next tile's K and V requested before the current one is used and V^T
// staged in two alternating LDS buffers (one barrier per tile: the buffer a
// wave fills was last read two tiles earlier, before the previous barrier);
// their partial softmaxes (running max m, sum l, unnormalised O) combine
// through LDS at the end, each wave finishing 16 / NW of every lane's
// accumulator entries.  p0 is a multiple of 32, so every query tile starts a
// key tile and every key tile a query reaches holds a key at or before it:
// the running max of a wave that had a tile is finite, and a wave that had
// none weighs 2^-inf = 0.
// Measured at 512 positions, 32 heads of 64 (before the 2^x exponentials,
// which took NW = 4 from 11.6 to 10.8 us): NW = 4 11.6 us, 8 16.9 us (155
// VGPRs allow one 8-wave block per CU, so the grid needs two dispatch
// passes), 2 14.2 us, 1 22.7 us.
template <int HD, int NW>
__global__ __launch_bounds__(NW * 64) void k_attn_prefill(const _Float16 *__restrict__ q, const _Float16 *__restrict__ kc,
                                                      const _Float16 *__restrict__ vc, _Float16 *__restrict__ out,
                                                      int p0, int n, int n_heads, int n_kv, int max_seq) {
    constexpr int KS = HD / 16;  // k-steps of the score product
    constexpr int DT = HD / 32;  // 32-dim tiles of the output
    constexpr int VR = HD / 64;  // staging rounds of a V tile (8 dims per lane each)
    constexpr int VST = 72;      // bytes per row of V^T in LDS: 32 keys + 8 bytes of padding
    constexpr int VT_BYTES = HD * VST;
    constexpr int CO_BYTES = NW * DT * 16 * 64 * 4;  // the combine's O partials, after the loop
    constexpr int LDS = 2 * NW * VT_BYTES > CO_BYTES ? 2 * NW * VT_BYTES : CO_BYTES;
    constexpr int RPW = 16 / NW;  // accumulator entries each wave finishes
    __shared__ __align__(16) unsigned char lds[LDS];
    __shared__ float cm[NW][64], cl[NW][64];
    const int nqt = (n + 31) / 32;
    const int head = blockIdx.x % n_heads;
    const int q0 = (nqt - 1 - (int)blockIdx.x / n_heads) * 32;
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6, col = lane & 31, hf = lane >> 5;
    const int g = head / (n_heads / n_kv);
    const int kv_len = p0 + n;
    const auto rk = make_rsrc(kc + (size_t)g * max_seq * HD, (uint32_t)kv_len * HD * 2u);
    const auto rv = make_rsrc(vc + (size_t)g * max_seq * HD, (uint32_t)kv_len * HD * 2u);
    const auto rq = make_rsrc(q, (uint32_t)n * n_heads * HD * 2u);

    half8 qf[KS];
    {
        const bool live = q0 + col < n;
#pragma unroll
        for (int s = 0; s < KS; ++s) {
            const uint32_t off = live ? (((uint32_t)(q0 + col) * n_heads + head) * HD + 16 * s + 8 * hf) * 2u : kOOB;
            qf[s] = __builtin_bit_cast(half8, bload(rq, off));
        }
    }
    const int qpos = p0 + q0 + col;
    const int last = min(p0 + q0 + 31, kv_len - 1);  // the tile's last live query
    const int ntiles = last / 32 + 1;
    const int iters = (ntiles + NW - 1) / NW;  // the same for every wave (barriers below)
    // scores are kept in log2 units, (q.k / sqrt(HD)) * log2(e), so every
    // exponential is one v_exp_f32 (2^x); the softmax is unchanged
    const float scale = 1.4426950408889634f / sqrtf((float)HD);
    float m_run = -__builtin_inff(), l_run = 0.0f;
    floatx16 o[DT];
#pragma unroll
    for (int d = 0; d < DT; ++d)
#pragma unroll
        for (int r = 0; r < 16; ++r) o[d][r] = 0.0f;
    const int kg = lane & 7, dg = lane >> 3;  // V staging: keys 4 kg..4 kg+3, dims 8 dg..8 dg+7 (+64 per round)

    // K rows (A operand) and V rows (staging) of key tile kt; rows past the
    // cache's written end (or a tile past the last) read as zero
    half8 kf[KS];
    uint4 vr[VR][4];
    auto load = [&](int kt, half8 (&kd)[KS], uint4 (&vd)[VR][4]) {
        const int k0 = kt * 32;
#pragma unroll
        for (int s = 0; s < KS; ++s)
            kd[s] = __builtin_bit_cast(half8, bload(rk, ((uint32_t)(k0 + col) * HD + 16 * s + 8 * hf) * 2u));
#pragma unroll
        for (int rd = 0; rd < VR; ++rd)
#pragma unroll
            for (int i = 0; i < 4; ++i)
                vd[rd][i] = bload(rv, ((uint32_t)(k0 + 4 * kg + i) * HD + 64 * rd + 8 * dg) * 2u);
    };
    // one key tile from registers kd / vd (V^T through LDS buffer buf)
    auto tile = [&](int kt, const half8 (&kd)[KS], const uint4 (&vd)[VR][4], int buf) {
        const int k0 = kt * 32;
        const bool live = kt < ntiles;  // wave-uniform
        unsigned char *vt = lds + (2 * wv + buf) * VT_BYTES;
        half8 pf[2];
        if (live) {
            floatx16 sc;
#pragma unroll
            for (int r = 0; r < 16; ++r) sc[r] = 0.0f;
#pragma unroll
            for (int s = 0; s < KS; ++s) sc = __builtin_amdgcn_mfma_f32_32x32x16_f16(kd[s], qf[s], sc, 0, 0, 0);
            // sc[r]: key k0 + 8 (r / 4) + 4 hf + r % 4 against query qpos
            float mt = -__builtin_inff();
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int key = k0 + 8 * (r >> 2) + 4 * hf + (r & 3);
                sc[r] = key <= qpos ? sc[r] * scale : -__builtin_inff();
                mt = fmaxf(mt, sc[r]);
            }
            mt = fmaxf(mt, __shfl_xor(mt, 32));
            const float m_new = fmaxf(m_run, mt);
            const float alpha = __builtin_amdgcn_exp2f(m_run - m_new);
            m_run = m_new;
            l_run *= alpha;
#pragma unroll
            for (int d = 0; d < DT; ++d)
#pragma unroll
                for (int r = 0; r < 16; ++r) o[d][r] *= alpha;
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const float p = __builtin_amdgcn_exp2f(sc[r] - m_new);
                l_run += p;
                pf[r >> 3][r & 7] = (_Float16)p;
            }
#pragma unroll
            for (int rd = 0; rd < VR; ++rd)
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    // halves j of the four key rows -> V^T[64 rd + 8 dg + j][4 kg .. 4 kg + 3]
                    const uint32_t w0 = word(vd[rd][0], j >> 1), w1 = word(vd[rd][1], j >> 1);
                    const uint32_t w2 = word(vd[rd][2], j >> 1), w3 = word(vd[rd][3], j >> 1);
                    const uint32_t sel = (j & 1) ? 0x07060302u : 0x05040100u;
                    const uint2 piece =
                        make_uint2(__builtin_amdgcn_perm(w1, w0, sel), __builtin_amdgcn_perm(w3, w2, sel));
                    *reinterpret_cast<uint2 *>(vt + (64 * rd + 8 * dg + j) * VST + 8 * kg) = piece;
                }
        }
        __syncthreads();  // V^T of this tile is written
        if (live) {
#pragma unroll
            for (int d = 0; d < DT; ++d) {
                const unsigned char *rowp = vt + (32 * d + col) * VST;
#pragma unroll
                for (int s2 = 0; s2 < 2; ++s2) {
                    const uint2 a = *reinterpret_cast<const uint2 *>(rowp + (16 * s2 + 4 * hf) * 2);
                    const uint2 b = *reinterpret_cast<const uint2 *>(rowp + (16 * s2 + 8 + 4 * hf) * 2);
                    const half8 va = __builtin_bit_cast(half8, make_uint4(a.x, a.y, b.x, b.y));
                    o[d] = __builtin_amdgcn_mfma_f32_32x32x16_f16(va, pf[s2], o[d], 0, 0, 0);
                }
            }
        }
    };
    // Ping-pong over two named register sets, every load unconditional (a
    // tile past the last reads zeros and is skipped), so the compiler's
    // in-order load counting lets the next tile's loads stay in flight while
    // the current one is used.
    half8 kb[KS];
    uint4 vb[VR][4];
    load(wv, kf, vr);
    for (int it = 0; it < iters; it += 2) {
        load(wv + NW * (it + 1), kb, vb);
        tile(wv + NW * it, kf, vr, 0);
        load(wv + NW * (it + 2), kf, vr);
        tile(wv + NW * (it + 1), kb, vb, 1);
    }

    // combine the waves' partials: wave wv finishes accumulator entries
    // RPW wv..RPW wv + RPW - 1 of every dim tile of its lanes
    __syncthreads();  // every wave's V^T reads are done: the area holds the O partials now
    float *co = reinterpret_cast<float *>(lds);
    cm[wv][lane] = m_run;
    cl[wv][lane] = l_run;
#pragma unroll
    for (int d = 0; d < DT; ++d)
#pragma unroll
        for (int r = 0; r < 16; ++r) co[((wv * DT + d) * 16 + r) * 64 + lane] = o[d][r];
    __syncthreads();
    float mx = cm[0][lane];
#pragma unroll
    for (int w = 1; w < NW; ++w) mx = fmaxf(mx, cm[w][lane]);
    float wt[NW], L = 0.0f;
#pragma unroll
    for (int w = 0; w < NW; ++w) {
        wt[w] = __builtin_amdgcn_exp2f(cm[w][lane] - mx);
        L = fmaf(wt[w], cl[w][lane] + cl[w][lane ^ 32], L);  // both halves of the query's keys
    }
    const float inv = 1.0f / L;
    if (q0 + col < n) {
        _Float16 *orow = out + ((size_t)(q0 + col) * n_heads + head) * HD;
#pragma unroll
        for (int d = 0; d < DT; ++d)
#pragma unroll
            for (int e = 0; e < RPW; ++e) {
                const int r = RPW * wv + e;
                float a = 0.0f;
#pragma unroll
                for (int w = 0; w < NW; ++w) a = fmaf(wt[w], co[((w * DT + d) * 16 + r) * 64 + lane], a);
                orow[32 * d + 8 * (r >> 2) + 4 * hf + (r & 3)] = (_Float16)(a * inv);
            }
    }
}

}  // namespace

int launch_embed_rows(const int *tokens, const _Float16 *embed, int H, float *x, int n, hipStream_t s) {
    hipLaunchKernelGGL(k_embed_rows, dim3(n), dim3(NT), 0, s, tokens, embed, H, x);
    RQ_LAUNCH_CHECK();
    return RQ_OK;
}

int launch_add_rmsnorm_rows(float *x, const float *y, const _Float16 *nw, float eps, _Float16 *xn, int n, int H,
                            hipStream_t s) {
    if (H % 4 != 0 || H > 4 * NT * 16 || !aligned(x, 16) || (y && !aligned(y, 16)) || (nw && !aligned(nw, 8)) ||
        (nw && !aligned(xn, 8)))
        return RQ_ERR_UNSUPPORTED;
    if (H <= 4 * NT * 2)
        hipLaunchKernelGGL(k_add_rmsnorm_rows<2>, dim3(n), dim3(NT), 0, s, x, y, nw, eps, xn, H);
    else if (H <= 4 * NT * 4)
        hipLaunchKernelGGL(k_add_rmsnorm_rows<4>, dim3(n), dim3(NT), 0, s, x, y, nw, eps, xn, H);
    else if (H <= 4 * NT * 8)
        hipLaunchKernelGGL(k_add_rmsnorm_rows<8>, dim3(n), dim3(NT), 0, s, x, y, nw, eps, xn, H);
    else
        hipLaunchKernelGGL(k_add_rmsnorm_rows<16>, dim3(n), dim3(NT), 0, s, x, y, nw, eps, xn, H);
    RQ_LAUNCH_CHECK();
    return RQ_OK;
}

int launch_rope_scatter(const float *qkv, const float2 *rope, int p0, int n, int n_heads, int n_kv, int hd,
                        int max_seq, _Float16 *q, _Float16 *kc, _Float16 *vc, hipStream_t s) {
    hipLaunchKernelGGL(k_rope_scatter, dim3(n), dim3(NT), 0, s, qkv, rope, p0, n_heads, n_kv, hd, max_seq, q, kc, vc);
    RQ_LAUNCH_CHECK();
    return RQ_OK;
}

int launch_attn_prefill(const _Float16 *q, const _Float16 *kc, const _Float16 *vc, _Float16 *out, int p0, int n,
                        int n_heads, int n_kv, int hd, int max_seq, hipStream_t s) {
    if (p0 % 32 != 0 || n < 1 || (hd != 64 && hd != 128) || n_heads % n_kv != 0) return RQ_ERR_UNSUPPORTED;
    const dim3 grid((unsigned)(n_heads * ((n + 31) / 32)));
    if (hd == 64)
        hipLaunchKernelGGL((k_attn_prefill<64, 4>), grid, dim3(256), 0, s, q, kc, vc, out, p0, n, n_heads, n_kv,
                           max_seq);
    else
        hipLaunchKernelGGL((k_attn_prefill<128, 4>), grid, dim3(256), 0, s, q, kc, vc, out, p0, n, n_heads, n_kv,
                           max_seq);
    RQ_LAUNCH_CHECK();
    return RQ_OK;
}

}  // namespace rq
