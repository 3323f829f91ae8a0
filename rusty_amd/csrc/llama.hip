// Quantized-weight Llama decode runner (per-row int8 or affine u8 Linears): one greedy decode step of a LlamaModel
// (rusty-graph/src/lib.rs:420-436) as a HIP graph of 5 launches per block
// plus 2 at the end, replayed once per token with no host round trip.
//
// Per block (LlamaBlock::forward, rusty-graph/src/lib.rs:364-378):
//   qkv  = rmsnorm(x, attn_norm) . [Wq;Wk;Wv]^T   decode GEMV with the RMSNorm
//                                                 in its prologue (q, k, v
//                                                 packed into one weight), RoPE
//                                                 and the KV append in its
//                                                 epilogue
//   attn = softmax(q . K^T / sqrt(d)) . V         k_attn_decode (GQA attention
//                                                 over the cache, split over
//                                                 positions: partials)
//   x   += attn . Wo^T                            decode GEMV: the partials are
//                                                 combined in its prologue, add
//                                                 epilogue
//   h    = silu(xn . Wg^T) * (xn . Wu^T),         fused gate/up decode GEMV,
//          xn = rmsnorm(x, mlp_norm)              norm in its prologue
//   x   += h . Wd^T                               decode GEMV, add epilogue
// then logits = rmsnorm(x, final_norm) . Wlm^T (norm fused likewise) and
// k_argmax_embed picks the greedy token (top_k with k = 1,
// kernels.wgsl:173-188), appends it to the sequence and gathers its embedding
// row into x for the next step (Embedding::forward, rusty-graph/src/lib.rs:
// 121-135, done on the device).
//
// All state the step reads (position, token sequence, residual x, KV cache)
// lives in device memory, so the same instantiated graph serves every
// position.  The residual stream x is f32; activations entering a GEMV are
// fp16; the KV cache is fp16 in [layer][kv_head][position][head_dim] order.
#include <math.h>

#include <algorithm>
#include <new>
#include <type_traits>
#include <vector>

#include "common.hpp"

struct rq_llama {
    struct Layer {
        const _Float16 *attn_norm, *mlp_norm;
        rq_qweight qkv, o, gate, up, down;
    };
    rq_ctx *ctx = nullptr;
    rq_llama_config cfg{};
    std::vector<Layer> layers;
    const _Float16 *embed = nullptr, *final_norm = nullptr;
    rq_qweight lm_head{};
    void *owned = nullptr;  // packed qkv weights + step state, one allocation
    float *x = nullptr, *qkv_out = nullptr, *logits = nullptr;
    // attention partials: fp16 acc / l [n_heads][n_split][head_dim], then f32 (m, l) pairs
    float *part = nullptr;
    int n_split = 1;        // attention blocks per query head
    _Float16 *h = nullptr, *kc = nullptr, *vc = nullptr;
    int *tokens = nullptr, *pos = nullptr, *n_prompt = nullptr;
    float2 *rope = nullptr;  // (cos, sin) per position and rotated pair
    // batched prompt buffers, prefill_cap rows: residual rows x and projection
    // outputs y (f32 [rows][H]), normalised rows xn (fp16 [rows][H]), q/k/v
    // (f32 [rows][QKV]), roped q and the attention output (fp16
    // [rows][n_heads * head_dim]), SwiGLU workspace h (fp16 [2][rows][I])
    float *px = nullptr, *py = nullptr, *pqkv = nullptr;
    _Float16 *pxn = nullptr, *pq = nullptr, *patt = nullptr, *ph = nullptr;
    int prefill_cap = 0;   // rows the buffers hold
    int prefill_rows = 0;  // rows per batched chunk; 0: one position at a time through the step graph
    hipGraph_t graph = nullptr;  // one decode step
    hipGraphExec_t exec = nullptr;
    hipGraph_t graph_k = nullptr;  // kGraphSteps consecutive steps
    hipGraphExec_t exec_k = nullptr;
    bool use_graph = true;
    int host_pos = 0;  // tokens already in the KV cache (the next step's position)
    int host_len = 0;  // tokens in the sequence, prompt + generated
};

namespace rq {
namespace {

constexpr int NT = 256;
constexpr int kMaxSeq = 32768;  // KV cache capacity limit (32-bit cache offsets)
// Rows of a batched prompt chunk: prompts up to this many positions (and
// max_seq) run as one chunk of [rows, H] GEMMs, longer ones in chunks.
constexpr int kPrefillRows = 2048;

typedef _Float16 h2_t __attribute__((ext_vector_type(2)));

// Cross-lane steps as DPP operand modifiers (one VALU op each) instead of
// LDS-routed shuffles; whole-wave results through four readlanes.
template <int CTRL>
__device__ __forceinline__ float dpp(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}
__device__ __forceinline__ float readlane(float v, int l) {
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), l));
}
// Sum over aligned groups of G lanes (G = 8 or 16); every lane of a group
// receives its group's sum.
template <int G>
__device__ __forceinline__ float group_sum(float v) {
    static_assert(G == 8 || G == 16, "DPP row steps cover groups of 8 or 16 lanes");
    v += dpp<0xB1>(v);   // quad_perm [1,0,3,2]
    v += dpp<0x4E>(v);   // quad_perm [2,3,0,1]
    v += dpp<0x141>(v);  // row_half_mirror: lane i of 8 reads lane 7 - i
    if constexpr (G == 16) v += dpp<0x140>(v);  // row_mirror: lane i of 16 reads lane 15 - i
    return v;
}
__device__ __forceinline__ float wave_sum(float v) {
    v = group_sum<16>(v);
    return (readlane(v, 0) + readlane(v, 16)) + (readlane(v, 32) + readlane(v, 48));
}
__device__ __forceinline__ float wave_max(float v) {
    v = fmaxf(v, dpp<0xB1>(v));
    v = fmaxf(v, dpp<0x4E>(v));
    v = fmaxf(v, dpp<0x141>(v));
    v = fmaxf(v, dpp<0x140>(v));
    return fmaxf(fmaxf(readlane(v, 0), readlane(v, 16)), fmaxf(readlane(v, 32), readlane(v, 48)));
}
constexpr uint32_t kOOB = 0x80000000u;  // any offset past a buffer resource reads zero

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void *p, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(p), 0, bytes, 0x00020000);
}
__device__ __forceinline__ uint4 bload(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    typedef unsigned u32x4 __attribute__((ext_vector_type(4)));
    const u32x4 v = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0));
    return make_uint4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ void widen8(const uint4 u, float *f) {
    const uint32_t wd[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const h2_t p = __builtin_bit_cast(h2_t, wd[i]);
        f[2 * i] = (float)p.x;
        f[2 * i + 1] = (float)p.y;
    }
}

// Decode attention at position pos = *pos_p, split over positions in tiles
// of one pass (PASS positions): block (head hd, split sp) of a grid of
// n_heads * S takes tiles sp, sp + S, sp + 2 S, ... of positions 0..pos and
// writes its partial softmax -- the running max m, the sum l of
// exp(score - m), and its output o[d] = acc[d] / l for the unnormalised
// accumulator acc[d] = sum exp(score - m) * v[d] -- as fp16 o to
// part[(hd * S + sp) * HD + d] and f32 ml[hd * S + sp] = (m, l).  A block
// with no position (sp * PASS > pos) writes o = 0, (m, l) = (-inf, 0).  The
// consumer (the o-projection GEMV's prologue) combines the S partials of a
// head: out = sum_s w_s o_s / sum_s w_s, w_s = e^(m_s - M) l_s,
// M = max_s m_s.  Normalised, o is within v's range, so fp16 holds it to
// 2^-11 (the combined row is rounded to fp16 anyway); half the bytes of f32
// partials, which every o-projection block reads (step +1.2 %).
//
// The q/k/v projection before it (launch_gemv_decode_qkv_rope) has already
// rotated q and k (RoPE, kernels.wgsl:60-79) and appended this position's
// key and value to the cache (rusty-graph/src/lib.rs:235-246), so the block
// reads only the rotated query (f32) and cache rows 0..pos.  Its first tile
// does not depend on the position, so the position, the query and that
// tile's K/V rows are requested together at the start: one memory round trip
// before the arithmetic (cache rows past pos are loaded -- whatever an
// earlier sequence left there -- and zeroed once the position is known).
// Scores q.k / sqrt(HD), softmax in f32.  GQA: query head h reads KV head
// h / (n_heads / n_kv) (flash_attention_v2.wgsl:79-83).
//
// Latency-bound: each block streams its tiles' K and V rows through one CU,
// so splitting a head's context over S blocks divides that stream.  A pass
// covers 8 waves x RW consecutive rows each; lane l holds 16-byte chunk
// l % CH of row i * RPI + l / CH for i < NI, all in flight before any is
// used.  The block's work is a serial chain of short dependent steps, so it
// is spread thin: 8 waves of 4 row loads measured 1.4-1.6 % more tokens/s
// for the whole decode step than 4 waves of 8 (16 waves of 2: +0.7 %), and 8
// waves of 2 another 1.0 %.  Row scores finish with DPP steps over the CH
// lanes of a row; each wave runs its own online softmax (max and sum by DPP
// steps and readlanes, tiles beyond the first by the rescale), and the P.V
// partials are summed over the lanes of a chunk, then over waves in LDS
// weighted by e^(m_w - M): one barrier per block.
constexpr int ATT = 512;  // threads per attention block

template <int HD>
__global__ __launch_bounds__(ATT) void k_attn_decode(const float *__restrict__ q, const _Float16 *__restrict__ kc,
                                                     const _Float16 *__restrict__ vc, const int *__restrict__ pos_p,
                                                     float *__restrict__ part, float2 *__restrict__ ml, int n_heads,
                                                     int n_kv, int max_seq, int S) {
    constexpr int NW = ATT / 64;
    constexpr int CH = HD / 8;         // 16-byte chunks per row
    constexpr int RPI = 64 / CH;       // rows per wave-wide load
    constexpr int NI = 2;              // loads of K (and of V) per lane per pass
    constexpr int RW = NI * RPI;       // rows per wave per pass
    constexpr int PASS = NW * RW;      // positions per pass (one tile)
    __shared__ float redm[NW], reds[NW];
    __shared__ float accs[NW][4][HD];
    const int hd = blockIdx.x / S, sp = blockIdx.x % S, t = threadIdx.x, lane = t & 63, w = t >> 6;
    const int grp = n_heads / n_kv, g = hd / grp;
    // the whole cache of this KV head: rows up to max_seq (past it: zeros)
    const auto rk = make_rsrc(kc + (size_t)g * max_seq * HD, (uint32_t)max_seq * HD * 2u);
    const auto rv = make_rsrc(vc + (size_t)g * max_seq * HD, (uint32_t)max_seq * HD * 2u);
    const int ch = lane % CH, rl = lane / CH;
    uint4 kr[NI], vr[NI];
    auto load_tile = [&](int c0) {
#pragma unroll
        for (int i = 0; i < NI; ++i) {
            const uint32_t row = (uint32_t)(c0 + RW * w + i * RPI + rl);
            const uint32_t off = ((row * HD + (uint32_t)ch * 8) * 2u);
            kr[i] = bload(rk, row < (uint32_t)max_seq ? off : kOOB);
            vr[i] = bload(rv, row < (uint32_t)max_seq ? off : kOOB);
        }
    };
    const int c_first = sp * PASS;
    load_tile(c_first);  // before the position is known
    const int pos = *pos_p;
    // this lane's 8 elements of the rotated query
    float qv[8];
    {
        const float4 *qp = reinterpret_cast<const float4 *>(q + (size_t)hd * HD + ch * 8);
        const float4 a = qp[0], b = qp[1];
        qv[0] = a.x; qv[1] = a.y; qv[2] = a.z; qv[3] = a.w;
        qv[4] = b.x; qv[5] = b.y; qv[6] = b.z; qv[7] = b.w;
    }
    const int T = pos + 1;

    // Each wave keeps its own online softmax over its rows of every tile
    // (running max m, sum l, accumulator acc): no barrier inside the loop.
    // The block's waves merge once at the end.
    const float scale = 1.0f / sqrtf((float)HD);
    float m_run = -__builtin_inff(), l_run = 0.0f, acc[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[e] = 0.0f;
    for (int c0 = c_first; c0 < T; c0 += S * PASS) {
        const int base = c0 + RW * w;
        if (c0 > c_first) load_tile(c0);  // the first tile was requested at the start
        if (base >= T) break;  // wave-uniform: this wave's rows of this and later tiles are past the position
        float sv[NI];
        float lm = -__builtin_inff();
#pragma unroll
        for (int i = 0; i < NI; ++i) {
            const int row = base + i * RPI + rl;
            if (row >= T) {  // a row past the position: not this sequence's (yet)
                kr[i] = make_uint4(0, 0, 0, 0);
                vr[i] = make_uint4(0, 0, 0, 0);
            }
            float f[8], sc = 0.0f;
            widen8(kr[i], f);
#pragma unroll
            for (int e = 0; e < 8; ++e) sc = fmaf(qv[e], f[e], sc);
            sc = group_sum<CH>(sc);
            sv[i] = row < T ? sc * scale : -__builtin_inff();
            lm = fmaxf(lm, sv[i]);
        }
        // finite: the wave's first row (base < T) is live
        const float m_new = fmaxf(m_run, wave_max(lm));
        const float alpha = expf(m_run - m_new);
        float ls = 0.0f;
#pragma unroll
        for (int e = 0; e < 8; ++e) acc[e] *= alpha;
#pragma unroll
        for (int i = 0; i < NI; ++i) {
            const float p = expf(sv[i] - m_new);  // 0 for rows past the position (their V is zeroed)
            float f[8];
            widen8(vr[i], f);
#pragma unroll
            for (int e = 0; e < 8; ++e) acc[e] = fmaf(p, f[e], acc[e]);
            ls += ch == 0 ? p : 0.0f;  // one lane per row counts it
        }
        l_run = l_run * alpha + wave_sum(ls);
        m_run = m_new;
    }
    // sum P.V partials over the lanes holding the same chunk: within a 16-lane
    // row (HD = 64: two rows of 8 chunks, row_ror 8 pairs lane i with i + 8),
    // then over the four rows of each wave and over waves in LDS, each wave's
    // sums weighted by e^(m_w - M), M the block's max; stored divided by the
    // block's sum l (0 for a block with no position)
    if constexpr (CH == 8) {
#pragma unroll
        for (int e = 0; e < 8; ++e) acc[e] += dpp<0x128>(acc[e]);
    }
    if ((lane & 15) < CH) {
#pragma unroll
        for (int e = 0; e < 8; ++e) accs[w][lane >> 4][ch * 8 + e] = acc[e];
    }
    if (lane == 0) {
        redm[w] = m_run;
        reds[w] = l_run;
    }
    __syncthreads();
    const size_t slot = (size_t)hd * S + sp;
    if (t < HD) {
        float M = redm[0];
#pragma unroll
        for (int i = 1; i < NW; ++i) M = fmaxf(M, redm[i]);
        float sum = 0.0f, L = 0.0f;
        if (M != -__builtin_inff()) {  // else: no position in this block's tiles
#pragma unroll
            for (int i = 0; i < NW; ++i) {
                const float f = expf(redm[i] - M);  // 0 for a wave with no row
                float a = 0.0f;
#pragma unroll
                for (int j = 0; j < 4; ++j) a += accs[i][j][t];
                sum = fmaf(f, a, sum);
                L = fmaf(f, reds[i], L);
            }
        }
        reinterpret_cast<_Float16 *>(part)[slot * HD + t] = (_Float16)(L > 0.0f ? sum / L : 0.0f);
        if (t == 0) ml[slot] = make_float2(M, L);
    }
}

constexpr int AT = 1024;

// RoPE table: rope[p * (HD/2) + d] = (cos, sin) of p * theta^(-2d/HD) in f32,
// the reference's angle formula (kernels.wgsl:63-69), for every position.
__global__ __launch_bounds__(NT) void k_rope_table(float2 *__restrict__ rope, int max_seq, int hd, float theta) {
    const int half = hd / 2;
    const int64_t i = (int64_t)blockIdx.x * NT + threadIdx.x;
    if (i >= (int64_t)max_seq * half) return;
    const int p = (int)(i / half), d = (int)(i % half);
    const float inv_freq = powf(theta, -2.0f * (float)d / (float)hd);
    float sn, cs;
    sincosf((float)p * inv_freq, &sn, &cs);
    rope[i] = make_float2(cs, sn);
}

// Greedy pick + embedding gather, one block.  The step processed the token at
// position pos = *pos_p.  The next token is the prompt's token pos + 1 while
// the prompt lasts (teacher forcing during prefill), else the argmax of the
// logits: the first index of the largest value greater than -1e9, index 0 if
// none (the reference's top_k scan, kernels.wgsl:177-186).  It is stored at
// tokens[pos + 1], its fp16 embedding row is widened into x, and *pos_p
// advances by one.
__global__ __launch_bounds__(AT) void k_argmax_embed(const float *__restrict__ logits, int V,
                                                     const _Float16 *__restrict__ embed, int H,
                                                     int *__restrict__ tokens, int *__restrict__ pos_p,
                                                     const int *__restrict__ n_prompt_p, float *__restrict__ x) {
    __shared__ float bv[AT / 64];
    __shared__ int bi[AT / 64];
    __shared__ int next_s;
    const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
    // position, prompt length and the prompt's next token are requested
    // before the scan, off the block's tail
    const int pos = *pos_p;
    const int n_prompt = *n_prompt_p;
    const bool teacher = pos + 1 < n_prompt;
    const int forced = teacher ? tokens[pos + 1] : 0;
    float best = -1e9f;
    int idx = 0;
    // each thread scans its indices in ascending order (strict >: the first
    // of equal maxima), 8 float4 loads in flight per round
    const auto rl = make_rsrc(logits, (uint32_t)V * 4u);
    const int n4 = (V + 3) / 4;
    for (int b = 0; b < n4; b += AT * 8) {
        uint4 v4[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            const int i4 = b + u * AT + t;
            v4[u] = bload(rl, i4 < n4 ? (uint32_t)i4 * 16u : kOOB);
        }
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            const uint32_t wd[4] = {v4[u].x, v4[u].y, v4[u].z, v4[u].w};
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int i = (b + u * AT + t) * 4 + e;
                const float v = __builtin_bit_cast(float, wd[e]);
                if (i < V && v > best) {
                    best = v;
                    idx = i;
                }
            }
        }
    }
    // (value, index) pairs combine by the larger value, then the smaller index:
    // a total order, so any reduction tree picks the scan's answer
    auto take = [&](float ov, int oi) {
        if (ov > best || (ov == best && oi < idx)) {
            best = ov;
            idx = oi;
        }
    };
    auto dpp_step = [&](auto ctrl) {
        constexpr int C = decltype(ctrl)::value;
        take(dpp<C>(best), __builtin_amdgcn_update_dpp(0, idx, C, 0xF, 0xF, false));
    };
    dpp_step(std::integral_constant<int, 0xB1>{});   // quad_perm [1,0,3,2]
    dpp_step(std::integral_constant<int, 0x4E>{});   // quad_perm [2,3,0,1]
    dpp_step(std::integral_constant<int, 0x141>{});  // row_half_mirror
    dpp_step(std::integral_constant<int, 0x140>{});  // row_mirror: each 16-lane row holds its pick
    {
        const float v0 = best;
        const int i0 = idx;
        best = readlane(v0, 0);
        idx = __builtin_amdgcn_readlane(i0, 0);
#pragma unroll
        for (int r = 16; r < 64; r += 16) take(readlane(v0, r), __builtin_amdgcn_readlane(i0, r));
    }
    if (lane == 0) {
        bv[wave] = best;
        bi[wave] = idx;
    }
    __syncthreads();
    if (t == 0) {
        for (int w = 1; w < AT / 64; ++w) take(bv[w], bi[w]);
        const int next = teacher ? forced : idx;
        tokens[pos + 1] = next;
        next_s = next;
    }
    __syncthreads();
    const _Float16 *row = embed + (size_t)next_s * H;
    for (int i = t; i < H; i += AT) x[i] = (float)row[i];
    if (t == 0) *pos_p = pos + 1;
}

// Start of a sequence: x = embed[tokens[0]], pos = 0, prompt length n.
__global__ __launch_bounds__(NT) void k_embed_start(const int *__restrict__ tokens, const _Float16 *__restrict__ embed,
                                                    int H, float *__restrict__ x, int *__restrict__ pos_p,
                                                    int *__restrict__ n_prompt_p, int n_prompt) {
    const _Float16 *row = embed + (size_t)tokens[0] * H;
    for (int i = threadIdx.x; i < H; i += NT) x[i] = (float)row[i];
    if (threadIdx.x == 0) {
        *pos_p = 0;
        *n_prompt_p = n_prompt;
    }
}

// The step state after a batched prompt: the last prompt position was
// processed (pos) and the prompt has n tokens.
__global__ void k_set_position(int *__restrict__ pos_p, int *__restrict__ n_prompt_p, int pos, int n) {
    *pos_p = pos;
    *n_prompt_p = n;
}

int enqueue_step(rq_llama *md, hipStream_t s) {
    const rq_llama_config &c = md->cfg;
    const int H = c.hidden;
    const size_t kv_layer = (size_t)c.n_kv_heads * c.max_seq * c.head_dim;
    int st;
    for (int l = 0; l < c.n_layers; ++l) {
        const rq_llama::Layer &L = md->layers[l];
        // q/k/v with RoPE and the KV append in the projection's epilogue
        RopeDecode rd;
        rd.pos = md->pos;
        rd.rope = md->rope;
        rd.q = md->qkv_out;  // rotated q: the first n_heads * head_dim values
        rd.kc = md->kc + l * kv_layer;
        rd.vc = md->vc + l * kv_layer;
        rd.n_heads = c.n_heads;
        rd.n_kv = c.n_kv_heads;
        rd.hd = c.head_dim;
        rd.max_seq = c.max_seq;
        if ((st = launch_gemv_decode_qkv_rope(L.qkv, md->x, L.attn_norm, c.norm_eps, rd, s)) != RQ_OK) return st;
        const int S = md->n_split;
        // (m, l) pairs after the fp16 partials (n_heads * S * head_dim halves)
        float2 *ml = reinterpret_cast<float2 *>(md->part + (size_t)c.n_heads * S * c.head_dim / 2);
        if (c.head_dim == 64)
            hipLaunchKernelGGL(k_attn_decode<64>, dim3(c.n_heads * S), dim3(ATT), 0, s, md->qkv_out,
                               md->kc + l * kv_layer, md->vc + l * kv_layer, md->pos, md->part, ml, c.n_heads,
                               c.n_kv_heads, c.max_seq, S);
        else
            hipLaunchKernelGGL(k_attn_decode<128>, dim3(c.n_heads * S), dim3(ATT), 0, s, md->qkv_out,
                               md->kc + l * kv_layer, md->vc + l * kv_layer, md->pos, md->part, ml, c.n_heads,
                               c.n_kv_heads, c.max_seq, S);
        RQ_LAUNCH_CHECK();
        if ((st = launch_gemv_decode_attn_add(L.o, md->part, S, c.head_dim, md->x, s)) != RQ_OK) return st;
        if ((st = launch_swiglu_decode_norm(L.gate, L.up, md->x, L.mlp_norm, c.norm_eps, md->h, s)) != RQ_OK)
            return st;
        if ((st = launch_gemv_decode_add(L.down, md->h, md->x, 1, s)) != RQ_OK) return st;
    }
    if ((st = launch_gemv_decode_norm(md->lm_head, md->x, md->final_norm, c.norm_eps, md->logits, s)) != RQ_OK)
        return st;
    hipLaunchKernelGGL(k_argmax_embed, dim3(1), dim3(AT), 0, s, md->logits, c.vocab, md->embed, H, md->tokens, md->pos,
                       md->n_prompt, md->x);
    RQ_LAUNCH_CHECK();
    return RQ_OK;
}

// The decode kernels this runner launches take per-row int8 or affine u8
// weights (affine: group % 16 == 0 and k % group == 0) with k % 16 == 0,
// k <= 16384 and 16-byte aligned codes.
int check_linear(const rq_qweight &w, int64_t n, int64_t k, const char *name, int layer) {
    int st = check_qweight(&w);
    if (st != RQ_OK) return st;
    if (w.n_out != n || w.k_in != k)
        return fail(RQ_ERR_SHAPE, "layer %d %s: weight is [%lld,%lld], expected [%lld,%lld]", layer, name,
                    (long long)w.n_out, (long long)w.k_in, (long long)n, (long long)k);
    if (w.format == RQ_Q_AFFINE_U8 && (w.group % 16 != 0 || k % w.group != 0))
        return fail(RQ_ERR_UNSUPPORTED, "layer %d %s: affine weights need group %% 16 == 0 and k %% group == 0",
                    layer, name);
    if (k % 16 != 0 || k > 16384 || !aligned(w.codes, 16))
        return fail(RQ_ERR_UNSUPPORTED, "layer %d %s: needs k %% 16 == 0, k <= 16384 and 16-byte aligned codes",
                    layer, name);
    return RQ_OK;
}

// Weights fused into one launch (q/k/v, gate/up) share format, group and the
// presence of biases.
int check_same(const rq_qweight &a, const rq_qweight &b, const char *what, int layer) {
    if (a.format != b.format || (a.format == RQ_Q_AFFINE_U8 && (a.group != b.group || !a.biases != !b.biases)))
        return fail(RQ_ERR_UNSUPPORTED, "layer %d: %s weights differ in format, group or biases", layer, what);
    return RQ_OK;
}

// Prompt positions p0..p0+n-1 (tokens already in md->tokens) through every
// layer at once: [n, H] GEMMs, the causal prefill attention writing the KV
// cache.  The last chunk (end) also computes the logits of position p0+n-1
// and appends the greedy token, leaving the step state where the decode
// steps continue (x = its embedding, pos = p0 + n).
int prefill_chunk(rq_llama *md, int p0, int n, bool end, hipStream_t s) {
    const rq_llama_config &c = md->cfg;
    const int H = c.hidden;
    const size_t kv_layer = (size_t)c.n_kv_heads * c.max_seq * c.head_dim;
    const GemmWorkspace ws = gemm_workspace(md->ctx, s);
    int st;
    if ((st = launch_embed_rows(md->tokens + p0, md->embed, H, md->px, n, s)) != RQ_OK) return st;
    for (int l = 0; l < c.n_layers; ++l) {
        const rq_llama::Layer &L = md->layers[l];
        // x += (previous layer's down projection), xn = rmsnorm(x)
        if ((st = launch_add_rmsnorm_rows(md->px, l ? md->py : nullptr, L.attn_norm, c.norm_eps, md->pxn, n, H, s)))
            return st;
        _Float16 *kc = md->kc + l * kv_layer, *vc = md->vc + l * kv_layer;
        // q/k/v with the rotation in the GEMM's epilogue where its tiles are one
        // head wide; else the f32 product, then the rotation and cache writes
        RopeOut ro;
        ro.rope = md->rope;
        ro.kc = kc;
        ro.vc = vc;
        ro.p0 = p0;
        ro.n_heads = c.n_heads;
        ro.n_kv = c.n_kv_heads;
        ro.max_seq = c.max_seq;
        st = c.head_dim == 64 ? launch_gemm_qkv_rope(L.qkv, md->pxn, n, ro, md->pq, md->ctx->num_cus, ws, s)
                              : RQ_ERR_UNSUPPORTED;
        if (st == RQ_ERR_UNSUPPORTED) {
            if ((st = qmatmul_dispatch(md->ctx, L.qkv, md->pxn, RQ_F16, md->pqkv, RQ_F32, n, ws, s))) return st;
            if ((st = launch_rope_scatter(md->pqkv, md->rope, p0, n, c.n_heads, c.n_kv_heads, c.head_dim, c.max_seq,
                                          md->pq, kc, vc, s)))
                return st;
        } else if (st != RQ_OK) {
            return st;
        }
        if (l == c.n_layers - 1) break;  // the last layer's rest: below, for the last position only
        if ((st = launch_attn_prefill(md->pq, kc, vc, md->patt, p0, n, c.n_heads, c.n_kv_heads, c.head_dim,
                                      c.max_seq, s)))
            return st;
        if ((st = qmatmul_dispatch(md->ctx, L.o, md->patt, RQ_F16, md->py, RQ_F32, n, ws, s))) return st;
        if ((st = launch_add_rmsnorm_rows(md->px, md->py, L.mlp_norm, c.norm_eps, md->pxn, n, H, s))) return st;
        if ((st = swiglu_run(md->ctx, L.gate, L.up, L.down, md->pxn, RQ_F16, md->ph, md->py, RQ_F32, n, ws, s)))
            return st;
    }
    // Past its KV-cache write, the last layer matters only through the last
    // position's output, and only in the final chunk (a later chunk starts
    // again from embeddings): its attention runs for the last query tile, its
    // o projection, norm and MLP for the last row (the decode GEMVs).
    if (!end) return RQ_OK;
    {
        const rq_llama::Layer &L = md->layers[c.n_layers - 1];
        const size_t l = (size_t)c.n_layers - 1, qrow = (size_t)c.n_heads * c.head_dim;
        const int t0 = 32 * ((n - 1) / 32);  // first row of the last query tile
        if ((st = launch_attn_prefill(md->pq + t0 * qrow, md->kc + l * kv_layer, md->vc + l * kv_layer,
                                      md->patt + t0 * qrow, p0 + t0, n - t0, c.n_heads, c.n_kv_heads, c.head_dim,
                                      c.max_seq, s)))
            return st;
        const size_t last = (size_t)(n - 1);
        if ((st = qmatmul_dispatch(md->ctx, L.o, md->patt + last * qrow, RQ_F16, md->py + last * H, RQ_F32, 1, ws, s)))
            return st;
        if ((st = launch_add_rmsnorm_rows(md->px + last * H, md->py + last * H, L.mlp_norm, c.norm_eps,
                                          md->pxn + last * H, 1, H, s)))
            return st;
        if ((st = swiglu_run(md->ctx, L.gate, L.up, L.down, md->pxn + last * H, RQ_F16, md->ph, md->py + last * H,
                             RQ_F32, 1, ws, s)))
            return st;
    }
    // the last position only: x += down projection, logits, greedy pick
    float *xl = md->px + (size_t)(n - 1) * H;
    if ((st = launch_add_rmsnorm_rows(xl, md->py + (size_t)(n - 1) * H, nullptr, 0.0f, nullptr, 1, H, s))) return st;
    if ((st = launch_gemv_decode_norm(md->lm_head, xl, md->final_norm, c.norm_eps, md->logits, s)) != RQ_OK)
        return st;
    hipLaunchKernelGGL(k_set_position, dim3(1), dim3(1), 0, s, md->pos, md->n_prompt, p0 + n - 1, p0 + n);
    RQ_LAUNCH_CHECK();
    hipLaunchKernelGGL(k_argmax_embed, dim3(1), dim3(AT), 0, s, md->logits, c.vocab, md->embed, H, md->tokens, md->pos,
                       md->n_prompt, md->x);
    RQ_LAUNCH_CHECK();
    return RQ_OK;
}

// Decode steps per replay of the multi-step graph: the steps are device-driven
// (position and token live in device memory), so one graph may hold several,
// which saves the gap between consecutive graph launches (~3-4 us each).
// 1.1B, 128 steps, tok/s: one step per graph 2006.7, two 2019.4, four 2022.4,
// eight 2018.0 (same box, two alternations).
constexpr int kGraphSteps = 4;

// Captures `steps` decode steps into a graph on stream s and instantiates it.
static int capture_steps(rq_llama *md, int steps, hipStream_t s, hipGraph_t *graph, hipGraphExec_t *exec) {
    RQ_HIP_TRY(hipStreamBeginCapture(s, hipStreamCaptureModeThreadLocal));
    int st = RQ_OK;
    for (int i = 0; i < steps && st == RQ_OK; ++i) st = enqueue_step(md, s);
    hipGraph_t g = nullptr;
    const hipError_t e = hipStreamEndCapture(s, &g);
    if (st != RQ_OK || e != hipSuccess) {
        if (g) (void)hipGraphDestroy(g);
        return st != RQ_OK ? st : fail(RQ_ERR_HIP, "hipStreamEndCapture: %s", hipGetErrorString(e));
    }
    hipGraphExec_t x = nullptr;
    const hipError_t ei = hipGraphInstantiate(&x, g, nullptr, nullptr, 0);
    if (ei != hipSuccess) {
        (void)hipGraphDestroy(g);
        return fail(RQ_ERR_HIP, "hipGraphInstantiate: %s", hipGetErrorString(ei));
    }
    *graph = g;
    *exec = x;
    return RQ_OK;
}

// Captures the one-step graph, the first time a step runs in graph mode (a
// runner that steps eagerly never captures one), and the kGraphSteps-step
// graph the first time a run has that many steps.  The step's kernels use no
// context workspace, so the graphs may be replayed on any stream.
int ensure_graph(rq_llama *md, hipStream_t s, int n) {
    if (!md->exec) {
        const int st = capture_steps(md, 1, s, &md->graph, &md->exec);
        if (st != RQ_OK) return st;
    }
    if (n >= kGraphSteps && !md->exec_k) return capture_steps(md, kGraphSteps, s, &md->graph_k, &md->exec_k);
    return RQ_OK;
}

int run_steps(rq_llama *md, int n, hipStream_t s) {
    if (!md->use_graph) {
        for (int i = 0; i < n; ++i) {
            const int st = enqueue_step(md, s);
            if (st != RQ_OK) return st;
        }
        return RQ_OK;
    }
    if (n <= 0) return RQ_OK;
    const int st = ensure_graph(md, s, n);
    if (st != RQ_OK) return st;
    int i = 0;
    for (; i + kGraphSteps <= n; i += kGraphSteps) RQ_HIP_TRY(hipGraphLaunch(md->exec_k, s));
    for (; i < n; ++i) RQ_HIP_TRY(hipGraphLaunch(md->exec, s));
    return RQ_OK;
}

void release(rq_llama *md) {
    if (md->exec) (void)hipGraphExecDestroy(md->exec);
    if (md->graph) (void)hipGraphDestroy(md->graph);
    if (md->exec_k) (void)hipGraphExecDestroy(md->exec_k);
    if (md->graph_k) (void)hipGraphDestroy(md->graph_k);
    if (md->owned) (void)hipFree(md->owned);
    delete md;
}

template <typename T>
T *carve(char *&p, size_t count) {
    T *r = reinterpret_cast<T *>(p);
    p += (count * sizeof(T) + 255) & ~size_t(255);
    return r;
}

}  // namespace
}  // namespace rq

using namespace rq;

extern "C" {

int rq_llama_create(rq_ctx *ctx, const rq_llama_config *cfg, const rq_llama_weights *w, rq_llama **out) {
    RQ_ENTER(ctx);
    if (!cfg || !w || !out) return fail(RQ_ERR_INVALID_ARGUMENT, "null argument");
    *out = nullptr;
    const rq_llama_config c = *cfg;
    if (c.n_layers < 1 || c.hidden < 1 || c.n_heads < 1 || c.n_kv_heads < 1 || c.intermediate < 1 || c.vocab < 1 ||
        c.max_seq < 1 || !(c.norm_eps >= 0.0f) || !(c.rope_theta > 0.0f))
        return fail(RQ_ERR_SHAPE, "config fields must be positive");
    if (c.head_dim != 64 && c.head_dim != 128) return fail(RQ_ERR_UNSUPPORTED, "head_dim must be 64 or 128");
    if (c.n_heads % c.n_kv_heads != 0) return fail(RQ_ERR_SHAPE, "n_heads must be a multiple of n_kv_heads");
    if (c.max_seq > kMaxSeq) return fail(RQ_ERR_UNSUPPORTED, "max_seq is limited to %d", kMaxSeq);
    if (!w->embed || !w->layers || !w->final_norm) return fail(RQ_ERR_INVALID_ARGUMENT, "null weight pointer");
    if (!aligned(w->final_norm, 16)) return fail(RQ_ERR_UNSUPPORTED, "final norm weight must be 16-byte aligned");
    const int64_t H = c.hidden, QW = (int64_t)c.n_heads * c.head_dim, KW = (int64_t)c.n_kv_heads * c.head_dim;
    const int64_t QKV = QW + 2 * KW, I = c.intermediate;
    int st;
    for (int l = 0; l < c.n_layers; ++l) {
        const rq_llama_layer &L = w->layers[l];
        if (!L.attn_norm || !L.mlp_norm) return fail(RQ_ERR_INVALID_ARGUMENT, "layer %d: null norm weight", l);
        if (!aligned(L.attn_norm, 16) || !aligned(L.mlp_norm, 16))
            return fail(RQ_ERR_UNSUPPORTED, "layer %d: norm weights must be 16-byte aligned", l);
        if ((st = check_linear(L.q, QW, H, "q_proj", l)) || (st = check_linear(L.k, KW, H, "k_proj", l)) ||
            (st = check_linear(L.v, KW, H, "v_proj", l)) || (st = check_linear(L.o, H, QW, "o_proj", l)) ||
            (st = check_linear(L.gate, I, H, "gate_proj", l)) || (st = check_linear(L.up, I, H, "up_proj", l)) ||
            (st = check_linear(L.down, H, I, "down_proj", l)) || (st = check_same(L.q, L.k, "q/k/v", l)) ||
            (st = check_same(L.q, L.v, "q/k/v", l)) || (st = check_same(L.gate, L.up, "gate/up", l)))
            return st;
    }
    if ((st = check_linear(w->lm_head, c.vocab, H, "lm_head", -1))) return st;

    rq_llama *md = new (std::nothrow) rq_llama;
    if (!md) return fail(RQ_ERR_ALLOC, "runner allocation failed");
    md->ctx = ctx;
    md->cfg = c;
    md->embed = static_cast<const _Float16 *>(w->embed);
    md->final_norm = static_cast<const _Float16 *>(w->final_norm);
    md->lm_head = w->lm_head;

    // one allocation: per layer packed [q;k;v] codes, scales (and biases),
    // then state; affine scales hold H / group entries per row
    const size_t L = (size_t)c.n_layers, kv = L * (size_t)c.n_kv_heads * c.max_seq * c.head_dim;
    auto pad = [](size_t b) { return (b + 255) & ~size_t(255); };
    std::vector<size_t> per_row(L);  // scale entries per row of each layer's q/k/v
    size_t bytes = 0;
    // Affine Linears: the prefill GEMM's scale tables (load-time preparation),
    // built here for the packed q/k/v and for any borrowed Linear that comes
    // without one.
    auto qkv_of = [&](size_t l) {
        const rq_qweight &q = w->layers[l].q;
        return rq_qweight{q.codes, q.scales, q.biases, QKV, H, q.format, q.group, nullptr};
    };
    auto table_bytes = [&](const rq_qweight &lw) { return lw.prep ? 0 : affine_prep_bytes(lw); };
    for (size_t l = 0; l < L; ++l) {
        const rq_llama_layer &src = w->layers[l];
        const rq_qweight &q = src.q;
        per_row[l] = q.format == RQ_Q_AFFINE_U8 ? (size_t)(H / q.group) : 1;
        bytes += pad((size_t)QKV * H) + pad((size_t)QKV * per_row[l] * 4) * (q.biases ? 2 : 1);
        bytes += pad(affine_prep_bytes(qkv_of(l))) + pad(table_bytes(src.o)) + pad(table_bytes(src.gate)) +
                 pad(table_bytes(src.up)) + pad(table_bytes(src.down));
    }
    // attention splits: enough blocks per head that a full cache is one tile
    // (one pass: 128 positions at head_dim 64, 64 at 128) per block, the
    // count a power of two up to 8 (the o-projection's combine serves 1, 2, 4
    // and 8); longer caches give each block several tiles
    const int pass_rows = c.head_dim == 64 ? 128 : 64;
    const int tiles = (int)cdiv(c.max_seq, pass_rows);
    const int n_split = tiles <= 1 ? 1 : (tiles <= 2 ? 2 : (tiles <= 4 ? 4 : 8));
    const size_t part_floats = (size_t)c.n_heads * n_split * (c.head_dim + 2);
    bytes += pad(H * 4) + pad(QKV * 4) + pad((size_t)c.vocab * 4) + pad(part_floats * 4) + pad(2 * I * 2) +
             2 * pad(kv * 2) + pad(((size_t)c.max_seq + 1) * 4) + 2 * pad(4) +
             pad((size_t)c.max_seq * (c.head_dim / 2) * sizeof(float2));
    // batched prompt buffers: up to kPrefillRows positions per chunk
    const int cap = (int)std::min<int64_t>(((int64_t)c.max_seq + 31) / 32 * 32, kPrefillRows);
    bytes += 2 * pad((size_t)cap * H * 4) + pad((size_t)cap * QKV * 4) + pad((size_t)cap * H * 2) +
             2 * pad((size_t)cap * QW * 2) + pad((size_t)2 * cap * I * 2);
    hipError_t e = hipMalloc(&md->owned, bytes);
    if (e != hipSuccess) {
        md->owned = nullptr;
        release(md);
        return fail(RQ_ERR_ALLOC, "hipMalloc(%zu): %s", bytes, hipGetErrorString(e));
    }
    char *p = static_cast<char *>(md->owned);
    hipStream_t s = ctx->stream;
    md->layers.resize(L);
    for (size_t l = 0; l < L; ++l) {
        const rq_llama_layer &src = w->layers[l];
        rq_llama::Layer &dst = md->layers[l];
        const size_t pr = per_row[l];
        uint8_t *codes = carve<uint8_t>(p, (size_t)QKV * H);
        float *scales = carve<float>(p, (size_t)QKV * pr);
        float *biases = src.q.biases ? carve<float>(p, (size_t)QKV * pr) : nullptr;
        const rq_qweight *parts[3] = {&src.q, &src.k, &src.v};
        size_t row = 0;
        for (const rq_qweight *pw : parts) {
            const size_t n = (size_t)pw->n_out;
            e = hipMemcpyAsync(codes + row * H, pw->codes, n * H, hipMemcpyDeviceToDevice, s);
            if (e == hipSuccess)
                e = hipMemcpyAsync(scales + row * pr, pw->scales, n * pr * 4, hipMemcpyDeviceToDevice, s);
            if (e == hipSuccess && biases)
                e = hipMemcpyAsync(biases + row * pr, pw->biases, n * pr * 4, hipMemcpyDeviceToDevice, s);
            if (e != hipSuccess) {
                release(md);
                return fail(RQ_ERR_HIP, "packing q/k/v: %s", hipGetErrorString(e));
            }
            row += n;
        }
        dst.qkv = rq_qweight{codes, scales, biases, QKV, H, src.q.format, src.q.group, nullptr};
        dst.o = src.o;
        dst.gate = src.gate;
        dst.up = src.up;
        dst.down = src.down;
        // scale tables (stream-ordered after the q/k/v packing above)
        for (rq_qweight *lw : {&dst.qkv, &dst.o, &dst.gate, &dst.up, &dst.down}) {
            const size_t tb = lw->prep ? 0 : affine_prep_bytes(*lw);
            if (tb == 0) continue;
            float *table = carve<float>(p, tb / 4);
            if ((st = launch_affine_prep(*lw, table, s)) != RQ_OK) {
                release(md);
                return st;
            }
            lw->prep = table;
        }
        dst.attn_norm = static_cast<const _Float16 *>(src.attn_norm);
        dst.mlp_norm = static_cast<const _Float16 *>(src.mlp_norm);
    }
    md->x = carve<float>(p, H);
    md->qkv_out = carve<float>(p, QKV);
    md->logits = carve<float>(p, c.vocab);
    md->part = carve<float>(p, part_floats);
    md->n_split = n_split;
    md->h = carve<_Float16>(p, 2 * I);
    md->kc = carve<_Float16>(p, kv);
    md->vc = carve<_Float16>(p, kv);
    md->tokens = carve<int>(p, (size_t)c.max_seq + 1);
    md->pos = carve<int>(p, 1);
    md->n_prompt = carve<int>(p, 1);
    md->rope = carve<float2>(p, (size_t)c.max_seq * (c.head_dim / 2));
    md->px = carve<float>(p, (size_t)cap * H);
    md->py = carve<float>(p, (size_t)cap * H);
    md->pqkv = carve<float>(p, (size_t)cap * QKV);
    md->pxn = carve<_Float16>(p, (size_t)cap * H);
    md->pq = carve<_Float16>(p, (size_t)cap * QW);
    md->patt = carve<_Float16>(p, (size_t)cap * QW);
    md->ph = carve<_Float16>(p, (size_t)2 * cap * I);
    md->prefill_cap = md->prefill_rows = cap;

    {
        const int64_t n = (int64_t)c.max_seq * (c.head_dim / 2);
        hipLaunchKernelGGL(k_rope_table, dim3((unsigned)cdiv(n, NT)), dim3(NT), 0, s, md->rope, c.max_seq, c.head_dim,
                           c.rope_theta);
        e = hipGetLastError();
        if (e != hipSuccess) {
            release(md);
            return fail(RQ_ERR_HIP, "rope table: %s", hipGetErrorString(e));
        }
    }
    e = hipStreamSynchronize(s);
    if (e != hipSuccess) {
        release(md);
        return fail(RQ_ERR_HIP, "packing q/k/v: %s", hipGetErrorString(e));
    }

    *out = md;
    return RQ_OK;
}

int rq_llama_destroy(rq_llama *md) {
    if (!md) return RQ_OK;
    RQ_ENTER(md->ctx);
    hipError_t e = hipStreamSynchronize(md->ctx->stream);
    release(md);
    if (e != hipSuccess) return fail(RQ_ERR_HIP, "hipStreamSynchronize: %s", hipGetErrorString(e));
    return RQ_OK;
}

int rq_llama_prefill(rq_llama *md, const int32_t *tokens, int32_t n, rq_stream stream) {
    if (!md) return fail(RQ_ERR_INVALID_ARGUMENT, "null runner");
    RQ_ENTER(md->ctx);
    if (!tokens) return fail(RQ_ERR_INVALID_ARGUMENT, "null tokens");
    if (n < 1 || n > md->cfg.max_seq) return fail(RQ_ERR_SHAPE, "prompt length %d outside 1..%d", n, md->cfg.max_seq);
    for (int i = 0; i < n; ++i)
        if (tokens[i] < 0 || tokens[i] >= md->cfg.vocab)
            return fail(RQ_ERR_INVALID_ARGUMENT, "token %d at %d outside the vocabulary", tokens[i], i);
    hipStream_t s = pick(md->ctx, stream);
    RQ_HIP_TRY(hipMemcpyAsync(md->tokens, tokens, (size_t)n * 4, hipMemcpyHostToDevice, s));
    RQ_HIP_TRY(hipStreamSynchronize(s));  // the host array may be released on return
    int st;
    if (md->prefill_rows > 0) {
        for (int p0 = 0; p0 < n; p0 += md->prefill_rows) {
            const int rows = std::min(md->prefill_rows, n - p0);
            if ((st = prefill_chunk(md, p0, rows, p0 + rows == n, s)) != RQ_OK) return st;
        }
    } else {
        hipLaunchKernelGGL(k_embed_start, dim3(1), dim3(NT), 0, s, md->tokens, md->embed, md->cfg.hidden, md->x,
                           md->pos, md->n_prompt, n);
        RQ_LAUNCH_CHECK();
        if ((st = run_steps(md, n, s)) != RQ_OK) return st;
    }
    md->host_pos = n;
    md->host_len = n + 1;
    return RQ_OK;
}

int rq_llama_decode(rq_llama *md, int32_t n_steps, rq_stream stream) {
    if (!md) return fail(RQ_ERR_INVALID_ARGUMENT, "null runner");
    RQ_ENTER(md->ctx);
    if (md->host_len == 0) return fail(RQ_ERR_INVALID_ARGUMENT, "no sequence: call rq_llama_prefill first");
    if (n_steps < 0 || n_steps > md->cfg.max_seq - md->host_pos)
        return fail(RQ_ERR_SHAPE, "%d steps from position %d exceed max_seq %d", n_steps, md->host_pos,
                    md->cfg.max_seq);
    hipStream_t s = pick(md->ctx, stream);
    int st;
    if ((st = run_steps(md, n_steps, s)) != RQ_OK) return st;
    md->host_pos += n_steps;
    md->host_len += n_steps;
    return RQ_OK;
}

int rq_llama_set_graph(rq_llama *md, int use_graph) {
    if (!md) return fail(RQ_ERR_INVALID_ARGUMENT, "null runner");
    RQ_ENTER(md->ctx);
    md->use_graph = use_graph != 0;
    return RQ_OK;
}

int rq_llama_set_prefill(rq_llama *md, int32_t rows) {
    if (!md) return fail(RQ_ERR_INVALID_ARGUMENT, "null runner");
    RQ_ENTER(md->ctx);
    if (rows < 0 || rows % 32 != 0 || rows > md->prefill_cap)
        return fail(RQ_ERR_SHAPE, "prefill chunk of %d rows: 0 or a multiple of 32 up to %d", rows, md->prefill_cap);
    md->prefill_rows = rows;
    return RQ_OK;
}

int rq_llama_tokens(rq_llama *md, int32_t *out, int32_t capacity, int32_t *length, rq_stream stream) {
    if (!md) return fail(RQ_ERR_INVALID_ARGUMENT, "null runner");
    RQ_ENTER(md->ctx);
    if (!length || (capacity > 0 && !out)) return fail(RQ_ERR_INVALID_ARGUMENT, "null output");
    *length = md->host_len;
    const int n = capacity < md->host_len ? capacity : md->host_len;
    if (n <= 0) return RQ_OK;
    hipStream_t s = pick(md->ctx, stream);
    RQ_HIP_TRY(hipMemcpyAsync(out, md->tokens, (size_t)n * 4, hipMemcpyDeviceToHost, s));
    RQ_HIP_TRY(hipStreamSynchronize(s));
    return RQ_OK;
}

int rq_llama_logits(rq_llama *md, float *out, rq_stream stream) {
    if (!md) return fail(RQ_ERR_INVALID_ARGUMENT, "null runner");
    RQ_ENTER(md->ctx);
    if (!out) return fail(RQ_ERR_INVALID_ARGUMENT, "null output");
    hipStream_t s = pick(md->ctx, stream);
    RQ_HIP_TRY(hipMemcpyAsync(out, md->logits, (size_t)md->cfg.vocab * 4, hipMemcpyDeviceToHost, s));
    RQ_HIP_TRY(hipStreamSynchronize(s));
    return RQ_OK;
}

}  // extern "C"
