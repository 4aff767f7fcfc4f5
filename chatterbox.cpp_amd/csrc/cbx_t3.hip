// cbx_t3.hip -- one decode step of the T3 transformer (GPT-2) for n streams,
// each at its own position with its own KV cache: the step graph of
// src/main.cpp:617-633 through build_transformer_core (main.cpp:469-575),
// up to ln_f's output.
//
// Per step, for every stream row:
//   x  = speech_emb[token] + wpe[pos]                       (main.cpp:628-630)
//   per layer l:
//     u   = LN(x) * ln_1_g + ln_1_b                          (:522-523)
//     qkv = c_attn u + b                                     (:524)
//     k, v of this position appended to the stream's cache   (:517-531)
//     a   = softmax(q . K^T / sqrt(64)) V over [0, pos]      (:542-548, N = 1)
//     x  += c_proj a + b                                     (:551)
//     u   = LN(x) * ln_2_g + ln_2_b                          (:554-555)
//     x  += mlp_proj gelu(mlp_fc u + b) + b                  (:556-559)
//   hidden = LN(x) * ln_f_g + ln_f_b                         (:562-563)
// LN(x) = (x - mean) / sqrt(var + eps), var the mean square of x - mean
// (ggml_norm); gelu the tanh form 0.5 x (1 + tanh(sqrt(2/pi) x (1 +
// 0.044715 x^2))) (Hendrycks and Gimpel's approximation, ggml_gelu's).
//
// The four matrix products of a layer have the speech_head's shape (rows of
// n_in weights per output, F16 / Q4_0 / Q5_0 / Q8_0): they run on the head's
// kernels (fp16 matrix cores on split activations from 16 rows, a mat-vec
// below).  From 16 rows the layer norms write the split activations of the
// products they feed themselves, and the two products the residual adds
// take a K split over workgroups when their grid is narrow, their slabs
// added by the norm that follows; gelu is applied as the mlp c_fc product
// stores its outputs.  The kernels here are the row-wise rest: the
// embedding, the residual add fused with the next layer norm, and the
// attention with its cache append (a workgroup of 4 waves per stream and
// head, 16 when there are few).
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>

#include "cbx_internal.h"
#include "cbx_split.h"
#include "../../include/cbx_t3.h"

namespace cbx {
namespace {

constexpr int kNormThreads = 256;
constexpr int kHeadDim = 64;
// Products split over K write up to this many slabs.
constexpr int kMaxKSplit = 8;

struct NormArgs {
    int32_t n_embd;
    float eps;
    float* x;              // residual rows [n_rows][n_embd], in/out
    const float* y;        // when set, the ny slabs y + z * ystride (a product
    int32_t ny;            //   split over K, in slab order) are added to x
    int64_t ystride;
    // embedding mode (emb set): x = emb[token] + wpe[pos], or x = inputs[r]
    const float* emb;
    const float* wpe;
    const float* inputs;
    const int32_t* tokens;
    int32_t* positions;
    const int32_t* state;
    const int32_t* slots;  // prefill: the cache slot of each row (NULL: the row)
    int32_t n_slots;
    int32_t n_vocab, n_pos, n_ctx;
    int32_t* act;          // per row: 1 when the stream takes this step
    const float* g;
    const float* b;
    float* out;            // LN(x) * g + b
    uint32_t* parts;       // when set, LN(x) * g + b goes there instead, split
    float* inv;            //   for the next product (cbx_split.h), the scales here
    int32_t advance;       // last norm of the step: positions[r] += 1
};

// One row per workgroup: the embedding or the residual add, then the layer
// norm.  Inactive rows (streams that take no step) keep x and write zeros.
// The next product's split activations for row r from its values in LDS: 8
// consecutive values per group, groups tid, tid + 256, ..., each block's
// scale from the largest magnitude of its 4 groups (4 consecutive threads).
__device__ __forceinline__ void norm_split(const NormArgs& a, int r, const float* row_s) {
    const int n = a.n_embd, tid = threadIdx.x, nball = n / 32;
    for (int j0 = 0; j0 < n / 8; j0 += kNormThreads) {  // whole waves in or out
        const int j = j0 + tid;
        if (j0 + (tid & ~63) >= n / 8) break;
        float v[8];
        float mx = 0.0f;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            v[i] = j < n / 8 ? row_s[8 * j + i] : 0.0f;
            mx = fmaxf(mx, fabsf(v[i]));
        }
        mx = split_block_max4(mx);
        if (j >= n / 8) continue;
        float sc, sinv;
        split_scale(mx, sc, sinv);
        split_store(a.parts, r >> 4, r & 15, nball, j, v, sc);
        if ((j & 3) == 0) a.inv[split_inv_index(r >> 4, r & 15, nball, j >> 2)] = sinv;
    }
}

template <int EPT>
__global__ __launch_bounds__(kNormThreads) void t3_norm(NormArgs a) {
    __shared__ float red[8];
    __shared__ float row_s[EPT * kNormThreads];
    int ph = 0;
    const int r = blockIdx.x, tid = threadIdx.x;
    const int n = a.n_embd;
    float* xr = a.x + (int64_t)r * n;
    float* orow = a.out + (int64_t)r * n;
    bool active;
    float xv[EPT];
    if (a.emb || a.inputs) {
        const int pos = a.positions[r];
        const int tok = a.tokens ? a.tokens[r] : 0;
        const int slot = a.slots ? a.slots[r] : r;
        active = (!a.state || a.state[r] == CBX_DECODE_RUNNING) && pos >= 0 && pos < a.n_ctx &&
                 pos < a.n_pos && (a.inputs || (tok >= 0 && tok < a.n_vocab)) &&
                 (!a.slots || (slot >= 0 && slot < a.n_slots));
        if (tid == 0) a.act[r] = active ? 1 : 0;
        if (!active) {
#pragma unroll
            for (int j = 0; j < EPT; ++j) {
                xr[j * kNormThreads + tid] = 0.0f;
                row_s[j * kNormThreads + tid] = 0.0f;
                if (!a.parts) orow[j * kNormThreads + tid] = 0.0f;
            }
            if (a.parts) {
                __syncthreads();
                norm_split(a, r, row_s);
            }
            return;
        }
        if (a.inputs) {
            const float* in = a.inputs + (int64_t)r * n;
#pragma unroll
            for (int j = 0; j < EPT; ++j) xv[j] = in[j * kNormThreads + tid];
        } else {
            const float* e = a.emb + (int64_t)tok * n;
            const float* p = a.wpe + (int64_t)pos * n;
#pragma unroll
            for (int j = 0; j < EPT; ++j)
                xv[j] = __fadd_rn(e[j * kNormThreads + tid], p[j * kNormThreads + tid]);
        }
    } else {
        active = a.act[r] != 0;
        if (!active) {
#pragma unroll
            for (int j = 0; j < EPT; ++j) {
                row_s[j * kNormThreads + tid] = 0.0f;
                if (!a.parts) orow[j * kNormThreads + tid] = 0.0f;
            }
            if (a.parts) {
                __syncthreads();
                norm_split(a, r, row_s);
            }
            return;
        }
        // the product's slabs (all loads issued first), added in slab order,
        // then the residual (main.cpp:551, :559)
        float ys[kMaxKSplit][EPT];
#pragma unroll
        for (int j = 0; j < EPT; ++j) xv[j] = xr[j * kNormThreads + tid];
        if (a.y) {
            const float* yr = a.y + (int64_t)r * n + tid;
#pragma unroll
            for (int z = 0; z < kMaxKSplit; ++z)
#pragma unroll
                for (int j = 0; j < EPT; ++j)
                    ys[z][j] = z < a.ny ? yr[z * a.ystride + j * kNormThreads] : 0.0f;
#pragma unroll
            for (int j = 0; j < EPT; ++j) {
                float c = ys[0][j];
#pragma unroll
                for (int z = 1; z < kMaxKSplit; ++z)
                    if (z < a.ny) c = __fadd_rn(c, ys[z][j]);
                xv[j] = __fadd_rn(c, xv[j]);
            }
        }
    }
    float s = 0.0f;
#pragma unroll
    for (int j = 0; j < EPT; ++j) s = __fadd_rn(s, xv[j]);
    const float mean = __fdiv_rn(block_sum256(s, red, ph), (float)n);
    float q = 0.0f;
#pragma unroll
    for (int j = 0; j < EPT; ++j) {
        const float d = __fsub_rn(xv[j], mean);
        q = __fadd_rn(q, __fmul_rn(d, d));
    }
    const float var = __fdiv_rn(block_sum256(q, red, ph), (float)n);
    const float scale = __fdiv_rn(1.0f, __fsqrt_rn(__fadd_rn(var, a.eps)));
#pragma unroll
    for (int j = 0; j < EPT; ++j) {
        const int i = j * kNormThreads + tid;
        xr[i] = xv[j];
        const float o =
            __fadd_rn(__fmul_rn(__fmul_rn(__fsub_rn(xv[j], mean), scale), a.g[i]), a.b[i]);
        if (a.parts)
            row_s[i] = o;
        else
            orow[i] = o;
    }
    if (a.parts) {
        __syncthreads();  // row_s complete
        norm_split(a, r, row_s);
    }
    if (a.advance && tid == 0) a.positions[r] += 1;
}

struct AttnArgs {
    const float* qkv;      // [n_rows][3 n_embd]: q | k | v, head h at h*64
    float* kc;             // this layer's caches: stream r, head h at
    float* vc;             //   ((r * n_layer + layer) * n_head + h) * n_ctx * 64
    int32_t n_layer, layer, n_head, n_ctx;
    const int32_t* positions;
    const int32_t* act;
    const int32_t* slots;  // prefill: the cache slot of each row (NULL: the row)
    int32_t appended;      // the rows' k, v already stored (t3_kv_append)
    float* out;            // [n_rows][n_embd]
    uint32_t* parts;       // when set, the rows go there instead, split for the
    float* inv;            //   next product (cbx_split.h), the scales here
    float scale;           // 1 / sqrt(64)
};

// Element `lane` (0..63) of head h of row r's attention output, o, from wave
// 0: to out, or split (the head's 64 values are blocks 2h and 2h + 1 of the
// row: lanes 0-31 and 32-63, each block scaled by its own largest magnitude,
// pairs of lanes joining their fp16 halves into dwords).
__device__ __forceinline__ void attn_store(const AttnArgs& a, int r, int h, int lane, float o) {
    const int n = a.n_head * kHeadDim;
    if (!a.parts) {
        a.out[(int64_t)r * n + h * kHeadDim + lane] = o;
        return;
    }
    float mx = fabsf(o);
#pragma unroll
    for (int q = 1; q < 32; q <<= 1) mx = fmaxf(mx, __shfl_xor(mx, q));
    float sc, sinv;
    split_scale(mx, sc, sinv);
    const float y = __fmul_rn(o, sc);
    const _Float16 hh = (_Float16)y;
    const _Float16 ll = (_Float16)__fsub_rn(y, (float)hh);
    const uint32_t hv = __builtin_bit_cast(uint16_t, hh), lv = __builtin_bit_cast(uint16_t, ll);
    const uint32_t ho = (uint32_t)__shfl_xor((int)hv, 1), lo = (uint32_t)__shfl_xor((int)lv, 1);
    const int nball = n / 32, kb = 2 * h + (lane >> 5), k = lane & 31;
    const int T = r >> 4, m = r & 15;
    if ((lane & 1) == 0) {
        // dword (k % 8) / 2 of lane 16 (k / 8) + m's hi (lo) 16 bytes
        uint32_t* const base =
            a.parts + ((int64_t)T * nball + kb) * 512 + 4 * (16 * (k >> 3) + m) + (k & 7) / 2;
        base[0] = hv | (ho << 16);
        base[256] = lv | (lo << 16);
    }
    if (k == 0) a.inv[split_inv_index(T, m, nball, kb)] = sinv;
}

// Prefill: every row's k and v stored at its slot and position before any
// row attends, so rows of one stream in one call see each other causally.
__global__ __launch_bounds__(kHeadDim) void t3_kv_append(AttnArgs a) {
    const int r = blockIdx.x, h = blockIdx.y, lane = threadIdx.x;
    if (!a.act[r]) return;
    const int n = a.n_head * kHeadDim;
    const int slot = a.slots ? a.slots[r] : r, pos = a.positions[r];
    const float* qr = a.qkv + (int64_t)r * 3 * n + h * kHeadDim;
    const int64_t base =
        (((int64_t)slot * a.n_layer + a.layer) * a.n_head + h) * a.n_ctx * kHeadDim + (int64_t)pos * kHeadDim;
    a.kc[base + lane] = qr[n + lane];
    a.vc[base + lane] = qr[2 * n + lane];
}

// One workgroup of kAttnWaves waves per (stream, head).  Wave 0 stores the
// new k and v at the stream's position (and keeps them in LDS: that position
// is never read back from memory).  The positions are cut into
// kAttnWaves runs, one per wave; a wave's lanes take 16 per cache row, 4 rows
// per load instruction, kAttnBatch rows per lane in flight, and go over the
// run once with a running softmax (max, sum, weighted v sums, rescaled as the
// max grows); the runs of the 4 row groups of a wave and of the waves are
// merged by the same rescaling in a fixed order.  Decode steps run 4 waves x
// 6 rows (every workgroup resident at once; 16 waves when rows x heads are
// under 256, see t3_attn_wide), the prompt pass 2 waves x 8 rows
// (many more workgroups: smaller ones keep more of them resident); measured
// at 64 streams 1.89 -> 1.85 ms per step against 4 x 8, and the prompt of
// 64 x 256 positions 93.8 -> 82.2 ms.
template <int kAttnBatch, int kAttnWaves>
__global__ __launch_bounds__(kAttnWaves * kHeadDim) void t3_attn(AttnArgs a) {
    __shared__ __align__(16) float kn_s[kHeadDim];
    __shared__ __align__(16) float vn_s[kHeadDim];
    __shared__ float red[2 * kAttnWaves];
    __shared__ __align__(16) float part[kAttnWaves][kHeadDim];
    const int r = blockIdx.x, h = blockIdx.y, tid = threadIdx.x;
    const int lane = tid & 63, w = tid >> 6;
    const int n = a.n_head * kHeadDim;
    if (!a.act[r]) {
        if (tid < kHeadDim) attn_store(a, r, h, tid, 0.0f);
        return;
    }
    const int pos = a.positions[r];
    const int slot = a.slots ? a.slots[r] : r;
    const float* qr = a.qkv + (int64_t)r * 3 * n + h * kHeadDim;
    const int64_t base = (((int64_t)slot * a.n_layer + a.layer) * a.n_head + h) * a.n_ctx * kHeadDim;
    float* kc = a.kc + base;
    float* vc = a.vc + base;
    if (w == 0) {
        const float kn = qr[n + lane], vn = qr[2 * n + lane];
        if (!a.appended) {
            kc[(int64_t)pos * kHeadDim + lane] = kn;
            vc[(int64_t)pos * kHeadDim + lane] = vn;
        }
        kn_s[lane] = kn;
        vn_s[lane] = vn;
    }
    // lane = 16 sub + e holds q[4e .. 4e + 3] and takes position c0 + sub + 4i,
    // dimensions 4e .. 4e + 3: a wave reads 4 rows of k per instruction
    const int sub = lane >> 4, e4 = 4 * (lane & 15);
    const float4 q4 = *reinterpret_cast<const float4*>(qr + e4);
    // positions [0, L) in kAttnWaves runs
    const int L = pos + 1;
    const int run = (L + kAttnWaves - 1) / kAttnWaves;
    const int c0 = min(w * run, L), c1 = min(c0 + run, L);
    __syncthreads();
    // Each lane keeps, over the positions of its 16-lane group (position order),
    // the running max m of the scores, the sum s of expf(score - m) and the
    // sums acc of expf(score - m) v[4e .. 4e + 3], rescaled whenever m grows
    // (one pass: k and v rows of a batch are loaded together, kAttnBatch per
    // lane, a row past the run reading the run's last row, unused; the new
    // position's k and v are taken from LDS, their stores above need not be
    // visible).
    const float4 kn4 = *reinterpret_cast<const float4*>(kn_s + e4);
    const float4 vn4 = *reinterpret_cast<const float4*>(vn_s + e4);
    float m = -INFINITY, s = 0.0f;
    float4 acc = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    for (int j0 = c0; j0 < c1; j0 += 4 * kAttnBatch) {
        float4 kk[kAttnBatch], vv[kAttnBatch];
#pragma unroll
        for (int u = 0; u < kAttnBatch; ++u) {
            const int64_t jc = min(j0 + 4 * u + sub, c1 - 1);
            kk[u] = *reinterpret_cast<const float4*>(kc + jc * kHeadDim + e4);
            vv[u] = *reinterpret_cast<const float4*>(vc + jc * kHeadDim + e4);
        }
        float sc[kAttnBatch];
        float bm = -INFINITY;
#pragma unroll
        for (int u = 0; u < kAttnBatch; ++u) {
            const int j = j0 + 4 * u + sub;
            const float4 k4 = j == pos ? kn4 : kk[u];
            float dot = __fadd_rn(__fadd_rn(__fmul_rn(q4.x, k4.x), __fmul_rn(q4.y, k4.y)),
                                  __fadd_rn(__fmul_rn(q4.z, k4.z), __fmul_rn(q4.w, k4.w)));
            // the 16 lanes of a row: butterfly over e (the same sum in each)
            dot = sum16_dpp(dot);
            sc[u] = __fmul_rn(dot, a.scale);
            if (j < c1) bm = fmaxf(bm, sc[u]);
        }
        if (bm > m) {
            const float f = m == -INFINITY ? 0.0f : expf(__fsub_rn(m, bm));
            s = __fmul_rn(s, f);
            acc.x = __fmul_rn(acc.x, f);
            acc.y = __fmul_rn(acc.y, f);
            acc.z = __fmul_rn(acc.z, f);
            acc.w = __fmul_rn(acc.w, f);
            m = bm;
        }
#pragma unroll
        for (int u = 0; u < kAttnBatch; ++u) {
            const int j = j0 + 4 * u + sub;
            if (j < c1) {
                const float e = expf(__fsub_rn(sc[u], m));
                const float4 v4 = j == pos ? vn4 : vv[u];
                s = __fadd_rn(s, e);
                acc.x = __fadd_rn(acc.x, __fmul_rn(e, v4.x));
                acc.y = __fadd_rn(acc.y, __fmul_rn(e, v4.y));
                acc.z = __fadd_rn(acc.z, __fmul_rn(e, v4.z));
                acc.w = __fadd_rn(acc.w, __fmul_rn(e, v4.w));
            }
        }
    }
    // the 4 groups of a wave, then the 4 waves, merged by the same rescaling:
    // each pair's two products added in either lane give the same sum
#pragma unroll
    for (int o = 16; o <= 32; o <<= 1) {
        const float mo = __shfl_xor(m, o), so = __shfl_xor(s, o);
        const float4 ao = make_float4(__shfl_xor(acc.x, o), __shfl_xor(acc.y, o),
                                      __shfl_xor(acc.z, o), __shfl_xor(acc.w, o));
        const float M = fmaxf(m, mo);
        const float f = m == -INFINITY ? 0.0f : expf(__fsub_rn(m, M));
        const float fo = mo == -INFINITY ? 0.0f : expf(__fsub_rn(mo, M));
        s = __fadd_rn(__fmul_rn(s, f), __fmul_rn(so, fo));
        acc.x = __fadd_rn(__fmul_rn(acc.x, f), __fmul_rn(ao.x, fo));
        acc.y = __fadd_rn(__fmul_rn(acc.y, f), __fmul_rn(ao.y, fo));
        acc.z = __fadd_rn(__fmul_rn(acc.z, f), __fmul_rn(ao.z, fo));
        acc.w = __fadd_rn(__fmul_rn(acc.w, f), __fmul_rn(ao.w, fo));
        m = M;
    }
    if (lane == 0) {
        red[w] = m;
        red[kAttnWaves + w] = s;
    }
    if (sub == 0) *reinterpret_cast<float4*>(&part[w][e4]) = acc;
    __syncthreads();
    if (w == 0) {
        float M = red[0];
#pragma unroll
        for (int q = 1; q < kAttnWaves; ++q) M = fmaxf(M, red[q]);
        float st = 0.0f, at = 0.0f;
#pragma unroll
        for (int q = 0; q < kAttnWaves; ++q) {
            const float f = red[q] == -INFINITY ? 0.0f : expf(__fsub_rn(red[q], M));
            st = __fadd_rn(st, __fmul_rn(red[kAttnWaves + q], f));
            at = __fadd_rn(at, __fmul_rn(part[q][lane], f));
        }
        attn_store(a, r, h, lane, __fdiv_rn(at, st));
    }
}

template <int EPT>
hipError_t launch_norm_ept(const NormArgs& a, int n_rows, hipStream_t st) {
    hipLaunchKernelGGL(t3_norm<EPT>, dim3((unsigned)n_rows), dim3(kNormThreads), 0, st, a);
    return hipGetLastError();
}

hipError_t launch_norm(const NormArgs& a, int n_rows, hipStream_t st) {
    switch (a.n_embd / kNormThreads) {
        case 1: return launch_norm_ept<1>(a, n_rows, st);
        case 2: return launch_norm_ept<2>(a, n_rows, st);
        case 3: return launch_norm_ept<3>(a, n_rows, st);
        case 4: return launch_norm_ept<4>(a, n_rows, st);
        case 6: return launch_norm_ept<6>(a, n_rows, st);
        case 8: return launch_norm_ept<8>(a, n_rows, st);
        case 12: return launch_norm_ept<12>(a, n_rows, st);
        case 16: return launch_norm_ept<16>(a, n_rows, st);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace

bool t3_shape_ok(int32_t n_embd, int32_t n_head) {
    const int e = n_embd / kNormThreads;
    return n_head >= 1 && n_embd == n_head * kHeadDim && n_embd % kNormThreads == 0 &&
           (e == 1 || e == 2 || e == 3 || e == 4 || e == 6 || e == 8 || e == 12 || e == 16);
}

size_t t3_attn_lds(int32_t) { return 0; }  // one pass: no per-position LDS

// Decode steps whose grid of rows x heads is small run 16 waves per (row,
// head) instead of 4, so the few workgroups still spread each stream's
// positions over many waves (measured at one stream, 16 heads: 0.91 ->
// 0.86 ms per step against 4 waves with the positions split over 16
// workgroups and merged by a second kernel).
bool t3_attn_wide(int32_t n_rows, int32_t n_head) { return (int64_t)n_rows * n_head < 256; }

// Workspace of a step: x, u, a [n_rows][n_embd], y [kMaxKSplit][n_rows][n_embd],
// qkv [n_rows][3 n_embd], f [n_rows][4 n_embd], act [n_rows], then two
// buffers of split activations for the matrix products (each for the widest
// input, 4 n_embd): the norms and the attention write the first, the mlp's
// c_fc the second (c_fc reads the first as it writes).

size_t t3_workspace_bytes(int32_t n_rows, int32_t n_embd) {
    const size_t row = (size_t)n_rows * n_embd * 4;
    const size_t body = (3 + kMaxKSplit) * row + 3 * row + 4 * row +
                        ((size_t)n_rows * 4 + 255) / 256 * 256;
    const size_t sp = (head_scratch_bytes(n_rows, false, 4 * n_embd) + 255) / 256 * 256;
    return body + 2 * sp;
}

hipError_t launch_t3_step(const cbx_t3_model& m, int32_t n_rows, const int32_t* tokens,
                          const float* inputs, int32_t* positions, const int32_t* state,
                          const int32_t* slots, int32_t n_slots, const cbx_t3_cache& c,
                          float* hidden, void* ws, hipStream_t st) {
    // slots set: a prefill (rows of one stream may share a call: their k and v
    // are stored before the attention, and positions do not advance)
    const bool prefill = slots != nullptr;
    const int n = m.n_embd;
    const size_t row = (size_t)n_rows * n;
    float* x = static_cast<float*>(ws);
    float* u = x + row;
    float* att = u + row;
    float* y = att + row;
    float* qkv = y + kMaxKSplit * row;
    float* f = qkv + 3 * row;
    int32_t* act = reinterpret_cast<int32_t*>(f + 4 * row);
    const bool wide = !prefill && t3_attn_wide(n_rows, m.n_head);
    void* split = reinterpret_cast<char*>(act) + ((size_t)n_rows * 4 + 255) / 256 * 256;
    void* split2 = static_cast<char*>(split) +
                   (head_scratch_bytes(n_rows, false, 4 * n) + 255) / 256 * 256;

    NormArgs na{};
    na.n_embd = n;
    na.eps = m.eps;
    na.x = x;
    na.emb = inputs ? nullptr : m.speech_emb;
    na.wpe = m.wpe;
    na.inputs = inputs;
    na.tokens = inputs ? nullptr : tokens;
    na.positions = positions;
    na.state = state;
    na.slots = slots;
    na.n_slots = n_slots;
    na.n_vocab = m.n_speech_vocab;
    na.n_pos = m.n_pos;
    na.n_ctx = c.n_ctx;
    na.act = act;
    na.g = m.layers[0].ln_1_g;
    na.b = m.layers[0].ln_1_b;
    na.out = u;
    // 16 streams and more (the matrix-core path): every product's input is
    // written split by its producer (the norms, the attention, c_fc); below,
    // plain rows for the mat-vec
    const bool mc = !head_uses_gemv(n_rows, false, n);
    uint32_t* const sparts = static_cast<uint32_t*>(split);
    float* const sinv = reinterpret_cast<float*>(static_cast<char*>(split) +
                                                 split_inv_offset(16 * ((n_rows + 15) / 16), n));
    na.parts = mc ? sparts : nullptr;
    na.inv = sinv;
    hipError_t e = launch_norm(na, n_rows, st);
    if (e != hipSuccess) return e;

    AttnArgs aa{};
    aa.qkv = qkv;
    aa.kc = c.k;
    aa.vc = c.v;
    aa.n_layer = m.n_layer;
    aa.n_head = m.n_head;
    aa.n_ctx = c.n_ctx;
    aa.positions = positions;
    aa.act = act;
    aa.slots = slots;
    aa.appended = prefill ? 1 : 0;
    aa.out = att;
    aa.parts = mc ? sparts : nullptr;  // c_attn has read them by then
    aa.inv = sinv;
    aa.scale = 0.125f;  // 1 / sqrt(64)
    const size_t lds = t3_attn_lds(c.n_ctx);

    const int kz_a = min(head_k_split(n_rows, n, n), kMaxKSplit);
    const int kz_f = min(head_k_split(n_rows, n, 4 * n), kMaxKSplit);
    // one or two streams: the residual adds and norms between the layer's
    // products run inside the mat-vec that consumes them (c_fc, and the next
    // layer's c_attn), the residual rows alternating between x and y's
    // second slab (the mat-vec products take no K split)
    const bool fold = !mc && n_rows <= 2 && kz_a == 1 && kz_f == 1;
    float* xcur = x;
    float* const xalt = y + row;
    GemvNorm gn{};
    gn.y = y;
    gn.act = act;
    gn.eps = m.eps;
    for (int l = 0; l < m.n_layer; ++l) {
        const cbx_t3_layer& L = m.layers[l];
        if (mc) {
            e = launch_head_presplit(L.attn_w, m.wtype, L.attn_b, qkv, 3 * n, n_rows, 3 * n, n,
                                     split, st, 1, false);
        } else if (fold && l > 0) {  // the previous layer's residual + this ln_1
            gn.x_in = xcur;
            gn.x_out = xcur = xcur == x ? xalt : x;
            gn.g = L.ln_1_g;
            gn.b = L.ln_1_b;
            e = launch_head_gemv_norm(L.attn_w, m.wtype, L.attn_b, gn, qkv, 3 * n, n_rows, 3 * n,
                                      n, st, false);
        } else {
            e = launch_head(L.attn_w, m.wtype, L.attn_b, u, nullptr, n, qkv, nullptr, 3 * n,
                            n_rows, 3 * n, n, split, st);
        }
        if (e != hipSuccess) return e;
        aa.layer = l;
        if (prefill) {
            hipLaunchKernelGGL(t3_kv_append, dim3((unsigned)n_rows, (unsigned)m.n_head),
                               dim3(kHeadDim), 0, st, aa);
            if ((e = hipGetLastError()) != hipSuccess) return e;
        }
        if (prefill)
            hipLaunchKernelGGL((t3_attn<8, 2>), dim3((unsigned)n_rows, (unsigned)m.n_head),
                               dim3(2 * kHeadDim), lds, st, aa);
        else if (wide)
            hipLaunchKernelGGL((t3_attn<6, 16>), dim3((unsigned)n_rows, (unsigned)m.n_head),
                               dim3(16 * kHeadDim), lds, st, aa);
        else
            hipLaunchKernelGGL((t3_attn<6, 4>), dim3((unsigned)n_rows, (unsigned)m.n_head),
                               dim3(4 * kHeadDim), lds, st, aa);
        if ((e = hipGetLastError()) != hipSuccess) return e;
        // the two products the residual adds take a K split when their grid
        // is narrow (the norm adds the slabs)
        e = mc ? launch_head_presplit(L.attn_proj_w, m.wtype, L.attn_proj_b, y, n, n_rows, n, n,
                                      split, st, kz_a, false)
               : launch_head_k(L.attn_proj_w, m.wtype, L.attn_proj_b, att, nullptr, n, y, nullptr,
                               n, n_rows, n, n, split, st, kz_a, false);
        if (e != hipSuccess) return e;
        NormArgs nb{};
        nb.n_embd = n;
        nb.eps = m.eps;
        nb.x = xcur;
        nb.y = y;
        nb.ny = kz_a;
        nb.ystride = (int64_t)row;
        nb.act = act;
        nb.g = L.ln_2_g;
        nb.b = L.ln_2_b;
        nb.out = u;
        nb.parts = mc ? sparts : nullptr;
        nb.inv = sinv;
        // gelu applied as the mlp rows are stored
        if (fold) {  // the residual + ln_2 inside c_fc
            gn.x_in = xcur;
            gn.x_out = xcur = xcur == x ? xalt : x;
            gn.g = L.ln_2_g;
            gn.b = L.ln_2_b;
            e = launch_head_gemv_norm(L.fc_w, m.wtype, L.fc_b, gn, f, 4 * n, n_rows, 4 * n, n, st,
                                      true);
        } else {
            if ((e = launch_norm(nb, n_rows, st)) != hipSuccess) return e;
            e = mc ? launch_head_presplit(L.fc_w, m.wtype, L.fc_b, f, 4 * n, n_rows, 4 * n, n,
                                          split, st, 1, true, split2)
                   : launch_head_k(L.fc_w, m.wtype, L.fc_b, u, nullptr, n, f, nullptr, 4 * n,
                                   n_rows, 4 * n, n, split, st, 1, true);
        }
        if (e != hipSuccess) return e;
        e = mc ? launch_head_presplit(L.fc_proj_w, m.wtype, L.fc_proj_b, y, n, n_rows, n, 4 * n,
                                      split2, st, kz_f, false)
               : launch_head_k(L.fc_proj_w, m.wtype, L.fc_proj_b, f, nullptr, 4 * n, y, nullptr, n,
                               n_rows, n, 4 * n, split, st, kz_f, false);
        if (e != hipSuccess) return e;
        // the residual, then the next layer's ln_1 or, after the last, ln_f
        // into `hidden` and the positions advanced
        const bool last = l + 1 == m.n_layer;
        if (fold && !last) continue;  // inside the next layer's c_attn
        NormArgs nc = nb;
        nc.x = xcur;
        nc.ny = kz_f;
        nc.g = last ? m.ln_f_g : m.layers[l + 1].ln_1_g;
        nc.b = last ? m.ln_f_b : m.layers[l + 1].ln_1_b;
        nc.out = last ? hidden : u;
        nc.parts = mc && !last ? sparts : nullptr;
        nc.positions = positions;
        nc.advance = last && !prefill ? 1 : 0;
        if ((e = launch_norm(nc, n_rows, st)) != hipSuccess) return e;
    }
    return hipSuccess;
}

}  // namespace cbx
