// smp_head.hip — the output head that produces the sampler's logits on the device: the final
// RMS norm and the lm_head product of the reference's `head` (crates/bfi-models/src/qwen3.rs:
// 258-265, `rms_norm` then `matmul_q` over f32 weights, crates/bfi-core/src/cpu.rs:92-120 and
// 498-514), with the reference's own rounding: every product and every addition of a dot
// product is one f32 operation, added in index order from -0.0 (Rust's `Sum` of f32), so the
// logits are bit-identical to the CPU backend's and the sampler downstream draws the same
// token. That order rules out matrix cores (an MFMA sums in its own order): the product is a
// register-tiled SIMT GEMM on the VALU, 2 instructions a term.
#include <hip/hip_runtime.h>

#include <cstdint>

namespace bfi {

namespace {

constexpr int HN_BLOCK = 256;
constexpr int HN_CHUNK = 2048;  // floats of a row staged in LDS at a time

// One row per block: the mean of squares summed by one lane in index order, over chunks of
// the row staged in LDS by the block (the lane reads 16 floats a round trip), then
// out = x * (1 / sqrt(mean + eps)) * w elementwise (cpu.rs:92-120).
__global__ __launch_bounds__(HN_BLOCK) void k_head_norm(const float* __restrict__ x, const float* __restrict__ w,
                                                        int w_per_row, float eps, int64_t d,
                                                        float* __restrict__ out) {
    __shared__ float4 buf[HN_CHUNK / 4];
    __shared__ float s_scale;
    const int64_t r = blockIdx.x;
    const float* xr = x + r * d;
    const float* wr = w_per_row ? w + r * d : w;
    float s = -0.0f;  // (lane 0's running sum)
    for (int64_t c0 = 0; c0 < d; c0 += HN_CHUNK) {
        const int n = d - c0 < HN_CHUNK ? (int)(d - c0) : HN_CHUNK;
        float* fb = reinterpret_cast<float*>(buf);
        for (int i = threadIdx.x; i < n; i += HN_BLOCK) fb[i] = xr[c0 + i];
        __syncthreads();
        if (threadIdx.x == 0) {
            int i = 0;
            for (; i + 16 <= n; i += 16) {
                const float4 a = buf[i / 4], b = buf[i / 4 + 1], c = buf[i / 4 + 2], e = buf[i / 4 + 3];
                const float v[16] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w, c.x, c.y, c.z, c.w, e.x, e.y, e.z, e.w};
#pragma unroll
                for (int k = 0; k < 16; k++) s = s + v[k] * v[k];
            }
            for (; i < n; i++) s = s + fb[i] * fb[i];
        }
        __syncthreads();  // (the chunk is summed before the next overwrites it)
    }
    if (threadIdx.x == 0) {
        const float mean_sq = s / (float)d;
        s_scale = 1.0f / __builtin_sqrtf(mean_sq + eps);
    }
    __syncthreads();
    const float scale = s_scale;
    for (int64_t i = threadIdx.x; i < d; i += HN_BLOCK) out[r * d + i] = xr[i] * scale * wr[i];
}

// ---- weight formats (GGML type ids, crates/bfi-gguf/src/types/mod.rs:35-42) ------------------
// Every weight dequantized exactly as the reference's dequant_row computes it (types/*.rs):
// F16 and BF16 widen exactly; Q8_0 is q * d, Q4_0 (nibble - 8) * d, Q6_K (d * scale) * q, Q4_K
// and Q5_K (d * scale) * q - dmin * min, each product and difference one f32 rounding, d an
// f16 widened exactly. One thread per weight.
constexpr int GT_F16 = 1, GT_Q4_0 = 2, GT_Q8_0 = 8, GT_Q4_K = 12, GT_Q5_K = 13, GT_Q6_K = 14, GT_BF16 = 30, GT_Q1_0 = 41,
              GT_PQ2_0 = 142, GT_PTQ1_0 = 143;

// The 6-bit scale and min of sub-block j of a K-quant block (k_scale.rs:3-11).
__device__ __forceinline__ void scale_min_k4(int j, const uint8_t* q, uint32_t& sc, uint32_t& m) {
    if (j < 4) {
        sc = q[j] & 63u;
        m = q[j + 4] & 63u;
    } else {
        sc = (q[j + 4] & 0x0Fu) | ((uint32_t)(q[j - 4] >> 6) << 4);
        m = (uint32_t)(q[j + 4] >> 4) | ((uint32_t)(q[j] >> 6) << 4);
    }
}

__device__ __forceinline__ float f16_at(const uint8_t* p) {
    const uint16_t h = (uint16_t)p[0] | ((uint16_t)p[1] << 8);
    return (float)__builtin_bit_cast(_Float16, h);
}

template <int TYPE>
__global__ __launch_bounds__(256) void k_dequant(const uint8_t* __restrict__ src, int64_t n, float* __restrict__ dst) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= n) return;
    float v;
    if (TYPE == GT_F16) {
        v = f16_at(src + 2 * i);
    } else if (TYPE == GT_BF16) {
        const uint32_t h = (uint32_t)src[2 * i] | ((uint32_t)src[2 * i + 1] << 8);
        v = __uint_as_float(h << 16);
    } else if (TYPE == GT_Q8_0) {  // q8_0.rs:4-9: 34-byte blocks of 32
        const uint8_t* b = src + (i / 32) * 34;
        v = (float)(int8_t)b[2 + i % 32] * f16_at(b);
    } else if (TYPE == GT_Q4_0) {  // q4_0.rs:4-12: 18-byte blocks of 32, low nibbles first
        const uint8_t* b = src + (i / 32) * 18;
        const int k = (int)(i % 32);
        const uint8_t byte = b[2 + (k & 15)];
        const int nib = k < 16 ? (byte & 0x0F) : (byte >> 4);
        v = ((float)nib - 8.0f) * f16_at(b);
    } else if (TYPE == GT_Q4_K || TYPE == GT_Q5_K) {
        // q4_k.rs:6-29 (144-byte blocks: d, dmin, 12 scale bytes, 128 qs) and q5_k.rs:6-36
        // (176 bytes: the same, then qh[32] before 128 qs): (d * sc) * q - dmin * m, q a nibble
        // (Q5_K: plus 16 for its high bit)
        const int BB = TYPE == GT_Q4_K ? 144 : 176;
        const uint8_t* b = src + (i / 256) * BB;
        const int k = (int)(i % 256), group = k / 64, hi = (k % 64) / 32, l = k % 32;
        uint32_t sc, m;
        scale_min_k4(2 * group + hi, b + 4, sc, m);
        const uint8_t byte = b[(TYPE == GT_Q4_K ? 16 : 48) + group * 32 + l];
        float qv = (float)(hi ? (byte >> 4) : (byte & 0x0F));
        if (TYPE == GT_Q5_K) qv = qv + (((b[16 + l] >> (2 * group + hi)) & 1u) ? 16.0f : 0.0f);
        v = (f16_at(b) * (float)sc) * qv - f16_at(b + 2) * (float)m;
    } else if (TYPE == GT_Q1_0) {  // q1_0.rs:34-45: 18-byte blocks of 128, sign bits LSB first
        const uint8_t* b = src + (i / 128) * 18;
        const int k = (int)(i % 128);
        const float d = f16_at(b);
        v = ((b[2 + k / 8] >> (k % 8)) & 1) ? d : -d;
    } else if (TYPE == GT_PQ2_0) {  // pq2_0.rs:26-36: 34-byte blocks of 128, 2-bit codes LSB first
        const uint8_t* b = src + (i / 128) * 34;
        const int k = (int)(i % 128);
        v = ((float)((b[2 + k / 4] >> (2 * (k % 4))) & 3) - 1.0f) * f16_at(b);
    } else if (TYPE == GT_PTQ1_0) {
        // ptq1_0.rs:30-75: 28-byte blocks (qs[24], qh[2], d); weight k is base-3 digit n of a
        // byte, read as ((u8)(byte * 3^n) * 3) >> 8: k < 80 digit k/16 of qs[k%16], k < 120
        // digit (k-80)/8 of qs[16 + (k-80)%8], else digit (k-120)/2 of qh[(k-120)%2]
        const uint8_t* b = src + (i / 128) * 28;
        const int k = (int)(i % 128);
        const int at = k < 80 ? k % 16 : k < 120 ? 16 + (k - 80) % 8 : 24 + (k - 120) % 2;
        const int n = k < 80 ? k / 16 : k < 120 ? (k - 80) / 8 : (k - 120) / 2;
        const uint32_t p3 = n == 0 ? 1u : n == 1 ? 3u : n == 2 ? 9u : n == 3 ? 27u : 81u;
        const uint32_t trit = (((uint32_t)b[at] * p3) & 0xFFu) * 3u >> 8;
        v = ((float)trit - 1.0f) * f16_at(b + 26);
    } else {  // GT_Q6_K, q6_k.rs:4-29: 210-byte blocks of 256 (ql[128], qh[64], scales[16], d)
        const uint8_t* b = src + (i / 256) * 210;
        const int k = (int)(i % 256), nh = k / 128, quarter = (k % 128) / 32, l = k % 32;
        const uint8_t* ql = b + nh * 64;
        const uint8_t qh = b[128 + nh * 32 + l];
        const uint8_t lo = ql[l + ((quarter & 1) ? 32 : 0)];
        const int q = ((quarter < 2 ? (lo & 0x0F) : (lo >> 4)) | (((qh >> (2 * quarter)) & 3) << 4)) - 32;
        const float sc = (float)(int8_t)b[192 + nh * 8 + l / 16 + 2 * quarter];
        v = (f16_at(b + 208) * sc) * (float)q;
    }
    dst[i] = v;
}

constexpr int HG_BO = 64;   // outputs (rows of W) a block
constexpr int HG_BT = 64;   // tokens a block
constexpr int HG_K = 16;    // inner-dimension chunk staged through LDS
constexpr int HG_BLOCK = 256;

// out[t][o] = sum over i in index order of W[o][i] * X[t][i]. A thread owns 4 outputs x 4
// tokens; each chunk of 16 inner positions is staged transposed in LDS so a thread reads
// its 4 weights and 4 inputs of one position as two 16-byte loads. BLK > 0: the fused block
// dot of the Q8_0 and Q4_0 (BLK 32), PQ2_0 and PTQ1_0 (BLK 128) formats (q8_0.rs:11-15,
// pq2_0.rs:38-42, cpu.rs:550-563): each block's products summed from -0.0, the block sums
// added from +0.0 (d a multiple of BLK). SIGNS: the Q1_0 dot (q1_0.rs:48-64, simd.rs:74-80)
// over its dequantized weights +-s: each input added with its weight's sign, the block's sum
// times the block's scale |w| (BLK 128).
template <int BLK, bool SIGNS>
__global__ __launch_bounds__(HG_BLOCK) void k_head_gemm(const float* __restrict__ W, const float* __restrict__ X,
                                                        int64_t n_out, int64_t n_tok, int64_t d, int vec,
                                                        float* __restrict__ out) {
    __shared__ float4 Ws[HG_K][HG_BO / 4];
    __shared__ float4 Xs[HG_K][HG_BT / 4];
    const int tid = threadIdx.x;
    const int to = tid % 16, tt = tid / 16;  // this thread: outputs 4 to.., tokens 4 tt..
    const int64_t o0 = (int64_t)blockIdx.x * HG_BO, t0 = (int64_t)blockIdx.y * HG_BT;
    constexpr bool BLOCKED = BLK > 0;
    static_assert(BLK % HG_K == 0 && (!SIGNS || BLOCKED), "a block is whole chunks");
    float acc[4][4], part[4][4];  // (part: the current block's sum, BLOCKED)
    float bs[4] = {0.0f, 0.0f, 0.0f, 0.0f};  // (SIGNS: the block's scale of each output)
#pragma unroll
    for (int a = 0; a < 4; a++)
#pragma unroll
        for (int b = 0; b < 4; b++) {
            acc[a][b] = BLOCKED ? 0.0f : -0.0f;
            part[a][b] = -0.0f;
        }
    // staging: thread tid loads 4 consecutive inner positions of one row of the tile
    const int lr = tid / 4, lc = (tid % 4) * 4;
    const int64_t wrow = o0 + lr, xrow = t0 + lr;
    for (int64_t k0 = 0; k0 < d; k0 += HG_K) {
        float wv[4], xv[4];
        if (vec && k0 + lc + 3 < d) {
            const float4 a = wrow < n_out ? *reinterpret_cast<const float4*>(W + wrow * d + k0 + lc) : make_float4(0, 0, 0, 0);
            const float4 b = xrow < n_tok ? *reinterpret_cast<const float4*>(X + xrow * d + k0 + lc) : make_float4(0, 0, 0, 0);
            wv[0] = a.x, wv[1] = a.y, wv[2] = a.z, wv[3] = a.w;
            xv[0] = b.x, xv[1] = b.y, xv[2] = b.z, xv[3] = b.w;
        } else {
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const int64_t i = k0 + lc + j;
                wv[j] = (wrow < n_out && i < d) ? W[wrow * d + i] : 0.0f;
                xv[j] = (xrow < n_tok && i < d) ? X[xrow * d + i] : 0.0f;
            }
        }
        __syncthreads();  // (the previous chunk has been read)
#pragma unroll
        for (int j = 0; j < 4; j++) {
            reinterpret_cast<float*>(&Ws[lc + j][0])[lr] = wv[j];
            reinterpret_cast<float*>(&Xs[lc + j][0])[lr] = xv[j];
        }
        __syncthreads();
        const int kn = d - k0 < HG_K ? (int)(d - k0) : HG_K;  // (a partial last chunk adds no padding)
        for (int k = 0; k < kn; k++) {
            const float4 a = Ws[k][to], b = Xs[k][tt];
            const float av[4] = {a.x, a.y, a.z, a.w}, bv[4] = {b.x, b.y, b.z, b.w};
            if (SIGNS && k == 0 && k0 % BLK == 0) {
#pragma unroll
                for (int p = 0; p < 4; p++) bs[p] = __builtin_fabsf(av[p]);
            }
#pragma unroll
            for (int p = 0; p < 4; p++)
#pragma unroll
                for (int q = 0; q < 4; q++) {
                    if (SIGNS)  // (x with the weight's sign bit: exact negation where it is set)
                        part[p][q] = part[p][q] + __uint_as_float(__float_as_uint(bv[q]) ^
                                                                  (__float_as_uint(av[p]) & 0x80000000u));
                    else if (BLOCKED) part[p][q] = part[p][q] + av[p] * bv[q];
                    else acc[p][q] = acc[p][q] + av[p] * bv[q];
                }
        }
        if (BLOCKED && ((k0 + HG_K) % BLK) == 0) {  // (the chunk ends a block)
#pragma unroll
            for (int p = 0; p < 4; p++)
#pragma unroll
                for (int q = 0; q < 4; q++) {
                    acc[p][q] = acc[p][q] + (SIGNS ? part[p][q] * bs[p] : part[p][q]);
                    part[p][q] = -0.0f;
                }
        }
    }
#pragma unroll
    for (int q = 0; q < 4; q++) {
        const int64_t t = t0 + tt * 4 + q;
        if (t >= n_tok) continue;
#pragma unroll
        for (int p = 0; p < 4; p++) {
            const int64_t o = o0 + to * 4 + p;
            if (o < n_out) out[t * n_out + o] = acc[p][q];
        }
    }
}

}  // namespace

// xn: n_tok * d floats of workspace; out: n_tok * n_out logits.
// vec: d % 4 == 0 and W 16-byte aligned (the rows then load as 16-byte vectors).
// blocked: the dot order of a format with a fused block dot: 1 blocks of 32 (Q8_0, Q4_0;
// d % 32 == 0), 2 blocks of 128 (PQ2_0, PTQ1_0), 3 Q1_0's signed blocks of 128 (d % 128 == 0).
hipError_t launch_head(const float* x, const float* norm_w, int norm_per_row, float eps, const float* W,
                       int64_t n_tok, int64_t d, int64_t n_out, int vec, int blocked, float* xn, float* out,
                       hipStream_t stream) {
    if (n_tok <= 0 || n_out <= 0) return hipSuccess;
    hipLaunchKernelGGL(k_head_norm, dim3((unsigned)n_tok), dim3(HN_BLOCK), 0, stream, x, norm_w, norm_per_row, eps, d, xn);
    const dim3 grid((unsigned)((n_out + HG_BO - 1) / HG_BO), (unsigned)((n_tok + HG_BT - 1) / HG_BT));
    if ((blocked == 1 && d % 32 != 0) || (blocked >= 2 && d % 128 != 0) || blocked < 0 || blocked > 3)
        return hipErrorInvalidValue;
    switch (blocked) {
        case 1: hipLaunchKernelGGL((k_head_gemm<32, false>), grid, dim3(HG_BLOCK), 0, stream, W, xn, n_out, n_tok, d, vec, out); break;
        case 2: hipLaunchKernelGGL((k_head_gemm<128, false>), grid, dim3(HG_BLOCK), 0, stream, W, xn, n_out, n_tok, d, vec, out); break;
        case 3: hipLaunchKernelGGL((k_head_gemm<128, true>), grid, dim3(HG_BLOCK), 0, stream, W, xn, n_out, n_tok, d, vec, out); break;
        default: hipLaunchKernelGGL((k_head_gemm<0, false>), grid, dim3(HG_BLOCK), 0, stream, W, xn, n_out, n_tok, d, vec, out);
    }
    return hipGetLastError();
}

// n weights of a GGML tensor (n a multiple of the type's block) to f32; hipErrorInvalidValue
// for a type this head does not take.
hipError_t launch_dequant(int type, const void* src, int64_t n, float* dst, hipStream_t stream) {
    if (n <= 0) return hipSuccess;
    const dim3 grid((unsigned)((n + 255) / 256));
    const uint8_t* s = static_cast<const uint8_t*>(src);
    switch (type) {
        case GT_F16: hipLaunchKernelGGL(k_dequant<GT_F16>, grid, dim3(256), 0, stream, s, n, dst); break;
        case GT_BF16: hipLaunchKernelGGL(k_dequant<GT_BF16>, grid, dim3(256), 0, stream, s, n, dst); break;
        case GT_Q8_0: hipLaunchKernelGGL(k_dequant<GT_Q8_0>, grid, dim3(256), 0, stream, s, n, dst); break;
        case GT_Q4_0: hipLaunchKernelGGL(k_dequant<GT_Q4_0>, grid, dim3(256), 0, stream, s, n, dst); break;
        case GT_Q6_K: hipLaunchKernelGGL(k_dequant<GT_Q6_K>, grid, dim3(256), 0, stream, s, n, dst); break;
        case GT_Q4_K: hipLaunchKernelGGL(k_dequant<GT_Q4_K>, grid, dim3(256), 0, stream, s, n, dst); break;
        case GT_Q5_K: hipLaunchKernelGGL(k_dequant<GT_Q5_K>, grid, dim3(256), 0, stream, s, n, dst); break;
        case GT_Q1_0: hipLaunchKernelGGL(k_dequant<GT_Q1_0>, grid, dim3(256), 0, stream, s, n, dst); break;
        case GT_PQ2_0: hipLaunchKernelGGL(k_dequant<GT_PQ2_0>, grid, dim3(256), 0, stream, s, n, dst); break;
        case GT_PTQ1_0: hipLaunchKernelGGL(k_dequant<GT_PTQ1_0>, grid, dim3(256), 0, stream, s, n, dst); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

}  // namespace bfi
