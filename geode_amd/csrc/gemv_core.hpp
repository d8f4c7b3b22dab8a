// gemv_core.hpp - the inner loop of the dequant-in-register skinny GEMM, shared by the plain product (q4.hip) and
// the grouped expert products (model.hip).
//
// The int8 path of matvec_rows_q_ref (engine/src/kernels.cpp:1304-1322): per 16-value block an exact integer sum
// of level x q, then acc += float(sum) x (e4m3(scale) x act scale). Here a wave is 64/S row-lanes x S k-lanes;
// lane (g, k) takes rows row0 + i * 64/S + g (i < R) and its k-lane's 32-value chunks c = s * S + k. Per step a
// lane loads R 16-byte code chunks (each load instruction of the wave reads 1 KB of consecutive bytes), turns
// the affine nibbles into doubled codes 2c' (int8 lanes), and for every token runs 8 dot4 per chunk on the
// activations in LDS: the integer sum starts from -15 x (the block's activation sum), which makes the affine
// codes' sum the levels' sum exactly. The k-lanes' fp32 partial sums are added by a fixed xor tree.
#pragma once

#include "common.hpp"

namespace gv {

template <int S, int R, int MT>
__device__ inline void gemv_wave(const uint8_t *__restrict__ codes, const uint8_t *__restrict__ scales, int64_t rows,
                                 int64_t cols, int steps, int64_t row0, const uint8_t *__restrict__ lds,
                                 int64_t abytes, int M, int g, int k, float (&acc)[R][MT]) {
    constexpr int G = 64 / S;
    const int64_t tile = row0 / kTileRows, rho0 = row0 % kTileRows;
    const int64_t th = min(static_cast<int64_t>(kTileRows), rows - tile * kTileRows);
    const int groups = q4_groups(steps);
    const uint8_t *cbase = codes + tile * kTileRows * (cols / 2);
    const uint8_t *sbase = scales + tile * kTileRows * S * groups * 16;
    bool valid[R];
    int64_t rho[R];
#pragma unroll
    for (int i = 0; i < R; ++i) {
        rho[i] = rho0 + i * G + g;
        valid[i] = row0 + i * G + g < rows;
    }
#pragma unroll
    for (int i = 0; i < R; ++i)
#pragma unroll
        for (int t = 0; t < MT; ++t) acc[i][t] = 0.0f;

    for (int s0 = 0; s0 < steps; s0 += 8) {
        uint4 scw[R];
#pragma unroll
        for (int i = 0; i < R; ++i)
            scw[i] = valid[i] ? *reinterpret_cast<const uint4 *>(sbase + (((s0 / 8) * th + rho[i]) * S + k) * 16)
                              : make_uint4(0, 0, 0, 0);
#pragma unroll
        for (int ss = 0; ss < 8; ++ss) {
            const int s = s0 + ss;
            if (s >= steps) break;
            uint32_t dec[R][8];
            float sc[R][2];
#pragma unroll
            for (int i = 0; i < R; ++i) {
                const uint4 cw = valid[i] ? *reinterpret_cast<const uint4 *>(cbase + ((s * th + rho[i]) * S + k) * 16)
                                          : make_uint4(0x88888888u, 0x88888888u, 0x88888888u, 0x88888888u);
                const uint32_t wd[4] = {cw.x, cw.y, cw.z, cw.w};
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    dec[i][2 * q] = (wd[q] << 1) & 0x1E1E1E1Eu;       // 2c' of values 0 2 4 6 of the word
                    dec[i][2 * q + 1] = (wd[q] >> 3) & 0x1E1E1E1Eu;   // 2c' of values 1 3 5 7
                }
                const uint32_t sword = (ss < 2) ? scw[i].x : (ss < 4) ? scw[i].y : (ss < 6) ? scw[i].z : scw[i].w;
                const uint32_t pair = (ss & 1) ? (sword >> 16) : (sword & 0xFFFFu);
                sc[i][0] = e4m3_to_f32(pair & 0xFFu);
                sc[i][1] = e4m3_to_f32((pair >> 8) & 0xFFu);
            }
            const uint8_t *ac = lds + static_cast<int64_t>(s * S + k) * kActChunkBytes;
#pragma unroll
            for (int t = 0; t < MT; ++t) {
                if (t >= M) break;
                const uint8_t *at = ac + t * abytes;
                const uint4 q0 = *reinterpret_cast<const uint4 *>(at);
                const uint4 q1 = *reinterpret_cast<const uint4 *>(at + 16);
                const float2 as = *reinterpret_cast<const float2 *>(at + 32);
                const int2 corr = *reinterpret_cast<const int2 *>(at + 40);
#pragma unroll
                for (int i = 0; i < R; ++i) {
                    int s_0 = corr.x;
                    s_0 = dot4(dec[i][0], q0.x, s_0);
                    s_0 = dot4(dec[i][1], q0.y, s_0);
                    s_0 = dot4(dec[i][2], q0.z, s_0);
                    s_0 = dot4(dec[i][3], q0.w, s_0);
                    int s_1 = corr.y;
                    s_1 = dot4(dec[i][4], q1.x, s_1);
                    s_1 = dot4(dec[i][5], q1.y, s_1);
                    s_1 = dot4(dec[i][6], q1.z, s_1);
                    s_1 = dot4(dec[i][7], q1.w, s_1);
                    acc[i][t] = __builtin_fmaf(static_cast<float>(s_0), __fmul_rn(sc[i][0], as.x), acc[i][t]);
                    acc[i][t] = __builtin_fmaf(static_cast<float>(s_1), __fmul_rn(sc[i][1], as.y), acc[i][t]);
                }
            }
        }
    }
}

// the k-lanes' partial sums added (a fixed xor tree: the same bits on every run)
template <int S, int R, int MT>
__device__ inline void gemv_reduce(float (&acc)[R][MT], int M) {
#pragma unroll
    for (int i = 0; i < R; ++i)
#pragma unroll
        for (int t = 0; t < MT; ++t) {
            if (t >= M) break;
#pragma unroll
            for (int o = S / 2; o > 0; o >>= 1) acc[i][t] += __shfl_xor(acc[i][t], o, 64);
        }
}

// M tokens' activations (abytes each, act_stride apart in global memory) into LDS
__device__ inline void load_acts(uint8_t *lds, const uint8_t *__restrict__ act, int64_t act_stride, int64_t abytes,
                                 int M) {
    for (int64_t i = static_cast<int64_t>(threadIdx.x) * 16; i < M * abytes; i += static_cast<int64_t>(blockDim.x) * 16) {
        const int64_t t = i / abytes, o = i % abytes;
        *reinterpret_cast<uint4 *>(lds + i) = *reinterpret_cast<const uint4 *>(act + t * act_stride + o);
    }
}

// One 16-value block of activations into the products' layout (quantize_activation, kernels.cpp:1254-1295, bit for
// bit): amax / 127 the scale, lrint(x x 127 / amax) clamped to +-127, and -15 x their sum for the affine codes.
__device__ inline void quantize_block16(const float (&v)[16], uint8_t *act_row, int b) {
    float amax = 0.0f;
#pragma unroll
    for (int i = 0; i < 16; ++i) amax = fmaxf(amax, fabsf(v[i]));
    const float s = __fdiv_rn(amax, 127.0f), qi = amax > 0.0f ? __fdiv_rn(127.0f, amax) : 0.0f;
    int sum = 0;
    uint32_t dw[4] = {0, 0, 0, 0};   // word 0: even, odd; word 1: even, odd
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        const int q = min(max(static_cast<int>(rintf(__fmul_rn(v[i], qi))), -127), 127);
        sum += q;
        dw[2 * (i / 8) + ((i % 8) & 1)] |= (static_cast<uint32_t>(q) & 0xFFu) << (8 * ((i % 8) >> 1));
    }
    uint8_t *chunk = act_row + static_cast<size_t>(b / 2) * kActChunkBytes;
    const int j = b % 2;
    *reinterpret_cast<uint4 *>(chunk + 16 * j) = make_uint4(dw[0], dw[1], dw[2], dw[3]);
    reinterpret_cast<float *>(chunk + 32)[j] = s;
    reinterpret_cast<int *>(chunk + 40)[j] = -15 * sum;
}

// a row of cols values (any memory) into act_row, the workgroup's threads over its blocks
__device__ inline void quantize_row(const float *v, int cols, uint8_t *act_row) {
    for (int b = threadIdx.x; b < cols / 16; b += blockDim.x) {
        float blk[16];
#pragma unroll
        for (int i = 0; i < 16; ++i) blk[i] = v[b * 16 + i];
        quantize_block16(blk, act_row, b);
    }
}

}  // namespace gv
