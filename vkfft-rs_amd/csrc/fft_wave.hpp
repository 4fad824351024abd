// fft_wave.hpp -- one wave per line, every exchange between stages in
// registers (gfx950, wave64, no LDS).
//
// A 1024-point f32 line lives in one wave as 64 lanes x 16 registers. Let
// n = n0..n9 be the input index bits and k = k0..k9 the output index bits.
// The load puts n0..n5 in the lane index and n6..n9 in the register index
// (lane l, register r holds x[l + 64 r]: 512 contiguous bytes per load
// instruction). The transform is Cooley-Tukey over index bits, highest input
// bits first, each pass a DFT over the four or two bits that sit in the
// register index at that point:
//
//   pass 1  DFT16 over n6..n9 (registers) -> k0..k3; twiddle W1024^(l*q)
//   swap    lane bits 0..3 <-> register bits 0..3 (DPP within rows of 16)
//   swap    lane bits 4,5  <-> register bits 0,1  (permlane16/32 swaps)
//   pass 2  DFT4 over n4,n5 (register bits 0,1) -> k4,k5; twiddle
//           W64^(a*c), a = n0..n3, c = k4 + 2 k5
//   swap    lane bits 4,5  <-> register bits 0,1
//   pass 3  DFT16 over n0..n3 (registers) -> k6..k9
//
// after which lane l, register d holds X[l + 64 d]: the store is as
// contiguous as the load. This is the Stockham schedule of radices
// (16, 4, 16) of src/kernel_ir.rs:4565-4608 up to where each intermediate
// element lives: with identity butterflies the kernel applies the same
// mixed-radix digit-reversal permutation as that stage sequence.
//
// A swap of lane bit b with register bit c moves, for every register pair
// (r, r | 1<<c), the element held at (register bit u, lane bit t) to
// (register bit t, lane bit u): half of each pair crosses to the partner
// lane, the other half stays. Within a row of 16 lanes the partner's value
// arrives through a DPP read folded into the select; lane bits 4 and 5 use
// gfx950's v_permlane16_swap / v_permlane32_swap, which exchange the two
// halves of a register pair in one instruction.
#pragma once

#include "fft_kernels_impl.hpp"

namespace vkfx {

// DPP16 controls (gfx9 encoding; lane mapping measured on gfx950):
// quad_perm [1,0,3,2] reads lane i^1, [2,3,0,1] lane i^2; row_ror:n reads
// lane (i - n) mod 16 of the lane's row of 16.
enum : int { kDppXor1 = 0xB1, kDppXor2 = 0x4E, kDppRor4 = 0x124, kDppRor8 = 0x128, kDppRor12 = 0x12C };

template <int CTRL>
__device__ __forceinline__ float dpp_read(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), CTRL, 0xF, 0xF, true));
}

template <int CTRL, int BANKS>
__device__ __forceinline__ float dpp_update(float old, float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(__builtin_bit_cast(int, old), __builtin_bit_cast(int, v),
                                                                 CTRL, 0xF, BANKS, false));
}

// Swap lane bit LB (< 4) with register bit LB over 16 registers. A lane with
// the bit set takes its partner's (lane - 2^LB) odd register into the even
// one; a lane with the bit clear takes its partner's (lane + 2^LB) even
// register into the odd one. For lane bits 2 and 3 the lanes that take a
// value are whole banks of 4 lanes, so one DPP move with a bank mask does it
// (the other banks keep their register); for bits 0 and 1 a DPP read feeds
// a select.
template <int LB>
__device__ __forceinline__ void wave_swap_row_bit(cpx<float>* x, int lane) {
    constexpr int B = 1 << LB;
    if constexpr (LB >= 2) {
        constexpr int kFromBelow = LB == 2 ? kDppRor4 : kDppRor8;
        constexpr int kFromAbove = LB == 2 ? kDppRor12 : kDppRor8;
        constexpr int kSetBanks = LB == 2 ? 0xA : 0xC;  // banks whose lanes have bit LB set
#pragma unroll
        for (int r0 = 0; r0 < 16; ++r0) {
            if (r0 & B) continue;
            const int r1 = r0 | B;
            const cpx<float> a = x[r0], b = x[r1];
            x[r0] = mk(dpp_update<kFromBelow, kSetBanks>(a.re, b.re), dpp_update<kFromBelow, kSetBanks>(a.im, b.im));
            x[r1] = mk(dpp_update<kFromAbove, 0xF ^ kSetBanks>(b.re, a.re),
                       dpp_update<kFromAbove, 0xF ^ kSetBanks>(b.im, a.im));
        }
    } else {
        constexpr int kXor = LB == 0 ? kDppXor1 : kDppXor2;
        const bool t = (lane & B) != 0, nt = (lane & B) == 0;
#pragma unroll
        for (int r0 = 0; r0 < 16; ++r0) {
            if (r0 & B) continue;
            const int r1 = r0 | B;
            const cpx<float> a = x[r0], b = x[r1];
            const float br = dpp_read<kXor>(b.re), bi = dpp_read<kXor>(b.im);
            const float ar = dpp_read<kXor>(a.re), ai = dpp_read<kXor>(a.im);
            x[r0].re = nt ? a.re : br;
            x[r0].im = nt ? a.im : bi;
            x[r1].re = t ? b.re : ar;
            x[r1].im = t ? b.im : ai;
        }
    }
}

__device__ __forceinline__ unsigned fbits(float v) { return __builtin_bit_cast(unsigned, v); }
__device__ __forceinline__ float bitsf(unsigned v) { return __builtin_bit_cast(float, v); }

// Swap lane bit 4 with register bit 0 and lane bit 5 with register bit 1.
// v_permlane16_swap(a, b) exchanges rows 1 and 3 of a with rows 0 and 2 of
// b; v_permlane32_swap(a, b) the upper 32 lanes of a with the lower 32 of b.
__device__ __forceinline__ void wave_swap_lane45(cpx<float>* x) {
#pragma unroll
    for (int r0 = 0; r0 < 16; r0 += 2) {
        auto p = __builtin_amdgcn_permlane16_swap(fbits(x[r0].re), fbits(x[r0 + 1].re), false, false);
        auto q = __builtin_amdgcn_permlane16_swap(fbits(x[r0].im), fbits(x[r0 + 1].im), false, false);
        x[r0] = mk(bitsf(p[0]), bitsf(q[0]));
        x[r0 + 1] = mk(bitsf(p[1]), bitsf(q[1]));
    }
#pragma unroll
    for (int r0 = 0; r0 < 16; ++r0) {
        if (r0 & 2) continue;
        auto p = __builtin_amdgcn_permlane32_swap(fbits(x[r0].re), fbits(x[r0 + 2].re), false, false);
        auto q = __builtin_amdgcn_permlane32_swap(fbits(x[r0].im), fbits(x[r0 + 2].im), false, false);
        x[r0] = mk(bitsf(p[0]), bitsf(q[0]));
        x[r0 + 2] = mk(bitsf(p[1]), bitsf(q[1]));
    }
}

// Twiddle table of k_wave1024 (kWave1024TableLen complex, forward roots;
// the inverse conjugates them), lane index fastest so that one load
// instruction reads contiguous memory: [j * 64 + l] = W1024^(l 2^j) for
// j < 4 and lanes l < 64, then [256 + m] = W64^m for m < 4.

// x[q] *= W^(q e) for q = 1..15 from the roots w1 = W^e, w2, w4, w8: every
// other power is a product of at most four of them (relative error a few
// ulp).
template <int S>
__device__ __forceinline__ void wave_twiddle16(cpx<float>* x, cpx<float> w1, cpx<float> w2, cpx<float> w4,
                                               cpx<float> w8) {
    const cpx<float> w3 = cmul(w1, w2), w5 = cmul(w1, w4), w6 = cmul(w2, w4), w7 = cmul(w3, w4);
    x[1] = twmul<S>(x[1], w1);
    x[2] = twmul<S>(x[2], w2);
    x[3] = twmul<S>(x[3], w3);
    x[4] = twmul<S>(x[4], w4);
    x[5] = twmul<S>(x[5], w5);
    x[6] = twmul<S>(x[6], w6);
    x[7] = twmul<S>(x[7], w7);
    x[8] = twmul<S>(x[8], w8);
    x[9] = twmul<S>(x[9], cmul(w8, w1));
    x[10] = twmul<S>(x[10], cmul(w8, w2));
    x[11] = twmul<S>(x[11], cmul(w8, w3));
    x[12] = twmul<S>(x[12], cmul(w8, w4));
    x[13] = twmul<S>(x[13], cmul(w8, w5));
    x[14] = twmul<S>(x[14], cmul(w8, w6));
    x[15] = twmul<S>(x[15], cmul(w8, w7));
}

// Pass-2 twiddles: register r = c + 4 g (c = k4 + 2 k5, g = n2 + 2 n3) of a
// lane with m = n0 + 2 n1 takes W64^((m + 4 g) c) = (W64^m)^c * W16^(g c);
// u = W64^m.
template <int S>
__device__ __forceinline__ void wave_twiddle64(cpx<float>* x, cpx<float> u1) {
    const cpx<float> u2 = cmul(u1, u1), u3 = cmul(u1, u2);
    const cpx<float> u[4] = {mk(1.0f, 0.0f), u1, u2, u3};
    constexpr float kC1 = 0.923879532511286756128183189396788933f, kS1 = 0.382683432365089771728459984030398866f;
    constexpr float kR = 0.707106781186547524400844362104849039f;
    // W16^j = exp(-2 pi i j / 16), j = 0..9 (forward roots)
    const cpx<float> w16[10] = {mk(1.0f, 0.0f), mk(kC1, -kS1), mk(kR, -kR),  mk(kS1, -kC1), mk(0.0f, -1.0f),
                                mk(-kS1, -kC1), mk(-kR, -kR),  mk(-kC1, -kS1), mk(-1.0f, 0.0f), mk(-kC1, kS1)};
#pragma unroll
    for (int g = 0; g < 4; ++g)
#pragma unroll
        for (int c = 1; c < 4; ++c) {
            const cpx<float> w = g == 0 ? u[c] : cmul(u[c], w16[g * c]);
            x[4 * g + c] = twmul<S>(x[4 * g + c], w);
        }
}

// The transform of one line held in x (lane l, register r = x[l + 64 r] on
// entry, X[l + 64 r] on exit); w1..w8 and u1 are the lane's twiddle roots.
template <int S>
__device__ __forceinline__ void wave1024_transform(cpx<float>* x, int lane, cpx<float> w1, cpx<float> w2,
                                                   cpx<float> w4, cpx<float> w8, cpx<float> u1) {
    dft<16, S>(x);
    wave_twiddle16<S>(x, w1, w2, w4, w8);

    wave_swap_row_bit<0>(x, lane);
    wave_swap_row_bit<1>(x, lane);
    wave_swap_row_bit<2>(x, lane);
    wave_swap_row_bit<3>(x, lane);
    wave_swap_lane45(x);

#pragma unroll
    for (int g = 0; g < 4; ++g) dft<4, S>(x + 4 * g);
    wave_twiddle64<S>(x, u1);

    wave_swap_lane45(x);
    dft<16, S>(x);
}

// Stores a transformed line (register d to dst[64 d]), scaled when asked.
template <bool NTO>
__device__ __forceinline__ void wave_store(cpx<float>* dst, cpx<float>* x, bool scaled, float s) {
    if (scaled) {
#pragma unroll
        for (int d = 0; d < 16; ++d) stg<NTO>(dst + 64 * d, scale(x[d], s));
    } else {
#pragma unroll
        for (int d = 0; d < 16; ++d) stg<NTO>(dst + 64 * d, x[d]);
    }
}

// Element offsets of line `line` in the input and output (IoPlain rows:
// line_default placement, element stride 1).
__device__ __forceinline__ void wave_line_offsets(const KArgs& a, long long line, long long* ib, long long* ob) {
    if (a.C == 1 && a.C1 == 1) {  // rows back to back
        *ib = line * a.in_os;
        *ob = line * a.out_os;
    } else {
        const LineInfo L = line_default(a, line / a.G, (int)(line % a.G));
        *ib = L.ib;
        *ob = L.ob;
    }
}

// One 1024-point f32 C2C line per wave, four waves (lines) per block, no LDS.
template <int S, bool NTI, bool NTO>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(8))) void k_wave1024(const KArgs a) {
    const int lane = (int)(threadIdx.x & 63);
    const int w = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));  // wave-uniform
    const long long line = (long long)blockIdx.x * 4 + w;
    if (line >= a.nlines) return;
    long long ib, ob;
    wave_line_offsets(a, line, &ib, &ob);

    cpx<float> x[16];
    const cpx<float>* src = (const cpx<float>*)a.in + ib + lane;
#pragma unroll
    for (int r = 0; r < 16; ++r) x[r] = ldg<NTI>(src + 64 * r);
    // the twiddle roots depend on the lane only: their loads go out with the
    // line's, so no pass waits on memory after the line has arrived
    const cpx<float>* tw = (const cpx<float>*)a.tw;
    const cpx<float> w1 = tw[lane], w2 = tw[64 + lane], w4 = tw[128 + lane], w8 = tw[192 + lane];
    const cpx<float> u1 = tw[256 + (lane >> 4)];
    __builtin_amdgcn_sched_barrier(0);

    wave1024_transform<S>(x, lane, w1, w2, w4, w8, u1);
    wave_store<NTO>((cpx<float>*)a.out + ob + lane, x, a.scale != 1.0, (float)a.scale);
}

}  // namespace vkfx
