// quantize_q8_k of one 256-block by one wave into the bit-exact batched
// GEMM's activation planes (uq_gemm_q8k.hip): the GEMM's own prep kernel and
// the rmsnorm launches that quantize the rows they normalise call it.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

#include "uq_device.h"
#include "uq_internal.h"
#include "uq_mfma.h"
#include "uq_q8k_tiles.h"

namespace uq {

// Lane l holds elements 4 l .. 4 l + 3 of block b of row m in v. As
// quantize_q8_k (quants.rs:250-290): the first strict argmax of |x| with its
// sign, iscale = -127 / max, nearest_int by the 12582912 add, min(127), the
// bsums, d = 1 / iscale; an all-zero block is d = 0, qs = 0, bsums = 0.
// Writes octet (l, h, o) = (t / 4, t / 2 % 2, t % 2) as eight f16 from lane
// t < 32, the bsums from lanes 32-33 and d from lane 34 (plane layout in
// uq_internal.h). qs[256] and bsum[16] are the wave's own LDS: a wave's LDS
// accesses complete in order, so no barrier is needed between its writes
// and reads.
template <bool Q6>
__device__ __forceinline__ void q8k_quantize_wave(const float (&v)[4], int lane, int8_t *qs, int *bsum,
                                                  const Q8Planes &P, int m, int b) {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");  // after the wave's earlier reads of qs / bsum
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    float am = 0.0f, mx = 0.0f;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const float a = fabsf(v[i]);
        if (a > am) {
            am = a;
            mx = v[i];
        }
    }
    wave_first_absmax(am, mx);  // larger |x| wins; equal |x|, the smaller index
    float d = 0.0f;
    int s = 0;
    if (am != 0.0f) {
        const float iscale = __fdiv_rn(-127.0f, mx);
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const float val = __fadd_rn(__fmul_rn(iscale, v[i]), 12582912.0f);
            int qv = (int)(__float_as_uint(val) & 0x007FFFFFu) - 0x00400000;
            qv = qv < 127 ? qv : 127;
            qs[lane * 4 + i] = (int8_t)qv;
            s += (int8_t)qv;
        }
        d = __fdiv_rn(1.0f, iscale);
    } else {
#pragma unroll
        for (int i = 0; i < 4; i++) qs[lane * 4 + i] = 0;
    }
    s = group4_sum_i(s);  // the bsum of the lane's quad: 16 elements
    if ((lane & 3) == 0) bsum[lane >> 2] = s;
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    if (lane < 32) {
        const int l = lane >> 2, h = (lane >> 1) & 1, o = lane & 1;
        h8 q;
#pragma unroll
        for (int sl = 0; sl < 8; sl++) q[sl] = (_Float16)(float)qs[q8k_slot_elem<Q6>(l, h, o, sl)];
        const size_t F = (size_t)16 * b + 2 * l + h;
        *(h8 *)(P.a + ((2 * F + o) * P.Mp + m) * 16) = q;
    } else if (lane < 34) {
        h8 q;
#pragma unroll
        for (int i = 0; i < 8; i++) q[i] = (_Float16)(float)bsum[8 * (lane - 32) + i];
        *(h8 *)(P.bs + ((size_t)b * P.Mp + m) * 32 + 16 * (lane - 32)) = q;
    } else if (lane == 34) {
        P.d8[(size_t)b * P.Mp + m] = d;
    }
}

}  // namespace uq
