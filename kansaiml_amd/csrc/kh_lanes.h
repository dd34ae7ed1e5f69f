// kh_lanes.h -- reductions across the lanes of a wave that stay in the VALU.
// Internal header.
//
// __shfl_xor compiles to ds_bpermute_b32 on gfx950: every step of a reduction
// is then an LDS round trip that the next step waits for.  These reductions
// use DPP row rotations within each 16-lane row, then the gfx950 lane swaps
// between rows: v_permlane16_swap (rows 0,1,2,3 of two copies -> 0,0,2,2 and
// 1,1,3,3) and v_permlane32_swap (halves lo,hi -> lo,lo and hi,hi).  After a
// rotation by 8, 4, 2 and 1 every lane of a row holds the row's total, bit
// for bit the same in every lane (each step adds two copies of the same
// partial tree), so float sums are the same in every lane too.
//
// Every lane of the wave must be active (the callers reduce in uniform
// control flow, before any per-lane branch or early return).
#pragma once

#include <hip/hip_runtime.h>

#include <type_traits>

namespace kh {
namespace lanes {

// Lane i of each 16-lane row reads lane (i - n) mod 16 of its row (DPP
// row_ror:n, n = 1..15).
template <int N>
__device__ __forceinline__ unsigned row_ror(unsigned v) {
    static_assert(N >= 1 && N <= 15, "row_ror");
    return (unsigned)__builtin_amdgcn_update_dpp(0, (int)v, 0x120 + N, 0xF, 0xF, false);
}

// Lane 4q + i reads lane 4q + ((CTRL >> 2i) & 3) (DPP quad_perm).
template <int CTRL>
__device__ __forceinline__ unsigned quad_perm(unsigned v) {
    static_assert(CTRL >= 0 && CTRL <= 0xFF, "quad_perm");
    return (unsigned)__builtin_amdgcn_update_dpp(0, (int)v, CTRL, 0xF, 0xF, false);
}

// Op over the 16 lanes of each row, in every lane of the row.
template <typename T, typename Op>
__device__ __forceinline__ T row16_reduce(T v, Op op) {
    auto rot = [](T x, auto n) {
        return __builtin_bit_cast(T, row_ror<decltype(n)::value>(__builtin_bit_cast(unsigned, x)));
    };
    v = op(v, rot(v, std::integral_constant<int, 8>{}));
    v = op(v, rot(v, std::integral_constant<int, 4>{}));
    v = op(v, rot(v, std::integral_constant<int, 2>{}));
    v = op(v, rot(v, std::integral_constant<int, 1>{}));
    return v;
}

// Combines rows 0 with 1 and 2 with 3.
template <typename T, typename Op>
__device__ __forceinline__ T swap16(T v, Op op) {
    const auto p = __builtin_amdgcn_permlane16_swap(__builtin_bit_cast(unsigned, v), __builtin_bit_cast(unsigned, v),
                                                    false, false);
    return op(__builtin_bit_cast(T, (unsigned)p[0]), __builtin_bit_cast(T, (unsigned)p[1]));
}

// Combines lanes 0-31 with 32-63.
template <typename T, typename Op>
__device__ __forceinline__ T swap32(T v, Op op) {
    const auto p = __builtin_amdgcn_permlane32_swap(__builtin_bit_cast(unsigned, v), __builtin_bit_cast(unsigned, v),
                                                    false, false);
    return op(__builtin_bit_cast(T, (unsigned)p[0]), __builtin_bit_cast(T, (unsigned)p[1]));
}

struct MaxU {
    __device__ unsigned operator()(unsigned a, unsigned b) const { return a > b ? a : b; }
};
struct AddI {
    __device__ int operator()(int a, int b) const { return a + b; }
};
struct AddF {
    __device__ float operator()(float a, float b) const { return a + b; }
};
struct MaxF {
    __device__ float operator()(float a, float b) const { return fmaxf(a, b); }
};

// Wave totals of P int values per lane (P a power of two, at most 64) by a
// transposed butterfly: each exchange over one lane bit hands the half of
// the remaining values the partner keeps to the partner (lanes with the bit
// set keep the upper half), so the wave spends about 2P operations where P
// wave_sum calls spend 12P.  Bits in the order 5, 4 (lane swaps, no select),
// 0, 1 (quad permutes), 2, 3 (row rotations); bits left once one value
// remains are plain sums.  On return v[0] of lane l holds the total of value
// transposed_index<P>(l), and every lane that differs from l only in the
// plain-sum bits holds the same total.
namespace detail {
// Lane bit of exchange step k: 5, 4, 0, 1, 2, 3.
__host__ __device__ constexpr int transpose_bit(int k) { return k == 0 ? 5 : k == 1 ? 4 : k - 2; }
template <int B>
__device__ __forceinline__ int xchg(int v, bool hi) {
    if constexpr (B == 0) return (int)quad_perm<0xB1>((unsigned)v);
    else if constexpr (B == 1) return (int)quad_perm<0x4E>((unsigned)v);
    else if constexpr (B == 3) return (int)row_ror<8>((unsigned)v);
    else {  // B == 2: both rotations in every lane, then the select (a
            // rotation under a branch would read its partner lane disabled)
        const int down = (int)row_ror<4>((unsigned)v), up = (int)row_ror<12>((unsigned)v);
        return hi ? down : up;
    }
}
template <int K, int P, int C>
__device__ __forceinline__ void transpose_step(int (&v)[P], int lane) {
    if constexpr (K < 6) {
        constexpr int B = transpose_bit(K);
        if constexpr (C > 1) {
            if constexpr (B == 5 || B == 4) {
#pragma unroll
                for (int j = 0; j < C / 2; ++j) {
                    const auto s = B == 5 ? __builtin_amdgcn_permlane32_swap((unsigned)v[j], (unsigned)v[j + C / 2],
                                                                             false, false)
                                          : __builtin_amdgcn_permlane16_swap((unsigned)v[j], (unsigned)v[j + C / 2],
                                                                             false, false);
                    v[j] = (int)s[0] + (int)s[1];
                }
            } else {
                const bool hi = (lane >> B) & 1;
#pragma unroll
                for (int j = 0; j < C / 2; ++j) {
                    const int send = hi ? v[j] : v[j + C / 2];
                    const int keep = hi ? v[j + C / 2] : v[j];
                    v[j] = keep + xchg<B>(send, hi);
                }
            }
            transpose_step<K + 1, P, C / 2>(v, lane);
        } else {
            if constexpr (B == 5 || B == 4) {
                const auto s = B == 5 ? __builtin_amdgcn_permlane32_swap((unsigned)v[0], (unsigned)v[0], false, false)
                                      : __builtin_amdgcn_permlane16_swap((unsigned)v[0], (unsigned)v[0], false, false);
                v[0] = (int)s[0] + (int)s[1];
            } else {
                v[0] = v[0] + xchg<B>(v[0], (lane >> B) & 1);
            }
            transpose_step<K + 1, P, 1>(v, lane);
        }
    }
}
}  // namespace detail

template <int P>
__device__ __forceinline__ void wave_sum_transposed(int (&v)[P], int lane) {
    static_assert(P >= 1 && P <= 64 && (P & (P - 1)) == 0, "P: a power of two up to 64");
    detail::transpose_step<0, P, P>(v, lane);
}

// The value whose total lane l holds after wave_sum_transposed<P>.
template <int P>
__host__ __device__ constexpr int transposed_index(int l) {
    int idx = 0, c = P;
    for (int k = 0; k < 6 && c > 1; ++k, c /= 2) idx += ((l >> detail::transpose_bit(k)) & 1) * (c / 2);
    return idx;
}

// A lane holding the total of value idx after wave_sum_transposed<P>.
template <int P>
__host__ __device__ constexpr int transposed_lane(int idx) {
    int l = 0, c = P;
    for (int k = 0; k < 6 && c > 1; ++k, c /= 2) l |= ((idx / (c / 2)) & 1) << detail::transpose_bit(k);
    return l;
}

// Over each half-wave (lanes 0-31 and 32-63), in every lane of the half.
__device__ __forceinline__ float half_sum(float v) { return swap16(row16_reduce(v, AddF{}), AddF{}); }
__device__ __forceinline__ unsigned half_max(unsigned v) { return swap16(row16_reduce(v, MaxU{}), MaxU{}); }

// Over the whole wave, in every lane.
__device__ __forceinline__ float wave_sum(float v) { return swap32(half_sum(v), AddF{}); }
__device__ __forceinline__ unsigned wave_max(unsigned v) { return swap32(half_max(v), MaxU{}); }
__device__ __forceinline__ int wave_sum(int v) {
    return swap32(swap16(row16_reduce(v, AddI{}), AddI{}), AddI{});
}

}  // namespace lanes
}  // namespace kh
