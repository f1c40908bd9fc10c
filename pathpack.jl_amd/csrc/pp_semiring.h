// pp_semiring.h -- the six semirings as device (and host) functors.
//
// Semantics follow the reference's scalar layer (src/CPU/semiring/*.jl) on x86:
//   plus      = vmin / vmax / + / |            (semiring.jl:124-138, tropical.jl:150-160, real.jl:37, boolean.jl:55)
//   muladd    = plus(a (x) b, c)               (tropical.jl:188-191, bottleneck.jl:57-59, real.jl:42-44)
//   prod      = a (x) b, NaN -> zero for the tropical semirings (tropical.jl:164-172)
//   star      = tropical: one if a <= one in the semiring order else the top; PlusProd 1/(1-a); lattices one
//               (tropical.jl:210-218, real.jl:50-58, bottleneck.jl:63-65, boolean.jl:65-67)
//   integral  = lattices (MaxMin, MinMax, OrAnd): no star scaling in the LU and the solves (semiring.jl:478-492)
//   muladd2   = plus(plus(a0 (x) b0, a1 (x) b1), c): two multiply-adds into one accumulator, which min/max
//               semirings issue as v_add, v_add, v_min3 (1.5 VALU instructions per multiply-add)
// min and max use the hardware v_min/v_max (IEEE minNum/maxNum, as the reference's GPU backend does with
// llvm.minnum/maxnum, PATHPACKCUDAExt.jl:37-49): identical to ifelse(x < y, x, y) whenever the accumulator is not
// NaN, which the factorization never produces, and apart from the sign of a zero when both operands are zeros of
// opposite signs.
#pragma once
#include <hip/hip_runtime.h>
#include <cstdint>

namespace pp {

enum { S_MINPLUS = 0, S_MAXPLUS = 1, S_MAXMIN = 2, S_MINMAX = 3, S_PLUSPROD = 4, S_ORAND = 5 };
enum { D_F32 = 0, D_F64 = 1, D_I32 = 2 };

template <class T> struct Lim;
template <> struct Lim<float> {
    __host__ __device__ static constexpr float inf() { return __builtin_huge_valf(); }
};
template <> struct Lim<double> {
    __host__ __device__ static constexpr double inf() { return __builtin_huge_val(); }
};

__host__ __device__ inline float pmin(float a, float b) { return __builtin_fminf(a, b); }
__host__ __device__ inline float pmax(float a, float b) { return __builtin_fmaxf(a, b); }
__host__ __device__ inline double pmin(double a, double b) { return __builtin_fmin(a, b); }
__host__ __device__ inline double pmax(double a, double b) { return __builtin_fmax(a, b); }

template <class T> struct MinPlus {
    typedef T value_type;
    static constexpr int id = S_MINPLUS;
    static constexpr bool integral = false;
    __host__ __device__ static T zero() { return Lim<T>::inf(); }
    __host__ __device__ static T one() { return T(0); }
    __host__ __device__ static T plus(T a, T b) { return pmin(a, b); }
    __host__ __device__ static T muladd(T a, T b, T c) { return pmin(a + b, c); }
    __host__ __device__ static T muladd2(T a0, T b0, T a1, T b1, T c) { return pmin(pmin(a0 + b0, a1 + b1), c); }
    __host__ __device__ static T prod(T a, T b) { T c = a + b; return c != c ? zero() : c; }
    __host__ __device__ static T star(T a) { return a >= T(0) ? one() : -Lim<T>::inf(); }
};

template <class T> struct MaxPlus {
    typedef T value_type;
    static constexpr int id = S_MAXPLUS;
    static constexpr bool integral = false;
    __host__ __device__ static T zero() { return -Lim<T>::inf(); }
    __host__ __device__ static T one() { return T(0); }
    __host__ __device__ static T plus(T a, T b) { return pmax(a, b); }
    __host__ __device__ static T muladd(T a, T b, T c) { return pmax(a + b, c); }
    __host__ __device__ static T muladd2(T a0, T b0, T a1, T b1, T c) { return pmax(pmax(a0 + b0, a1 + b1), c); }
    __host__ __device__ static T prod(T a, T b) { T c = a + b; return c != c ? zero() : c; }
    __host__ __device__ static T star(T a) { return a <= T(0) ? one() : Lim<T>::inf(); }
};

template <class T> struct MaxMin {
    typedef T value_type;
    static constexpr int id = S_MAXMIN;
    static constexpr bool integral = true;
    __host__ __device__ static T zero() { return -Lim<T>::inf(); }
    __host__ __device__ static T one() { return Lim<T>::inf(); }
    __host__ __device__ static T plus(T a, T b) { return pmax(a, b); }
    __host__ __device__ static T muladd(T a, T b, T c) { return pmax(pmin(a, b), c); }
    __host__ __device__ static T muladd2(T a0, T b0, T a1, T b1, T c) { return pmax(pmax(pmin(a0, b0), pmin(a1, b1)), c); }
    __host__ __device__ static T prod(T a, T b) { return pmin(a, b); }
    __host__ __device__ static T star(T) { return one(); }
};

template <class T> struct MinMax {
    typedef T value_type;
    static constexpr int id = S_MINMAX;
    static constexpr bool integral = true;
    __host__ __device__ static T zero() { return Lim<T>::inf(); }
    __host__ __device__ static T one() { return -Lim<T>::inf(); }
    __host__ __device__ static T plus(T a, T b) { return pmin(a, b); }
    __host__ __device__ static T muladd(T a, T b, T c) { return pmin(pmax(a, b), c); }
    __host__ __device__ static T muladd2(T a0, T b0, T a1, T b1, T c) { return pmin(pmin(pmax(a0, b0), pmax(a1, b1)), c); }
    __host__ __device__ static T prod(T a, T b) { return pmax(a, b); }
    __host__ __device__ static T star(T) { return one(); }
};

template <class T> struct PlusProd {
    typedef T value_type;
    static constexpr int id = S_PLUSPROD;
    static constexpr bool integral = false;
    __host__ __device__ static T zero() { return T(0); }
    __host__ __device__ static T one() { return T(1); }
    __host__ __device__ static T plus(T a, T b) { return a + b; }
    __host__ __device__ static T muladd(T a, T b, T c) { return __builtin_fma(a, b, c); }
    __host__ __device__ static T muladd2(T a0, T b0, T a1, T b1, T c) { return muladd(a1, b1, muladd(a0, b0, c)); }
    __host__ __device__ static T prod(T a, T b) { return a * b; }
    __host__ __device__ static T star(T a) { return a < T(1) ? T(1) / (T(1) - a) : Lim<T>::inf(); }
};
template <> __host__ __device__ inline float PlusProd<float>::muladd(float a, float b, float c) {
    return __builtin_fmaf(a, b, c);
}

struct OrAnd {
    typedef int32_t value_type;
    static constexpr int id = S_ORAND;
    static constexpr bool integral = true;
    __host__ __device__ static int32_t zero() { return 0; }
    __host__ __device__ static int32_t one() { return 0x7fffffff; }
    __host__ __device__ static int32_t plus(int32_t a, int32_t b) { return a | b; }
    __host__ __device__ static int32_t muladd(int32_t a, int32_t b, int32_t c) { return (a & b) | c; }
    __host__ __device__ static int32_t muladd2(int32_t a0, int32_t b0, int32_t a1, int32_t b1, int32_t c) {
        return (a0 & b0) | (a1 & b1) | c;
    }
    __host__ __device__ static int32_t prod(int32_t a, int32_t b) { return a & b; }
    __host__ __device__ static int32_t star(int32_t) { return one(); }
};

// Call F.template operator()<S>() for the semiring/type pair; returns false when the pair is unsupported.
template <class Fn> bool dispatch(int semiring, int dtype, Fn &&fn) {
    if (dtype == D_F32) {
        switch (semiring) {
        case S_MINPLUS: fn.template operator()<MinPlus<float>>(); return true;
        case S_MAXPLUS: fn.template operator()<MaxPlus<float>>(); return true;
        case S_MAXMIN: fn.template operator()<MaxMin<float>>(); return true;
        case S_MINMAX: fn.template operator()<MinMax<float>>(); return true;
        case S_PLUSPROD: fn.template operator()<PlusProd<float>>(); return true;
        }
    } else if (dtype == D_F64) {
        switch (semiring) {
        case S_MINPLUS: fn.template operator()<MinPlus<double>>(); return true;
        case S_MAXPLUS: fn.template operator()<MaxPlus<double>>(); return true;
        case S_MAXMIN: fn.template operator()<MaxMin<double>>(); return true;
        case S_MINMAX: fn.template operator()<MinMax<double>>(); return true;
        case S_PLUSPROD: fn.template operator()<PlusProd<double>>(); return true;
        }
    } else if (dtype == D_I32 && semiring == S_ORAND) {
        fn.template operator()<OrAnd>();
        return true;
    }
    return false;
}

inline int dtype_size(int dtype) { return dtype == D_F64 ? 8 : 4; }

}  // namespace pp
