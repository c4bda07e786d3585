// expert_dispatch.h - the host side of the expert-matmul path over
// libeahmmf_hip.so: when an expert matmul goes to the GPU, when it falls back
// to the CPU, the gate/up pair, the counters, and the shadow check of a GPU
// result against the CPU kernel.
//
// It restates, over the HIP C ABI, the reference's dispatch in
// qwen3moe.cpp:
//   gpu_matmul        :471-474   GPU only if the view has a device pointer and
//                                the type is Q8_0/Q4_K/Q5_K/Q6_K
//   gpu_matmul_pair   :476-491   gate and up of equal shape in one call
//   expert_matmul     :512-525   a false return (or no device copy) means the
//                                CPU kernel computes the result; counted
//   the MoE loop      :1035-1055 the pair unless EAHMMF_DISABLE_PAIR is set,
//                                else two single calls
//   shadow            :449-458, :494-508   max|cpu - gpu| / max(max|cpu|, 1e-3)
//                                must stay below 1e-4; the CPU result is
//                                computed and compared, the GPU result kept
// Header-only and templated on the weight-view type (fields dev, type, ne0,
// ne1, row_bytes, as the reference's eahmmf::WeightView, eahmmf.h:54-62) and
// on the CPU matmul (the reference's matmul(W, x, nb, ldx, out, ldo),
// qwen3moe.cpp:397-419), so the reference's engine can use it as it stands.
#ifndef EAHMMF_HIP_EXPERT_DISPATCH_H
#define EAHMMF_HIP_EXPERT_DISPATCH_H
#include <math.h>
#include <stdint.h>
#include <stdlib.h>

#include <vector>

#include "eahmmf_hip.h"

namespace eahmmf_hip {

// The reference's counters (g_gpu_calls, g_gpu_fallbacks, g_pair_calls,
// g_sh_calls, g_sh_bad, g_sh_max_rel; qwen3moe.cpp:425-470).
struct DispatchStats {
    long gpu_calls = 0, cpu_fallbacks = 0, pair_calls = 0;
    long shadow_calls = 0, shadow_bad = 0;
    double shadow_max_rel = 0.0;
};

inline bool gpu_type_supported(uint32_t t) { return t == 8 || t == 12 || t == 13 || t == 14; }

// The shadow criterion: max|cpu - gpu| / max(max|cpu|, 1e-3) over the first
// n values of nb rows at stride ld.
inline double shadow_rel_err(const float* cpu, const float* gpu, int nb, int n, int ld) {
    double maxerr = 0.0, maxout = 1e-3;
    for (int t = 0; t < nb; t++)
        for (int r = 0; r < n; r++) {
            const double c = cpu[(size_t)t * ld + r], g = gpu[(size_t)t * ld + r];
            maxerr = fmax(maxerr, fabs(c - g));
            maxout = fmax(maxout, fabs(c));
        }
    return maxerr / maxout;
}

template <class View>
bool gpu_matmul(const View& W, const float* x, int nb, int ldx, float* out, int ldo) {
    if (!W.dev || !gpu_type_supported((uint32_t)W.type)) return false;
    return eahmmf_hip_matmul(W.dev, (int)W.type, (int)W.ne0, (int)W.ne1, W.row_bytes, x, nb, ldx, out, ldo);
}

template <class View>
bool gpu_matmul_pair(const View& G, const View& U, const float* x, int nb, int ldx, float* gout, int ldg, float* uout,
                     int ldu) {
    if (!G.dev || !U.dev || !gpu_type_supported((uint32_t)G.type) || !gpu_type_supported((uint32_t)U.type))
        return false;
    if (G.ne0 != U.ne0 || G.ne1 != U.ne1) return false;
    return eahmmf_hip_matmul_pair(G.dev, (int)G.type, (int)G.ne0, (int)G.ne1, G.row_bytes, U.dev, (int)U.type,
                                  (int)U.ne0, (int)U.ne1, U.row_bytes, x, nb, ldx, gout, ldg, uout, ldu);
}

// The shadow check of a GPU result: the CPU kernel's result is computed and
// compared; the GPU result stays in `out`.
template <class View, class CpuMatmul>
void shadow_compare(const View& W, const float* x, int nb, int ldx, const float* gpu_out, int ldo, CpuMatmul&& cpu,
                    DispatchStats& st) {
    std::vector<float> c((size_t)nb * ldo, 0.f);
    cpu(W, x, nb, ldx, c.data(), ldo);
    const double rel = shadow_rel_err(c.data(), gpu_out, nb, (int)W.ne1, ldo);
    st.shadow_calls++;
    st.shadow_max_rel = fmax(st.shadow_max_rel, rel);
    if (!(rel < 1e-4)) st.shadow_bad++;
}

// One expert matmul: GPU when the view has a device copy and the call
// succeeds, else the CPU kernel (counted as a fallback).
template <class View, class CpuMatmul>
void expert_matmul(const View& W, const float* x, int nb, int ldx, float* out, int ldo, CpuMatmul&& cpu,
                   DispatchStats& st, bool shadow) {
    if (gpu_matmul(W, x, nb, ldx, out, ldo)) {
        st.gpu_calls++;
        if (shadow) shadow_compare(W, x, nb, ldx, out, ldo, cpu, st);
        return;
    }
    st.cpu_fallbacks++;
    cpu(W, x, nb, ldx, out, ldo);
}

// Gate and up of one expert: the pair call unless EAHMMF_DISABLE_PAIR is set
// or the pair does not apply, else two expert_matmul calls.
template <class View, class CpuMatmul>
void expert_matmul_gate_up(const View& G, const View& U, const float* x, int nb, int ldx, float* gout, int ldg,
                           float* uout, int ldu, CpuMatmul&& cpu, DispatchStats& st, bool shadow) {
    if (getenv("EAHMMF_DISABLE_PAIR") == nullptr && gpu_matmul_pair(G, U, x, nb, ldx, gout, ldg, uout, ldu)) {
        st.pair_calls++;
        st.gpu_calls += 2;
        if (shadow) {
            shadow_compare(G, x, nb, ldx, gout, ldg, cpu, st);
            shadow_compare(U, x, nb, ldx, uout, ldu, cpu, st);
        }
        return;
    }
    expert_matmul(G, x, nb, ldx, gout, ldg, cpu, st, shadow);
    expert_matmul(U, x, nb, ldx, uout, ldu, cpu, st, shadow);
}

}  // namespace eahmmf_hip
#endif
