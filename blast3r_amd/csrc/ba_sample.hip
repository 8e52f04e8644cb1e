// F sampling: the multi-depth values of every observation, bilinearly sampled from its image's map.
//
// Restates gather_data_from_dense_tracks (src/blast3r/inference/tracks.py:865-872), which calls
// bilinear_sampling (src/blast3r/utils/geometry.py:167-198) once per image, as one launch over all
// images.  For a pixel (x, y) of an H x W map with Cm channels:
//   grid coordinate     g = x * fl32(2 / W) - 1, two roundings          (geometry.py:188)
//   source index        i = fma(g + 1, W, -1) / 2, clamped to [0, W-1]  (grid_sample with
//                       align_corners=False, padding_mode='border', geometry.py:189-193)
//   weights             nw = (x0 + 1 - i)(y0 + 1 - j), ne = (i - x0)(y0 + 1 - j),
//                       sw = (x0 + 1 - i)(j - y0), se = (i - x0)(j - y0)
//   value               v = map[nw] * nw, then v = fma(map[c], c, v) for c = ne, sw, se; corners
//                       past the last row or column are skipped.
// These are the roundings torch's CPU grid_sample performs (its unnormalise and its corner sum are
// fused multiply-adds), so the kernel reproduces that routine bit for bit.
//
// Optionally a constant-one channel is sampled at output column 1 (the channel stack
// [F0, 1, F1, ...] of src/blast3r/inference/multidepth.py:53-54), so that callers holding the raw
// K-channel maps need not build the stacked copy.
//
// Memory: observations are image-major, so the blocks of one image gather from one map (a few MB,
// resident in L2 / MALL while they run); each block stages its output rows in LDS and writes them
// as one contiguous run.  (Laying the blocks out so that each XCD takes a contiguous range of them
// cut the fetched bytes from 2.72 to 2.04 GB per launch at config 2 but took 4% longer: the kernel
// is bound by its gathers' latency, not by the bytes.)
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "ba_common.h"
#include "ba_error.h"

// Every fp32 expression below rounds on its own: no multiply-add contraction in this file.  The two
// fused steps are written as fmaf.  (HIP's __fmul_rn / __fadd_rn are plain operators in its headers
// and would be contracted there, so they are not used.)
#pragma clang fp contract(off)

namespace ba {

#define SMP_T 256

// the map addresses come from a device table, so the compiler cannot infer their address space:
// state it, so that texel reads are global (not flat) loads
typedef const __attribute__((address_space(1))) float gfloat;

__device__ __forceinline__ float src_index(float pix, int size) {
    const float sc = 2.0f / (float)size;                        // correctly rounded division
    const float g = pix * sc - 1.0f;
    const float i = fmaf(g + 1.0f, (float)size, -1.0f) * 0.5f;
    return fminf((float)(size - 1), fmaxf(i, 0.0f));
}

// CM > 0: channel count fixed at compile time (output rows staged in LDS); CM == 0: a.Cm at run time.
template <int CM, int INS>
__global__ void __launch_bounds__(SMP_T) k_sample(ba_sample_args a) {
    constexpr int STAGE_C = CM > 0 ? CM + INS : 1;
    __shared__ float sOut[SMP_T * STAGE_C];
    const int cm = CM > 0 ? CM : a.Cm;
    const int co = cm + INS;
    const int ps = a.pix_stride > 0 ? a.pix_stride : cm;
    const int64_t o0 = (int64_t)blockIdx.x * SMP_T;
    const int nloc = (int)(a.n_obs - o0 < SMP_T ? a.n_obs - o0 : SMP_T);
    const int t = threadIdx.x;
    if (t < nloc) {
        const int64_t o = o0 + t;
        const int img = obs_image(a.cum_nppi, (int)a.n_imgs, (int)o);
        int H = a.H, W = a.W;
        if (a.map_hw != nullptr) { H = a.map_hw[2 * img]; W = a.map_hw[2 * img + 1]; }
        const bool empty = H < 1 || W < 1;                         // an empty map gives a NaN row, nothing is read
        if (empty) H = W = 1;
        const gfloat* map = reinterpret_cast<const gfloat*>(a.map_addr[img]);
        const float2 p = reinterpret_cast<const float2*>(a.pix2d)[o];
        const float ix = src_index(p.x, W), iy = src_index(p.y, H);
        const float fx0 = floorf(ix), fy0 = floorf(iy);
        const int x0 = (int)fx0, y0 = (int)fy0;
        const bool xin = x0 + 1 < W, yin = y0 + 1 < H;            // east column / south row inside the map
        const float e = (fx0 + 1.0f) - ix, w = ix - fx0;
        const float s = (fy0 + 1.0f) - iy, n = iy - fy0;
        const float wnw = e * s, wne = w * s, wsw = e * n, wse = w * n;
        // texel addresses; a corner outside the map reads its in-map neighbour and is masked out below
        const int64_t rn = (int64_t)y0 * W, rs = (int64_t)(yin ? y0 + 1 : y0) * W;
        const int xe = xin ? x0 + 1 : x0;
        const gfloat* pnw = map + (rn + x0) * ps;
        const gfloat* pne = map + (rn + xe) * ps;
        const gfloat* psw = map + (rs + x0) * ps;
        const gfloat* pse = map + (rs + xe) * ps;
        float* dst = CM > 0 ? sOut + t * STAGE_C : a.out + o * co;
        auto mix = [&](float vnw, float vne, float vsw, float vse) {
            float v = vnw * wnw;
            if (xin) v = fmaf(vne, wne, v);
            if (yin) v = fmaf(vsw, wsw, v);
            if (xin && yin) v = fmaf(vse, wse, v);
            return v;
        };
        if (empty) {
            for (int c = 0; c < cm; ++c) dst[INS && c > 0 ? c + 1 : c] = __builtin_nanf("");
        } else if constexpr (CM > 0) {
            // all 4 CM texel values are requested before the first one is used
            float vnw[CM], vne[CM], vsw[CM], vse[CM];
#pragma unroll
            for (int c = 0; c < CM; ++c) { vnw[c] = pnw[c]; vne[c] = pne[c]; vsw[c] = psw[c]; vse[c] = pse[c]; }
#pragma unroll
            for (int c = 0; c < CM; ++c) dst[INS && c > 0 ? c + 1 : c] = mix(vnw[c], vne[c], vsw[c], vse[c]);
        } else {
            for (int c = 0; c < cm; ++c) dst[INS && c > 0 ? c + 1 : c] = mix(pnw[c], pne[c], psw[c], pse[c]);
        }
        if (INS) {                                   // the constant-one channel: fma(1, w, v) = v + w
            float v = empty ? __builtin_nanf("") : wnw;
            if (xin) v = v + wne;
            if (yin) v = v + wsw;
            if (xin && yin) v = v + wse;
            dst[1] = v;
        }
    }
    if (CM > 0) {
        __syncthreads();
        float* out = a.out + o0 * STAGE_C;
        for (int q = t; q < nloc * STAGE_C; q += SMP_T) out[q] = sOut[q];
    }
}

template <int INS>
static void launch_ins(const ba_sample_args& a, unsigned nb, hipStream_t st) {
    switch (a.Cm) {
#define BA_SMP_CASE(c) \
    case c: hipLaunchKernelGGL((k_sample<c, INS>), dim3(nb), dim3(SMP_T), 0, st, a); return;
        BA_SMP_CASE(1) BA_SMP_CASE(2) BA_SMP_CASE(3) BA_SMP_CASE(4) BA_SMP_CASE(5) BA_SMP_CASE(6)
        BA_SMP_CASE(7) BA_SMP_CASE(8) BA_SMP_CASE(9) BA_SMP_CASE(10) BA_SMP_CASE(11) BA_SMP_CASE(12)
        BA_SMP_CASE(13) BA_SMP_CASE(14) BA_SMP_CASE(15) BA_SMP_CASE(16)
#undef BA_SMP_CASE
        default: hipLaunchKernelGGL((k_sample<0, INS>), dim3(nb), dim3(SMP_T), 0, st, a); return;
    }
}

}  // namespace ba

using namespace ba;

extern "C" int ba_sample_depth(const ba_sample_args* args, void* stream) {
    clear_error();
    BA_REQUIRE(args != nullptr, "null args");
    const ba_sample_args& a = *args;
    BA_REQUIRE(a.n_obs >= 0 && a.n_imgs >= 0 && a.n_obs < (int64_t)1 << 31, "bad sizes");
    BA_REQUIRE(a.Cm >= 1 && a.Cm <= 1024, "map channels must be in [1, 1024]");
    BA_REQUIRE(a.pix_stride == 0 || a.pix_stride >= a.Cm, "pix_stride must be 0 or at least Cm");
    BA_REQUIRE(a.insert_ones == 0 || a.insert_ones == 1, "insert_ones must be 0 or 1");
    if (a.n_obs == 0) return BA_OK;
    BA_REQUIRE(a.n_imgs >= 1, "observations without images");
    BA_REQUIRE(a.map_hw != nullptr || (a.H >= 1 && a.W >= 1), "map size must be at least 1 x 1");
    BA_REQUIRE(a.map_addr && a.cum_nppi && a.pix2d && a.out, "null pointer");
    const unsigned nb = (unsigned)((a.n_obs + SMP_T - 1) / SMP_T);
    hipStream_t st = (hipStream_t)stream;
    if (a.insert_ones) launch_ins<1>(a, nb, st); else launch_ins<0>(a, nb, st);
    BA_LAUNCHED();
    return BA_OK;
}
