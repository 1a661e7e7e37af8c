// DefaultStrategy steps written against the C++ class surface
// (include/tinygs_amd/tinygs.hpp): create_optimizer / create_strategy over
// shared GPUGaussian3d, with the densification info of every step given.
//
// Usage: densify_step <input.bin> <output.bin>
// input  (little endian): int64 n; int32 sh_half; float scene_scale, grad_scaler;
//        uint32 width, height; int32 n_keys, then n_keys x (char name[48], double value)
//        strategy parameters; int32 steps;
//        float means[3n], opacities[n], rotations[4n], scales[3n], sh0[3n], sh_rest[45n];
//        float first moments and second moments of the six groups in that order;
//        per step: int64 rows; float info[4 rows]
// output: int64 n_final; the six parameter arrays (SH as float); first and
//         second moments of the six groups; per step int64 duplicated, split,
//         kept; uint64 rng state, inc.
#include <cstdio>
#include <fstream>

#include "tinygs_amd/tinygs.hpp"

using namespace tinygs_amd;

template <class T>
static void rd(std::ifstream& f, T* p, size_t n) {
    f.read(reinterpret_cast<char*>(p), sizeof(T) * n);
    if (!f) throw std::runtime_error("short input file");
}
template <class T>
static void wr(std::ofstream& f, const T* p, size_t n) {
    f.write(reinterpret_cast<const char*>(p), sizeof(T) * n);
}

static const size_t kMult[6] = {3, 1, 4, 3, 3, 45};

int main(int argc, char** argv) {
    if (argc != 3) {
        std::fprintf(stderr, "usage: %s <input.bin> <output.bin>\n", argv[0]);
        return 2;
    }
    try {
        std::ifstream in(argv[1], std::ios::binary);
        int64_t n = 0;
        int32_t sh_half = 0, n_keys = 0, steps = 0;
        float scene_scale = 1.0f, grad_scaler = 1.0f;
        uint32_t wh[2] = {0, 0};
        rd(in, &n, 1);
        rd(in, &sh_half, 1);
        rd(in, &scene_scale, 1);
        rd(in, &grad_scaler, 1);
        rd(in, wh, 2);
        rd(in, &n_keys, 1);
        ParamMap cfg;
        for (int k = 0; k < n_keys; ++k) {
            char name[48];
            double v = 0.0;
            rd(in, name, 48);
            rd(in, &v, 1);
            name[47] = 0;
            cfg[name] = v;
        }
        rd(in, &steps, 1);
        Gaussian3d host;
        std::vector<float>* arr[6] = {&host.means, &host.opacities, &host.rotations, &host.scales,
                                      &host.sh_coefficient_0, &host.sh_coefficients_rest};
        for (int k = 0; k < 6; ++k) {
            arr[k]->resize(kMult[k] * (size_t)n);
            rd(in, arr[k]->data(), arr[k]->size());
        }
        std::vector<float> mom[2][6];
        for (int b = 0; b < 2; ++b)
            for (int k = 0; k < 6; ++k) {
                mom[b][k].resize(kMult[k] * (size_t)n);
                rd(in, mom[b][k].data(), mom[b][k].size());
            }

        auto g = std::make_shared<GPUGaussian3d>((size_t)n, sh_half ? DataType::Float16 : DataType::Float32);
        g->copy_from_host(host);
        g->set_scene_scale(scene_scale);
        auto grads = g->gradient_like();
        auto opt = create_optimizer("simple_adam", g, grads);
        auto* adam = dynamic_cast<SimpleAdam*>(opt.get());
        for (int b = 0; b < 2; ++b)
            for (int k = 0; k < 6; ++k) {
                auto mm = adam->moments(k);
                hip_check(hipMemcpy(b == 0 ? mm.first : mm.second, mom[b][k].data(), 4 * mom[b][k].size(),
                                    hipMemcpyHostToDevice),
                          "hipMemcpy");
            }
        auto strategy = create_strategy("default", g, grads, opt.get());
        strategy->set_params(cfg);
        auto* ds = dynamic_cast<DefaultStrategy*>(strategy.get());
        RasterizeContext ctx;
        ctx.fwd_input.width = wh[0];
        ctx.fwd_input.height = wh[1];
        ctx.grad_scaler = grad_scaler;
        std::vector<int64_t> counts;
        for (int st = 0; st < steps; ++st) {
            int64_t rows = 0;
            rd(in, &rows, 1);
            std::vector<float> info(4 * (size_t)rows);
            rd(in, info.data(), info.size());
            if ((size_t)rows != g->size()) throw std::runtime_error("info rows do not match the Gaussians");
            ctx.densification_info = std::make_shared<GPUBuffer<DensificationInfo>>((size_t)rows);
            hip_check(hipMemcpy(ctx.densification_info->data(), info.data(), 4 * info.size(), hipMemcpyHostToDevice),
                      "hipMemcpy");
            ds->last_duplicated = ds->last_split = ds->last_kept = -1;
            strategy->step(ctx);
            counts.push_back(ds->last_duplicated);
            counts.push_back(ds->last_split);
            counts.push_back(ds->last_kept);
        }
        hip_check(hipDeviceSynchronize(), "hipDeviceSynchronize");

        std::ofstream out(argv[2], std::ios::binary);
        const int64_t nf = (int64_t)g->size();
        wr(out, &nf, 1);
        Gaussian3d res;
        g->copy_to_host(res);
        const std::vector<float>* ra[6] = {&res.means, &res.opacities, &res.rotations, &res.scales,
                                           &res.sh_coefficient_0, &res.sh_coefficients_rest};
        for (int k = 0; k < 6; ++k) wr(out, ra[k]->data(), ra[k]->size());
        for (int b = 0; b < 2; ++b)
            for (int k = 0; k < 6; ++k) {
                std::vector<float> h(kMult[k] * (size_t)nf);
                auto mm = adam->moments(k);
                hip_check(hipMemcpy(h.data(), b == 0 ? mm.first : mm.second, 4 * h.size(), hipMemcpyDeviceToHost),
                          "hipMemcpy");
                wr(out, h.data(), h.size());
            }
        wr(out, counts.data(), counts.size());
        const uint64_t rng[2] = {ds->rng().state, ds->rng().inc};
        wr(out, rng, 2);
        return 0;
    } catch (const std::exception& e) {
        std::fprintf(stderr, "densify_step: %s\n", e.what());
        return 1;
    }
}
