// One training iteration written against the C++ class surface
// (include/tinygs_amd/tinygs.hpp) in the order of Orchestrator::train_step
// (tinygs/src/orchestrator.cu:335-439): zero gradients and loss images,
// forward, L1 / fused SSIM losses, backward (accumulating), SimpleAdam step.
//
// Usage: train_step <input.bin> <output.bin>
// input  (little endian): int64 n; int32 sh_degree, sh_half, image_half; uint32 width, height;
//        float near, far, K[9], w2c[16], l1_weight, ssim_weight, grad_scaler, epsilon, shs_lr;
//        float means[3n], scales[3n], rotations[4n], opacities[n], sh0[3n], sh_rest[45n];
//        target[3 * channel_stride] (8x8-tiled planar; float, or half bits when image_half)
// output: image[3 * channel_stride], grad_image[3 * channel_stride] (float, or half bits
//         when image_half: the training data type of the reference's float16 configs,
//         configs/default.json:99, which renders with the fp16-image rasterizer);
//         gradients means, scales, rotations, opacities, sh0, sh_rest (fp32);
//         parameters after the step in the same order (SH as float);
//         int64 n_visible, n_instances, n_tiles.
#include <cstdio>
#include <fstream>
#include <iostream>

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

int main(int argc, char** argv) {
    if (argc != 3) {
        std::fprintf(stderr, "usage: %s <input.bin> <output.bin>\n", argv[0]);
        return 2;
    }
    try {
        std::ifstream in(argv[1], std::ios::binary);
        if (!in) throw std::runtime_error("cannot open input");
        int64_t n;
        int32_t sh_degree, sh_half, image_half;
        GPUBatchInput cam;
        float l1_w, ssim_w, grad_scaler, eps, shs_lr;
        rd(in, &n, 1);
        rd(in, &sh_degree, 1);
        rd(in, &sh_half, 1);
        rd(in, &image_half, 1);
        rd(in, &cam.width, 1);
        rd(in, &cam.height, 1);
        rd(in, &cam.near, 1);
        rd(in, &cam.far, 1);
        rd(in, cam.K.data(), 9);
        rd(in, cam.w2c.data(), 16);
        rd(in, &l1_w, 1);
        rd(in, &ssim_w, 1);
        rd(in, &grad_scaler, 1);
        rd(in, &eps, 1);
        rd(in, &shs_lr, 1);
        Gaussian3d host;
        host.means.resize(3 * n);
        host.scales.resize(3 * n);
        host.rotations.resize(4 * n);
        host.opacities.resize(n);
        host.sh_coefficient_0.resize(3 * n);
        host.sh_coefficients_rest.resize(45 * n);
        rd(in, host.means.data(), 3 * n);
        rd(in, host.scales.data(), 3 * n);
        rd(in, host.rotations.data(), 4 * n);
        rd(in, host.opacities.data(), n);
        rd(in, host.sh_coefficient_0.data(), 3 * n);
        rd(in, host.sh_coefficients_rest.data(), 45 * n);
        const ImageShape shape{cam.width, cam.height, 3};
        const size_t img_n = (size_t)shape.padded_size();
        const DataType img_dt = image_half ? DataType::Float16 : DataType::Float32;
        // images as 4-byte words: a half image fills the first half of its buffer
        const size_t img_words = image_half ? (img_n + 1) / 2 : img_n;
        const size_t img_bytes = image_half ? 2 * img_n : 4 * img_n;
        std::vector<float> target(img_words);
        rd(in, reinterpret_cast<char*>(target.data()), img_bytes);

        auto gaussians = std::make_shared<GPUGaussian3d>(0, sh_half ? DataType::Float16 : DataType::Float32);
        gaussians->copy_from_host(host);
        gaussians->set_sh_degree(sh_degree);
        auto grads = gaussians->gradient_like();

        DeviceArray<float> pred(img_words), tgt, loss(img_words), grad(img_words);
        tgt.copy_from_host(target.data(), img_words);

        hipStream_t stream;
        hip_check(hipStreamCreate(&stream), "hipStreamCreate");

        auto rasterizer = create_rasterizer("fastgs");
        rasterizer->set_gaussians(gaussians);
        std::vector<std::pair<std::unique_ptr<LossBase>, float>> losses;
        if (l1_w != 0.0f) losses.emplace_back(create_loss("l1"), l1_w);
        if (ssim_w != 0.0f) losses.emplace_back(create_loss("fused_ssim"), ssim_w);
        auto optimizer = create_optimizer("simple_adam", gaussians, grads);
        optimizer->set_params({{"epsilon", eps}, {"shs_lr", shs_lr}});

        RasterizeContext ctx;
        ctx.stream = stream;
        ctx.grad_scaler = grad_scaler;
        ctx.fwd_input = cam;
        ctx.fwd_output.image = Image(shape, img_dt, pred.data());
        ctx.grad_output.image = Image(shape, img_dt, grad.data());
        ctx.gaussians_grad = grads;
        LossContext lctx{ctx.fwd_output.image, Image(shape, img_dt, tgt.data()), Image(shape, img_dt, loss.data()),
                         ctx.grad_output.image, stream};

        // Orchestrator::train_step
        grads->memset_async(0, stream);
        hip_check(hipMemsetAsync(loss.data(), 0, loss.bytes(), stream), "hipMemsetAsync");
        hip_check(hipMemsetAsync(grad.data(), 0, grad.bytes(), stream), "hipMemsetAsync");
        rasterizer->forward(ctx);
        for (auto& [l, w] : losses) l->evaluate(lctx, w * grad_scaler);
        rasterizer->backward(ctx);
        optimizer->step(1.0f / grad_scaler, stream);
        hip_check(hipStreamSynchronize(stream), "hipStreamSynchronize");

        std::ofstream out(argv[2], std::ios::binary);
        const std::vector<float> img_h = pred.to_host(), grad_h = grad.to_host();
        out.write(reinterpret_cast<const char*>(img_h.data()), (std::streamsize)img_bytes);
        out.write(reinterpret_cast<const char*>(grad_h.data()), (std::streamsize)img_bytes);
        Gaussian3d gh, ph;
        grads->copy_to_host(gh);
        gaussians->copy_to_host(ph);
        for (const Gaussian3d* g : {&gh, &ph}) {
            wr(out, g->means.data(), g->means.size());
            wr(out, g->scales.data(), g->scales.size());
            wr(out, g->rotations.data(), g->rotations.size());
            wr(out, g->opacities.data(), g->opacities.size());
            wr(out, g->sh_coefficient_0.data(), g->sh_coefficient_0.size());
            wr(out, g->sh_coefficients_rest.data(), g->sh_coefficients_rest.size());
        }
        const auto counts = static_cast<FastGSRasterizer*>(rasterizer.get())->counts();
        wr(out, counts.data(), 3);
        if (!out) throw std::runtime_error("cannot write output");
        hip_check(hipStreamDestroy(stream), "hipStreamDestroy");

        // error paths: the reference throws on an unknown type and on a
        // prediction / target data type mismatch (l1.cu:110-115)
        try {
            create_loss("l3");
            std::cerr << "expected an exception for an unknown loss\n";
            return 1;
        } catch (const std::runtime_error&) {
        }
        try {
            LossContext bad = lctx;
            bad.target.data_type = image_half ? DataType::Float32 : DataType::Float16;
            create_loss("l1")->evaluate(bad, 1.0f);
            std::cerr << "expected an exception for mixed image data types\n";
            return 1;
        } catch (const std::runtime_error&) {
        }
        // a backward whose gradient image is not of the forward's data type is refused
        try {
            RasterizeContext bad = ctx;
            bad.grad_output.image.data_type = image_half ? DataType::Float32 : DataType::Float16;
            rasterizer->backward(bad);
            std::cerr << "expected an exception for a gradient image of another data type\n";
            return 1;
        } catch (const std::runtime_error&) {
        }
        std::cout << "train_step ok n=" << n << " visible=" << counts[0] << " instances=" << counts[1] << "\n";
        return 0;
    } catch (const std::exception& e) {
        std::cerr << "train_step failed: " << e.what() << "\n";
        return 1;
    }
}
