// tinygs_amd C++ interface: the class surface of tinygs's rasterizer, loss and
// optimizer plugins, implemented over the C ABI in tinygs_amd.h.
//
// Names, argument meaning, accumulation rules and error behaviour follow the
// reference classes so that a caller written against them switches by
// changing includes and the namespace:
//   RasterizeContext / RasterizerBase / create_rasterizer
//       tinygs/include/tinygs/rasterizer/rasterizer.hpp:9-61
//   FastGSRasterizer              tinygs/include/tinygs/rasterizer/fastgs.hpp:14-37
//   LossContext / LossBase        tinygs/include/tinygs/loss/loss.hpp:6-28
//   L1Loss, FusedSSIMLoss         tinygs/include/tinygs/loss/l1.hpp:7-19,
//                                 tinygs/include/tinygs/loss/fused_ssim.hpp:7-17
//   GaussianOptimizationParams, OptimizerBase, create_optimizer
//                                 tinygs/include/tinygs/optim/optim.hpp:8-100
//   SimpleAdam                    tinygs/include/tinygs/optim/simple_adam.hpp:30-60
//   GPUGaussian3d                 tinygs/include/tinygs/core/gpu_gaussian.hpp:9-73
//   Gaussian3d, DensificationInfo tinygs/include/tinygs/core/gaussian.hpp:9-23
//   ImageShape, Image, DataType   tinygs/include/tinygs/core/image.hpp:35-85
//   GPUBatchInput/Output          tinygs/include/tinygs/dataloader/dataloader.hpp:8-19
//
// Differences, all on purpose:
//   * hipStream_t replaces cudaStream_t; DeviceArray<T> (hipMalloc-backed)
//     replaces thrust::device_vector; vec3/vec4 are spelled as float arrays
//     (3 or 4 floats per element, same memory layout as glm).
//   * get_params/set_params take a flat name -> number map instead of json.
//   * Densification and reordering (GPUGaussian3d::remove/append/reorder,
//     SimpleAdam::remove/duplicate/reset(indices)/reorder/reset_opacity,
//     DefaultStrategy) run through the tgs_densify_* / tgs_*_gather /
//     tgs_*_reorder / tgs_adam_reset_rows entry points.
//   * GPUGaussian3d can store sh0 / sh_rest as fp16 (sh_dtype), the storage
//     mode of the 1M-Gaussian 1080p benchmark; gradients stay fp32.
// Every failing call throws std::runtime_error carrying tgs_last_error(), as
// the reference's CUDA_CHECK_THROW (tinygs/include/tinygs/cuda/common_host.hpp:104-109).
#pragma once

#include <hip/hip_runtime.h>

#include <algorithm>
#include <array>
#include <cctype>
#include <cmath>
#include <cstring>
#include <cstdint>
#include <map>
#include <memory>
#include <stdexcept>
#include <string>
#include <type_traits>
#include <utility>
#include <vector>

#include "../tinygs_amd.h"

namespace tinygs_amd {

inline void throw_on(int status, const char* what) {
    if (status != TGS_OK) throw std::runtime_error(std::string(what) + ": " + tgs_last_error());
}

inline void hip_check(hipError_t e, const char* what) {
    if (e != hipSuccess) throw std::runtime_error(std::string(what) + ": " + hipGetErrorString(e));
}

using ParamMap = std::map<std::string, double>;

enum class DataType { Float32 = 0, Float16 = 1 };

// The C ABI's element type of an image or parameter array.
inline int32_t c_dtype(DataType t) { return t == DataType::Float16 ? TGS_DTYPE_FLOAT16 : TGS_DTYPE_FLOAT32; }

// ---------------------------------------------------------------- device memory

template <class T>
class DeviceArray {
public:
    DeviceArray() = default;
    explicit DeviceArray(size_t n) { resize(n); }
    DeviceArray(const DeviceArray&) = delete;
    DeviceArray& operator=(const DeviceArray&) = delete;
    DeviceArray(DeviceArray&& o) noexcept : m_ptr(o.m_ptr), m_size(o.m_size) { o.m_ptr = nullptr; o.m_size = 0; }
    DeviceArray& operator=(DeviceArray&& o) noexcept {
        std::swap(m_ptr, o.m_ptr);
        std::swap(m_size, o.m_size);
        return *this;
    }
    ~DeviceArray() {
        if (m_ptr) (void)hipFree(m_ptr);
    }
    void resize(size_t n) {
        if (n == m_size) return;
        if (m_ptr) hip_check(hipFree(m_ptr), "hipFree");
        m_ptr = nullptr;
        m_size = 0;
        if (n) hip_check(hipMalloc(&m_ptr, n * sizeof(T)), "hipMalloc");
        m_size = n;
    }
    T* data() noexcept { return m_ptr; }
    const T* data() const noexcept { return m_ptr; }
    size_t size() const noexcept { return m_size; }
    size_t bytes() const noexcept { return m_size * sizeof(T); }
    void copy_from_host(const T* src, size_t n) {
        resize(n);
        if (n) hip_check(hipMemcpy(m_ptr, src, n * sizeof(T), hipMemcpyHostToDevice), "hipMemcpy H2D");
    }
    void copy_to_host(T* dst) const {
        if (m_size) hip_check(hipMemcpy(dst, m_ptr, bytes(), hipMemcpyDeviceToHost), "hipMemcpy D2H");
    }
    std::vector<T> to_host() const {
        std::vector<T> v(m_size);
        copy_to_host(v.data());
        return v;
    }

private:
    T* m_ptr = nullptr;
    size_t m_size = 0;
};

template <class T>
using GPUBuffer = DeviceArray<T>;

// ---------------------------------------------------------------- Gaussians

struct DensificationInfo {
    float accum_counter = 0;
    float accum_grad_mean2d = 0;
    float accum_absgrad_mean2d = 0;
    float max_radii_screen = 0;
};

// Host SoA Gaussians: means[3n], opacities[n], rotations[4n] (r,x,y,z),
// scales[3n] (log), sh_coefficient_0[3n], sh_coefficients_rest[45n].
struct Gaussian3d {
    std::vector<float> means, opacities, rotations, scales, sh_coefficient_0, sh_coefficients_rest;
    size_t size() const { return opacities.size(); }
};

class GPUGaussian3d {
public:
    static constexpr int kMaxSphericalHarmonicsDegree = 3;
    static constexpr int kShRestPerGaussian = 15;

    GPUGaussian3d() = default;
    explicit GPUGaussian3d(size_t n, DataType sh_dtype = DataType::Float32) { allocate(n, sh_dtype); }

    void allocate(size_t n, DataType sh_dtype = DataType::Float32) {
        m_sh_dtype = sh_dtype;
        const size_t sh_bytes = sh_dtype == DataType::Float16 ? 2 : 4;
        m_means.resize(3 * n);
        m_opacities.resize(n);
        m_rotations.resize(4 * n);
        m_scales.resize(3 * n);
        // fp16 storage packs two scalars per float slot; round up to keep 16-byte alignment
        m_sh0.resize((3 * n * sh_bytes + 3) / 4);
        m_sh_rest.resize((45 * n * sh_bytes + 3) / 4);
        m_size = n;
    }

    // Parameters in float32; converted to fp16 (round to nearest even) when
    // the storage is fp16.
    void copy_from_host(const Gaussian3d& g) {
        const size_t n = g.size();
        if (g.means.size() != 3 * n || g.rotations.size() != 4 * n || g.scales.size() != 3 * n ||
            g.sh_coefficient_0.size() != 3 * n || g.sh_coefficients_rest.size() != 45 * n)
            throw std::runtime_error("GPUGaussian3d::copy_from_host: inconsistent array sizes");
        allocate(n, m_sh_dtype);
        m_means.copy_from_host(g.means.data(), 3 * n);
        m_opacities.copy_from_host(g.opacities.data(), n);
        m_rotations.copy_from_host(g.rotations.data(), 4 * n);
        m_scales.copy_from_host(g.scales.data(), 3 * n);
        upload_sh(m_sh0, g.sh_coefficient_0);
        upload_sh(m_sh_rest, g.sh_coefficients_rest);
    }

    void copy_to_host(Gaussian3d& g) const {
        g.means = m_means.to_host();
        g.opacities = m_opacities.to_host();
        g.rotations = m_rotations.to_host();
        g.scales = m_scales.to_host();
        g.sh_coefficient_0 = download_sh(m_sh0, 3 * m_size);
        g.sh_coefficients_rest = download_sh(m_sh_rest, 45 * m_size);
    }

    size_t size() const { return m_size; }
    DataType sh_dtype() const { return m_sh_dtype; }

    DeviceArray<float>& means() { return m_means; }
    DeviceArray<float>& opacities() { return m_opacities; }
    DeviceArray<float>& rotations() { return m_rotations; }
    DeviceArray<float>& scales() { return m_scales; }
    DeviceArray<float>& sh_coefficient_0() { return m_sh0; }
    DeviceArray<float>& sh_coefficients_rest() { return m_sh_rest; }
    const DeviceArray<float>& means() const { return m_means; }
    const DeviceArray<float>& opacities() const { return m_opacities; }
    const DeviceArray<float>& rotations() const { return m_rotations; }
    const DeviceArray<float>& scales() const { return m_scales; }
    const DeviceArray<float>& sh_coefficient_0() const { return m_sh0; }
    const DeviceArray<float>& sh_coefficients_rest() const { return m_sh_rest; }

    void memset_async(char value, hipStream_t stream) {
        for (DeviceArray<float>* a : {&m_means, &m_opacities, &m_rotations, &m_scales, &m_sh0, &m_sh_rest})
            if (a->size()) hip_check(hipMemsetAsync(a->data(), value, a->bytes(), stream), "hipMemsetAsync");
    }
    void memset(char value) {
        memset_async(value, nullptr);
        hip_check(hipStreamSynchronize(nullptr), "hipStreamSynchronize");
    }

    std::unique_ptr<GPUGaussian3d> clone_async(hipStream_t stream = nullptr) const {
        auto c = std::make_unique<GPUGaussian3d>(m_size, m_sh_dtype);
        c->m_scene_scale = m_scene_scale;
        c->m_sh_degree = m_sh_degree;
        const DeviceArray<float>* src[] = {&m_means, &m_opacities, &m_rotations, &m_scales, &m_sh0, &m_sh_rest};
        DeviceArray<float>* dst[] = {&c->m_means, &c->m_opacities, &c->m_rotations, &c->m_scales, &c->m_sh0,
                                     &c->m_sh_rest};
        for (int k = 0; k < 6; ++k)
            if (src[k]->size())
                hip_check(hipMemcpyAsync(dst[k]->data(), src[k]->data(), src[k]->bytes(), hipMemcpyDeviceToDevice,
                                         stream),
                          "hipMemcpyAsync");
        return c;
    }
    std::unique_ptr<GPUGaussian3d> clone() const {
        auto c = clone_async(nullptr);
        hip_check(hipStreamSynchronize(nullptr), "hipStreamSynchronize");
        return c;
    }

    // Gradient storage of the same size: always fp32.
    std::shared_ptr<GPUGaussian3d> gradient_like() const {
        auto g = std::make_shared<GPUGaussian3d>(m_size, DataType::Float32);
        g->set_sh_degree(m_sh_degree);
        return g;
    }

    // GPUGaussian3d::remove (gpu_gaussian.cu:117-160): keep the Gaussians with
    // kept_flag[i] != 0 (device bytes, one per Gaussian), num_kept of them, in order.
    void remove(char* kept_flag, int num_kept) {
        if (num_kept < 0 || (size_t)num_kept > m_size)
            throw std::runtime_error("GPUGaussian3d::remove: num_kept out of range");
        DeviceArray<int32_t> rows(std::max<size_t>(m_size, 1));
        int64_t count = 0;
        throw_on(tgs_flags_compact((const uint8_t*)kept_flag, (int64_t)m_size, rows.data(), &count, nullptr),
                 "GPUGaussian3d::remove");
        if (count != num_kept) throw std::runtime_error("GPUGaussian3d::remove: num_kept does not match the flags");
        gather_rows(rows.data(), (size_t)num_kept);
    }
    // The rows rows[0 .. num) (device int32 indices) become the Gaussians.
    void gather_rows(const int32_t* rows, size_t num) {
        GPUGaussian3d g(num, m_sh_dtype);
        const tgs_gaussians src = to_c(), dst = g.to_c();
        if (num) throw_on(tgs_gaussians_gather(&src, &dst, rows, nullptr), "GPUGaussian3d::remove");
        hip_check(hipStreamSynchronize(nullptr), "hipStreamSynchronize");
        adopt(g);
    }
    // GPUGaussian3d::append (gpu_gaussian.cu:162-170): num_dup zero rows appended.
    void append(int num_dup) {
        if (num_dup <= 0) throw std::runtime_error("GPUGaussian3d::append: num_dup must be positive");
        GPUGaussian3d g(m_size + (size_t)num_dup, m_sh_dtype);
        g.memset(0);
        const size_t shb = m_sh_dtype == DataType::Float16 ? 2 : 4;
        const size_t bytes[6] = {12 * m_size, 4 * m_size, 16 * m_size, 12 * m_size, 3 * shb * m_size,
                                 45 * shb * m_size};
        DeviceArray<float>* src[] = {&m_means, &m_opacities, &m_rotations, &m_scales, &m_sh0, &m_sh_rest};
        DeviceArray<float>* dst[] = {&g.m_means, &g.m_opacities, &g.m_rotations, &g.m_scales, &g.m_sh0, &g.m_sh_rest};
        for (int k = 0; k < 6; ++k)
            if (bytes[k]) hip_check(hipMemcpy(dst[k]->data(), src[k]->data(), bytes[k], hipMemcpyDeviceToDevice),
                                    "hipMemcpy");
        adopt(g);
    }
    // GPUGaussian3d::reorder (gpu_gaussian.cu:273-310): in place, row i
    // becomes old row indices[i] (device array of size() indices).
    void reorder(uint32_t* indices, hipStream_t stream = nullptr) {
        const tgs_gaussians g = to_c();
        throw_on(tgs_gaussians_reorder(&g, indices, stream), "GPUGaussian3d::reorder");
    }

    float scene_scale() const { return m_scene_scale; }
    void set_scene_scale(float s) { m_scene_scale = s; }
    void set_sh_degree(int d) { m_sh_degree = std::min(kMaxSphericalHarmonicsDegree, d); }
    int get_sh_degree() const { return m_sh_degree; }

    // Takes g's arrays (and size) in place of this one's; scene scale and SH degree stay.
    void adopt(GPUGaussian3d& g) {
        std::swap(m_means, g.m_means);
        std::swap(m_opacities, g.m_opacities);
        std::swap(m_rotations, g.m_rotations);
        std::swap(m_scales, g.m_scales);
        std::swap(m_sh0, g.m_sh0);
        std::swap(m_sh_rest, g.m_sh_rest);
        std::swap(m_size, g.m_size);
    }

    // C view for the ABI.
    tgs_gaussians to_c() const {
        tgs_gaussians c{};
        c.means = (void*)m_means.data();
        c.scales = (void*)m_scales.data();
        c.rotations = (void*)m_rotations.data();
        c.opacities = (void*)m_opacities.data();
        c.sh0 = (void*)m_sh0.data();
        c.sh_rest = (void*)m_sh_rest.data();
        c.n = (int64_t)m_size;
        c.sh_degree = m_sh_degree;
        c.sh_dtype = m_sh_dtype == DataType::Float16 ? TGS_DTYPE_FLOAT16 : TGS_DTYPE_FLOAT32;
        c.scene_scale = m_scene_scale;
        return c;
    }

private:
    static uint16_t to_half(float f) {  // round to nearest even, IEEE binary16
        uint32_t x;
        std::memcpy(&x, &f, 4);
        const uint32_t sign = (x >> 16) & 0x8000u;
        const uint32_t ax = x & 0x7fffffffu;
        if (ax >= 0x7f800000u) return (uint16_t)(sign | 0x7c00u | (ax > 0x7f800000u ? 0x200u : 0u));
        if (ax >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u);  // rounds to infinity
        if (ax < 0x38800000u) {  // half subnormal or zero: round(|x| / 2^-24)
            const int e = (int)(ax >> 23);
            const int shift = 126 - e;  // |x| / 2^-24 = mant * 2^-shift
            if (e == 0 || shift > 24) return (uint16_t)sign;
            const uint32_t mant = (ax & 0x7fffffu) | 0x800000u;
            uint32_t r = mant >> shift;
            const uint32_t rem = mant & ((1u << shift) - 1u), halfway = 1u << (shift - 1);
            if (rem > halfway || (rem == halfway && (r & 1u))) ++r;
            return (uint16_t)(sign | r);
        }
        uint32_t r = ((ax - 0x38000000u) >> 13);
        const uint32_t rem = ax & 0x1fffu;
        if (rem > 0x1000u || (rem == 0x1000u && (r & 1u))) ++r;
        return (uint16_t)(sign | r);
    }
    static float from_half(uint16_t h) {
        const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
        const uint32_t e = (h >> 10) & 0x1f, m = h & 0x3ff;
        float f;
        if (e == 0) {
            f = std::ldexp((float)m, -24);
            return sign ? -f : f;
        }
        uint32_t x = sign | (e == 31 ? 0x7f800000u | (m << 13) : ((e + 112u) << 23) | (m << 13));
        std::memcpy(&f, &x, 4);
        return f;
    }
    void upload_sh(DeviceArray<float>& dst, const std::vector<float>& src) {
        if (m_sh_dtype == DataType::Float32) {
            dst.copy_from_host(src.data(), src.size());
            return;
        }
        std::vector<uint16_t> h(2 * dst.size(), 0);
        for (size_t i = 0; i < src.size(); ++i) h[i] = to_half(src[i]);
        if (dst.size())
            hip_check(hipMemcpy(dst.data(), h.data(), dst.bytes(), hipMemcpyHostToDevice), "hipMemcpy H2D");
    }
    std::vector<float> download_sh(const DeviceArray<float>& src, size_t count) const {
        if (m_sh_dtype == DataType::Float32) return src.to_host();
        std::vector<uint16_t> h(2 * src.size());
        if (src.size())
            hip_check(hipMemcpy(h.data(), src.data(), src.bytes(), hipMemcpyDeviceToHost), "hipMemcpy D2H");
        std::vector<float> out(count);
        for (size_t i = 0; i < count; ++i) out[i] = from_half(h[i]);
        return out;
    }

    size_t m_size = 0;
    DataType m_sh_dtype = DataType::Float32;
    int m_sh_degree = 0;
    float m_scene_scale = 1.0f;
    DeviceArray<float> m_means, m_opacities, m_rotations, m_scales, m_sh0, m_sh_rest;
};

// ---------------------------------------------------------------- images, camera

constexpr uint32_t kImageTileLog2 = 3;
constexpr uint32_t kImageTileMask = 7;

struct ImageShape {
    uint32_t width = 0, height = 0, channel = 3;
    uint32_t size() const noexcept { return width * height * channel; }
    uint32_t tiled_width() const noexcept { return (width + kImageTileMask) >> kImageTileLog2; }
    uint32_t tiled_height() const noexcept { return (height + kImageTileMask) >> kImageTileLog2; }
    uint32_t padded_width() const noexcept { return tiled_width() << kImageTileLog2; }
    uint32_t padded_height() const noexcept { return tiled_height() << kImageTileLog2; }
    uint32_t padded_size() const noexcept { return padded_width() * padded_height() * channel; }
    uint32_t channel_stride() const noexcept { return padded_width() * padded_height(); }
    bool operator==(const ImageShape& o) const noexcept {
        return width == o.width && height == o.height && channel == o.channel;
    }
    bool operator!=(const ImageShape& o) const noexcept { return !(*this == o); }
};

// Channel-planar, 8x8-tiled element index (tinygs/include/tinygs/common.hpp:366-414).
inline uint32_t tiled_index(const ImageShape& s, uint32_t x, uint32_t y, uint32_t c) {
    return c * s.channel_stride() + ((y >> 3) * s.tiled_width() + (x >> 3)) * 64 + (y & 7) * 8 + (x & 7);
}

struct Image {
    ImageShape shape;
    DataType data_type = DataType::Float32;
    void* data = nullptr;
    Image() = default;
    Image(ImageShape s, DataType t, void* d) : shape(s), data_type(t), data(d) {}
    explicit operator bool() const noexcept { return data != nullptr; }
    uint32_t size() const noexcept { return shape.size(); }
};

// K: glm column-major 3x3 (fx = K[0], fy = K[4], cx = K[6], cy = K[7]);
// w2c: glm column-major 4x4, translation in w2c[12..14].
struct GPUBatchInput {
    uint32_t width = 0, height = 0;
    float near = 0.01f, far = 100.0f;
    std::array<float, 9> K{};
    std::array<float, 16> w2c{};
    uint64_t timestamp = 0;

    tgs_camera to_c() const {
        tgs_camera c{};
        c.width = width;
        c.height = height;
        c.near_plane = near;
        c.far_plane = far;
        std::copy(K.begin(), K.end(), c.K);
        std::copy(w2c.begin(), w2c.end(), c.w2c);
        return c;
    }
};

struct GPUBatchOutput {
    Image image;
};

// ---------------------------------------------------------------- rasterizer

struct RasterizeContext {
    bool prepare_input_gradients = false;
    bool inference = false;
    hipStream_t stream = nullptr;
    float grad_scaler = 1.0f;
    GPUBatchInput fwd_input;
    GPUBatchOutput fwd_output;
    GPUBatchInput grad_input;
    GPUBatchOutput grad_output;
    std::shared_ptr<GPUGaussian3d> gaussians_grad;
    mutable std::shared_ptr<GPUBuffer<DensificationInfo>> densification_info;
};

class RasterizerBase {
public:
    virtual ~RasterizerBase() = default;
    virtual void forward(const RasterizeContext& ctx) = 0;
    virtual void backward(RasterizeContext& ctx) = 0;
    virtual void set_gaussians(std::shared_ptr<GPUGaussian3d> gaussians) { m_gaussians = std::move(gaussians); }
    virtual ParamMap get_params() const = 0;
    virtual void set_params(const ParamMap& p) = 0;

protected:
    std::shared_ptr<GPUGaussian3d> m_gaussians;
};

class FastGSRasterizer final : public RasterizerBase {
public:
    FastGSRasterizer() { throw_on(tgs_rasterizer_create("fastgs", &m_handle), "create_rasterizer"); }
    ~FastGSRasterizer() override {
        if (m_handle) tgs_rasterizer_destroy(m_handle);
    }
    FastGSRasterizer(const FastGSRasterizer&) = delete;
    FastGSRasterizer& operator=(const FastGSRasterizer&) = delete;

    void set_gaussians(std::shared_ptr<GPUGaussian3d> gaussians) override {
        m_gaussians = std::move(gaussians);
        bind();
    }

    // Renders ctx.fwd_input into ctx.fwd_output.image (every padded element
    // written; padding zero). The image's data type selects the rasterizer as
    // in fastgs.cu:143-188: Float32 the fp32 path, Float16 the fp16-image
    // rasterizer (FGS16: half conic and opacity, 8-bit colour, 255-scaled
    // blending). Updates densification max radii when
    // ctx.densification_info is set.
    void forward(const RasterizeContext& ctx) override {
        if (!m_gaussians) throw std::runtime_error("FastGSRasterizer::forward: Gaussians not set");
        const Image& img = ctx.fwd_output.image;
        if (img.shape.width != ctx.fwd_input.width || img.shape.height != ctx.fwd_input.height)
            throw std::runtime_error("FastGSRasterizer::forward: image shape does not match the camera");
        bind();
        const tgs_camera cam = ctx.fwd_input.to_c();
        m_fwd_dtype = img.data_type;
        m_fwd_valid = false;
        throw_on(tgs_rasterizer_forward(m_handle, &cam, img.data, c_dtype(img.data_type), densif(ctx), ctx.stream),
                 "FastGSRasterizer::forward");
        m_fwd_valid = true;
    }

    // Accumulates (+=) dL/dparams into ctx.gaussians_grad from
    // ctx.grad_output.image = dL/dimage. Must follow forward() on the same
    // Gaussians and camera.
    void backward(RasterizeContext& ctx) override { backward(ctx, false); }

    // assign = true writes the gradients (zero for culled Gaussians) instead
    // of accumulating: the caller's zeroing fused into the backward.
    void backward(RasterizeContext& ctx, bool assign) {
        if (!m_gaussians || !ctx.gaussians_grad)
            throw std::runtime_error("FastGSRasterizer::backward: Gaussians or gradient Gaussians not set");
        if (ctx.gaussians_grad->size() != m_gaussians->size())
            throw std::runtime_error("FastGSRasterizer::backward: gradient size does not match the Gaussians");
        // fastgs.cu:273-274: the forward's image type picks the backward (half
        // image and half gradient image after an fp16 forward); the buffers
        // are read with that element size, so they must all be of it
        if (m_fwd_valid && (ctx.fwd_output.image.data_type != m_fwd_dtype ||
                            ctx.grad_output.image.data_type != m_fwd_dtype))
            throw std::runtime_error("FastGSRasterizer::backward: image / gradient image data type differs from "
                                     "the forward's image");
        const tgs_gaussians g = ctx.gaussians_grad->to_c();
        const int32_t flags = (assign ? TGS_BACKWARD_ASSIGN : 0) | (m_pose_opt ? TGS_BACKWARD_POSE : 0);
        throw_on(tgs_rasterizer_backward_ex(m_handle, ctx.grad_output.image.data, ctx.fwd_output.image.data, &g,
                                            densif(ctx), flags, ctx.stream),
                 "FastGSRasterizer::backward");
        // fastgs.cu:373-383: grad_input.w2c is the pose gradient, zero without pose optimisation
        if (m_pose_opt)
            throw_on(tgs_rasterizer_grad_w2c(m_handle, ctx.grad_input.w2c.data(), ctx.stream),
                     "FastGSRasterizer::backward");
        else
            ctx.grad_input.w2c.fill(0.0f);
    }

    // Visible primitives, instances and tiles of the last forward.
    std::array<int64_t, 3> counts() const {
        int64_t v = 0, i = 0, t = 0;
        throw_on(tgs_rasterizer_counts(m_handle, &v, &i, &t), "FastGSRasterizer::counts");
        return {v, i, t};
    }

    // enable_pose_opt turns on the pose gradient (FastGSRasterizerParams,
    // tinygs/include/tinygs/rasterizer/fastgs.hpp:6-12). The reference's
    // set_params ignores its argument (fastgs.cu:398), so there the flag keeps
    // its default (off); here it can be set.
    ParamMap get_params() const override {
        return {{"f16_grad_scaler", 1.0}, {"enable_pose_opt", m_pose_opt ? 1.0 : 0.0}};
    }
    void set_params(const ParamMap& p) override {
        auto it = p.find("enable_pose_opt");
        if (it != p.end()) m_pose_opt = it->second != 0.0;
    }

    tgs_rasterizer* handle() const { return m_handle; }

private:
    bool m_pose_opt = false;
    DataType m_fwd_dtype = DataType::Float32;   // image type of the last forward
    bool m_fwd_valid = false;
    void bind() {
        const tgs_gaussians g = m_gaussians->to_c();
        throw_on(tgs_rasterizer_set_gaussians(m_handle, &g), "FastGSRasterizer::set_gaussians");
    }
    static void* densif(const RasterizeContext& ctx) {
        return ctx.densification_info ? (void*)ctx.densification_info->data() : nullptr;
    }
    tgs_rasterizer* m_handle = nullptr;
};

inline std::unique_ptr<RasterizerBase> create_rasterizer(const std::string& type) {
    std::string t = type;
    std::transform(t.begin(), t.end(), t.begin(), [](unsigned char c) { return (char)std::tolower(c); });
    if (t == "fastgs") return std::make_unique<FastGSRasterizer>();
    throw std::runtime_error("Unknown rasterizer type: " + type);
}

// ---------------------------------------------------------------- losses

struct LossContext {
    Image pred, target, loss, grad;
    hipStream_t stream = nullptr;
};

class LossBase {
public:
    virtual ~LossBase() = default;
    // Accumulates loss and gradient: loss[i] += ..., grad[i] += ...
    virtual void evaluate(LossContext ctx, float scale) = 0;
    virtual std::string name() const = 0;
};

class FusedLoss : public LossBase {
public:
    explicit FusedLoss(const char* type) : m_name(type) { throw_on(tgs_loss_create(type, &m_handle), "create_loss"); }
    ~FusedLoss() override {
        if (m_handle) tgs_loss_destroy(m_handle);
    }
    FusedLoss(const FusedLoss&) = delete;
    FusedLoss& operator=(const FusedLoss&) = delete;

    // l1.cu:109-151, fused_ssim.cu:797-916: the target's data type selects
    // the fp32 or fp16 kernels; prediction, loss and gradient images are of it.
    void evaluate(LossContext ctx, float scale) override {
        if (ctx.pred.shape != ctx.target.shape)
            throw std::runtime_error(m_name + ": prediction and target shapes differ");
        const DataType dt = ctx.target.data_type;
        if (ctx.pred.data_type != dt)
            throw std::runtime_error(m_name + ": prediction and target data type must be the same");
        if ((ctx.loss && ctx.loss.data_type != dt) || (ctx.grad && ctx.grad.data_type != dt))
            throw std::runtime_error(m_name + ": loss / gradient image data type differs from the target's");
        tgs_loss_context c{};
        c.pred = ctx.pred.data;
        c.target = ctx.target.data;
        c.loss = ctx.loss.data;
        c.grad = ctx.grad.data;
        c.width = ctx.pred.shape.width;
        c.height = ctx.pred.shape.height;
        c.channel = ctx.pred.shape.channel;
        c.dtype = c_dtype(dt);
        throw_on(tgs_loss_evaluate(m_handle, &c, scale, ctx.stream), m_name.c_str());
    }
    std::string name() const override { return m_name; }

private:
    std::string m_name;
    tgs_loss* m_handle = nullptr;
};

class L1Loss final : public FusedLoss {
public:
    L1Loss() : FusedLoss("l1") {}
};

class FusedSSIMLoss final : public FusedLoss {
public:
    FusedSSIMLoss() : FusedLoss("fused_ssim") {}
};

inline std::unique_ptr<LossBase> create_loss(const std::string& type) {
    if (type == "l1") return std::make_unique<L1Loss>();
    if (type == "fused_ssim") return std::make_unique<FusedSSIMLoss>();
    throw std::runtime_error("Unknown loss type: " + type);
}

// ---------------------------------------------------------------- optimizer

struct GaussianOptimizationParams {
    float max_grad_1 = 1.0f;
    bool skip_zero_grad = false;
    float means_lr = 1.6e-4f;
    float shs_lr = 2.5e-3f;
    float opacities_lr = 5.0e-2f;
    float scales_lr = 5.0e-3f;
    float rotations_lr = 1.0e-3f;
    float opacities_l1 = 0.0f;
    float scales_l1 = 0.0f;
};

class OptimizerBase {
public:
    OptimizerBase(std::shared_ptr<GPUGaussian3d> gaussians, std::shared_ptr<GPUGaussian3d> gaussians_grad)
        : m_gaussians(std::move(gaussians)), m_gaussians_grad(std::move(gaussians_grad)) {}
    virtual ~OptimizerBase() = default;
    virtual void set_lr(float lr) = 0;
    virtual float get_lr() const = 0;
    virtual void set_params(const ParamMap& p) = 0;
    virtual ParamMap get_params() const = 0;
    // θ ← Adam(θ, scale · grad); gradients are read, not cleared.
    virtual void step(float scale, hipStream_t stream) = 0;
    virtual void reset() = 0;
    // optim.hpp:61-76: remove / duplicate default to no-ops, the rest are pure
    virtual void remove(char*, int) {}
    virtual void duplicate(int*, int*, int) {}
    virtual void reset(int* indices, int num_reset) = 0;
    virtual void reorder(uint32_t* indices) = 0;
    virtual void reset_opacity() = 0;
    virtual void set_gaussians(std::shared_ptr<GPUGaussian3d> g, std::shared_ptr<GPUGaussian3d> gg) = 0;
    std::shared_ptr<GPUGaussian3d> get_gaussians() const { return m_gaussians; }
    std::shared_ptr<GPUGaussian3d> get_gaussians_grad() const { return m_gaussians_grad; }
    virtual GaussianOptimizationParams get_optimization_params() const = 0;

protected:
    std::shared_ptr<GPUGaussian3d> m_gaussians, m_gaussians_grad;
};

class SimpleAdam final : public OptimizerBase {
public:
    SimpleAdam(std::shared_ptr<GPUGaussian3d> g, std::shared_ptr<GPUGaussian3d> gg) : OptimizerBase(g, gg) {
        const tgs_gaussians p = m_gaussians->to_c(), q = m_gaussians_grad->to_c();
        throw_on(tgs_adam_create(&p, &q, &m_handle), "create_optimizer");
    }
    ~SimpleAdam() override {
        if (m_handle) tgs_adam_destroy(m_handle);
    }
    SimpleAdam(const SimpleAdam&) = delete;
    SimpleAdam& operator=(const SimpleAdam&) = delete;

    void set_lr(float lr) override { throw_on(tgs_adam_set_lr(m_handle, lr), "SimpleAdam::set_lr"); }
    float get_lr() const override { return tgs_adam_get_lr(m_handle); }

    // Keys: beta1, beta2, epsilon, means_lr, shs_lr, opacities_lr, scales_lr,
    // rotations_lr, max_grad_1, opacities_l1, scales_l1, decay_mean (0/1).
    void set_params(const ParamMap& p) override {
        tgs_adam_params a{};
        throw_on(tgs_adam_get_params(m_handle, &a), "SimpleAdam::get_params");
        for (const auto& [k, v] : p) {
            float* f = field(a, k);
            if (f)
                *f = (float)v;
            else if (k == "decay_mean")
                a.decay_mean = v != 0.0;
            else
                throw std::runtime_error("SimpleAdam::set_params: unknown key " + k);
        }
        throw_on(tgs_adam_set_params(m_handle, &a), "SimpleAdam::set_params");
    }
    ParamMap get_params() const override {
        tgs_adam_params a{};
        throw_on(tgs_adam_get_params(m_handle, &a), "SimpleAdam::get_params");
        ParamMap m;
        for (const char* k : kKeys) m[k] = *field(a, k);
        m["decay_mean"] = a.decay_mean;
        return m;
    }
    GaussianOptimizationParams get_optimization_params() const override {
        tgs_adam_params a{};
        throw_on(tgs_adam_get_params(m_handle, &a), "SimpleAdam::get_params");
        GaussianOptimizationParams o;
        o.max_grad_1 = a.max_grad_1;
        o.means_lr = a.means_lr;
        o.shs_lr = a.shs_lr;
        o.opacities_lr = a.opacities_lr;
        o.scales_lr = a.scales_lr;
        o.rotations_lr = a.rotations_lr;
        o.opacities_l1 = a.opacities_l1;
        o.scales_l1 = a.scales_l1;
        return o;
    }

    void step(float scale, hipStream_t stream) override {
        const tgs_gaussians p = m_gaussians->to_c(), q = m_gaussians_grad->to_c();
        throw_on(tgs_adam_set_gaussians(m_handle, &p, &q), "SimpleAdam::step");
        throw_on(tgs_adam_step(m_handle, scale, stream), "SimpleAdam::step");
    }
    void reset() override { throw_on(tgs_adam_reset(m_handle, nullptr), "SimpleAdam::reset"); }
    using OptimizerBase::reset;

    // SimpleAdam::remove (simple_adam.cu:841-906). The reference maps over the
    // optimiser's Gaussians, which the strategy has already shrunk to num_kept
    // rows: moment row k = the k-th set flag among the first num_kept flags,
    // and the rows past those read row 0 (its zero-initialised map).
    void remove(char* kept_flag, int num_kept) override {
        if (num_kept <= 0) return;
        DeviceArray<int32_t> rows((size_t)num_kept);
        hip_check(hipMemset(rows.data(), 0, rows.bytes()), "hipMemset");
        int64_t count = 0;
        throw_on(tgs_flags_compact((const uint8_t*)kept_flag, num_kept, rows.data(), &count, nullptr),
                 "SimpleAdam::remove");
        throw_on(tgs_adam_gather(m_handle, rows.data(), num_kept, nullptr), "SimpleAdam::remove");
        hip_check(hipStreamSynchronize(nullptr), "hipStreamSynchronize");
    }
    // SimpleAdam::duplicate (simple_adam.cu:908-924): zero moment rows appended.
    void duplicate(int*, int*, int num_duplicate) override {
        if (num_duplicate > 0)
            throw_on(tgs_adam_append(m_handle, num_duplicate, nullptr), "SimpleAdam::duplicate");
    }
    // SimpleAdam::reset_opacity (simple_adam.cu:981-985).
    void reset_opacity() override { throw_on(tgs_adam_reset_opacity(m_handle, nullptr), "SimpleAdam::reset_opacity"); }
    // SimpleAdam::reset(int*, int) (simple_adam.cu:944-979): moments of the
    // rows indices[0 .. num_reset) (device) zeroed.
    void reset(int* indices, int num_reset) override {
        throw_on(tgs_adam_reset_rows(m_handle, indices, num_reset, nullptr), "SimpleAdam::reset");
    }
    // SimpleAdam::reorder (simple_adam.cu:1037-1097): new row i = old row indices[i].
    void reorder(uint32_t* indices) override {
        throw_on(tgs_adam_reorder(m_handle, indices, nullptr), "SimpleAdam::reorder");
    }
    // Device pointers of a group's moments (0..5 = means, opacities, rotations, scales, sh0, sh_rest).
    std::pair<float*, float*> moments(int group) const {
        float *a = nullptr, *b = nullptr;
        throw_on(tgs_adam_moments(m_handle, group, &a, &b), "SimpleAdam::moments");
        return {a, b};
    }

    void set_gaussians(std::shared_ptr<GPUGaussian3d> g, std::shared_ptr<GPUGaussian3d> gg) override {
        if (g->size() != m_gaussians->size())
            throw std::runtime_error("SimpleAdam::set_gaussians: size changes need densification support");
        m_gaussians = std::move(g);
        m_gaussians_grad = std::move(gg);
        const tgs_gaussians p = m_gaussians->to_c(), q = m_gaussians_grad->to_c();
        throw_on(tgs_adam_set_gaussians(m_handle, &p, &q), "SimpleAdam::set_gaussians");
        reset();
    }
    int64_t global_steps() const { return tgs_adam_global_steps(m_handle); }

private:
    static constexpr const char* kKeys[] = {"beta1",    "beta2",        "epsilon",   "means_lr",
                                            "shs_lr",   "opacities_lr", "scales_lr", "rotations_lr",
                                            "max_grad_1", "opacities_l1", "scales_l1"};
    static float* field(tgs_adam_params& a, const std::string& k) {
        if (k == "beta1") return &a.beta1;
        if (k == "beta2") return &a.beta2;
        if (k == "epsilon") return &a.epsilon;
        if (k == "means_lr") return &a.means_lr;
        if (k == "shs_lr") return &a.shs_lr;
        if (k == "opacities_lr") return &a.opacities_lr;
        if (k == "scales_lr") return &a.scales_lr;
        if (k == "rotations_lr") return &a.rotations_lr;
        if (k == "max_grad_1") return &a.max_grad_1;
        if (k == "opacities_l1") return &a.opacities_l1;
        if (k == "scales_l1") return &a.scales_l1;
        return nullptr;
    }
    static const float* field(const tgs_adam_params& a, const std::string& k) {
        return field(const_cast<tgs_adam_params&>(a), k);
    }
    tgs_adam* m_handle = nullptr;
};

inline std::unique_ptr<OptimizerBase> create_optimizer(const std::string& type, std::shared_ptr<GPUGaussian3d> g,
                                                       std::shared_ptr<GPUGaussian3d> gg) {
    if (type == "simple_adam") return std::make_unique<SimpleAdam>(std::move(g), std::move(gg));
    throw std::runtime_error("Unknown optimizer type: " + type);
}

// ---------------------------------------------------------------- densification strategy
// StrategyParams / StrategyBase / DefaultStrategy / create_strategy
// (tinygs/include/tinygs/strategy/strategy.hpp:7-121, tinygs/src/strategy/
// strategy.cpp:10-177, tinygs/src/strategy/default.cu:17-359): same parameter
// names, defaults, schedule, RNG (pcg32 seeded with `seed`, stream 1) and
// order of the Gaussian / gradient / optimiser updates. The device work runs
// behind tgs_densify_select / tgs_random_logistic / tgs_densify_apply /
// tgs_prune_select / tgs_gaussians_gather / tgs_reset_opacity.

struct StrategyParams {
    float pruning_opacity_threshold = 0.005f;
    float pruning_scale_threshold = 0.1f;
    float max_screen_size = 10.0f;
    float duplicate_grad_threshold = 0.0002f;
    float duplicate_scale_threshold = 0.01f;
    bool reset_reset_optimizer = false;
    bool absgrad = false;
    int refine_every = 100;
    int start_refine = 500;
    int end_refine = 15000;
    int max_num_gaussians = 10000000;
    int reset_every = 3000;
    uint64_t seed = 42;

    void from_map(const ParamMap& m) {
        auto f = [&](const char* k, auto& v) {
            auto it = m.find(k);
            if (it != m.end()) v = static_cast<std::remove_reference_t<decltype(v)>>(it->second);
        };
        f("pruning_opacity_threshold", pruning_opacity_threshold);
        f("pruning_scale_threshold", pruning_scale_threshold);
        f("max_screen_size", max_screen_size);
        f("duplicate_grad_threshold", duplicate_grad_threshold);
        f("duplicate_scale_threshold", duplicate_scale_threshold);
        f("reset_reset_optimizer", reset_reset_optimizer);
        f("absgrad", absgrad);
        f("refine_every", refine_every);
        f("start_refine", start_refine);
        f("end_refine", end_refine);
        f("max_num_gaussians", max_num_gaussians);
        f("reset_every", reset_every);
        f("seed", seed);
    }
};

class StrategyBase {
public:
    StrategyBase(std::shared_ptr<GPUGaussian3d> g, std::shared_ptr<GPUGaussian3d> gg, OptimizerBase* optimizer)
        : m_gaussians(std::move(g)), m_gaussians_grad(std::move(gg)), m_optimizer(optimizer) {}
    virtual ~StrategyBase() = default;
    void step(RasterizeContext& ctx) {
        step_impl(ctx);
        ++m_step_count;
    }
    int this_step() const { return m_step_count; }
    virtual void set_params(const ParamMap& p) { m_params.from_map(p); }
    const StrategyParams& params() const { return m_params; }

protected:
    virtual void step_impl(RasterizeContext& ctx) = 0;
    // strategy.cpp:19-31: Gaussians, gradients, then the optimiser
    void on_remove(char* kept_flag, const int32_t* kept_rows, int num_kept) {
        if (num_kept <= 0) return;
        if (m_gaussians) m_gaussians->gather_rows(kept_rows, (size_t)num_kept);
        if (m_gaussians_grad) m_gaussians_grad->gather_rows(kept_rows, (size_t)num_kept);
        if (m_optimizer) m_optimizer->remove(kept_flag, num_kept);
    }
    // strategy.cpp:33-45
    void on_duplicate(int n) {
        if (n <= 0) return;
        if (m_gaussians) m_gaussians->append(n);
        if (m_gaussians_grad) m_gaussians_grad->append(n);
        if (m_optimizer) m_optimizer->duplicate(nullptr, nullptr, n);
    }
    // strategy.cpp:55-63
    void on_reset_opacity() {
        if (!m_optimizer) return;
        m_optimizer->reset_opacity();
        if (m_params.reset_reset_optimizer) m_optimizer->reset();
    }

    std::shared_ptr<GPUGaussian3d> m_gaussians, m_gaussians_grad;
    OptimizerBase* m_optimizer;
    StrategyParams m_params;
    int m_step_count = 0;
};

class DefaultStrategy final : public StrategyBase {
public:
    using StrategyBase::StrategyBase;
    // default.cu:349-352: set_params reseeds the generator
    void set_params(const ParamMap& p) override {
        StrategyBase::set_params(p);
        tgs_pcg32_seed(&m_rng, m_params.seed, 1);
    }
    const tgs_pcg32& rng() const { return m_rng; }
    int64_t last_duplicated = 0, last_split = 0, last_kept = 0;

protected:
    // default.cu:40-69
    void step_impl(RasterizeContext& ctx) override {
        hip_check(hipStreamSynchronize(ctx.stream), "hipStreamSynchronize");
        const size_t n = m_gaussians->size();
        if (!ctx.densification_info) fresh_info(ctx, n);
        const StrategyParams& p = m_params;
        const int step = this_step();
        if (step % p.refine_every == 0 && p.start_refine <= step && step <= p.end_refine) {
            if ((int64_t)m_gaussians->size() < (int64_t)p.max_num_gaussians) duplicate(ctx);
            prune(ctx);
            fresh_info(ctx, m_gaussians->size());
        }
        if (p.reset_every > 0 && step % p.reset_every == 0 && p.start_refine <= step && step < p.end_refine) {
            const tgs_gaussians g = m_gaussians->to_c();
            throw_on(tgs_reset_opacity(&g, 2.0f * p.pruning_opacity_threshold, ctx.stream), "reset_opacity");
            on_reset_opacity();
        }
    }

private:
    static void fresh_info(RasterizeContext& ctx, size_t n) {
        ctx.densification_info = std::make_shared<GPUBuffer<DensificationInfo>>(std::max<size_t>(n, 1));
        hip_check(hipMemset(ctx.densification_info->data(), 0, ctx.densification_info->bytes()), "hipMemset");
    }
    // default.cu:71-297
    void duplicate(RasterizeContext& ctx) {
        const size_t n = m_gaussians->size();
        if (!ctx.densification_info || ctx.densification_info->size() < n) return;
        DeviceArray<uint8_t> flags(std::max<size_t>(n, 1));
        DeviceArray<int32_t> src(std::max<size_t>(n, 1));
        int64_t nd = 0, ns = 0;
        const tgs_gaussians g = m_gaussians->to_c();
        throw_on(tgs_densify_select(&g, (const float*)ctx.densification_info->data(),
                                    m_params.duplicate_grad_threshold * ctx.grad_scaler,
                                    m_params.duplicate_scale_threshold * m_gaussians->scene_scale(),
                                    m_params.absgrad ? 1 : 0, flags.data(), src.data(), &nd, &ns, ctx.stream),
                 "DefaultStrategy::duplicate");
        last_duplicated = nd;
        last_split = ns;
        const int64_t grows = nd + ns;
        if (grows == 0) return;
        on_duplicate((int)grows);
        DeviceArray<float> rnd((size_t)(6 * grows));
        throw_on(tgs_random_logistic(&m_rng, 6 * grows, rnd.data(), 0.0f, 1.0f, ctx.stream),
                 "generate_random_logistic");
        const tgs_gaussians g2 = m_gaussians->to_c();
        throw_on(tgs_densify_apply(&g2, (int64_t)n, src.data(), grows, flags.data(), rnd.data(), ctx.stream),
                 "DefaultStrategy::duplicate");
        hip_check(hipStreamSynchronize(ctx.stream), "hipStreamSynchronize");
    }
    // default.cu:300-341
    void prune(RasterizeContext& ctx) {
        const size_t n = m_gaussians->size();
        const int64_t n_info = ctx.densification_info ? (int64_t)ctx.densification_info->size() : 0;
        DeviceArray<uint8_t> alive(std::max<size_t>(n, 1));
        DeviceArray<int32_t> kept(std::max<size_t>(n, 1));
        int64_t nk = 0;
        const tgs_gaussians g = m_gaussians->to_c();
        const float limit_ss = (float)std::max(ctx.fwd_input.width, ctx.fwd_input.height) * m_params.max_screen_size;
        throw_on(tgs_prune_select(&g, (const float*)ctx.densification_info->data(), n_info,
                                  m_params.pruning_opacity_threshold,
                                  m_params.pruning_scale_threshold * m_gaussians->scene_scale(), limit_ss,
                                  this_step() > m_params.reset_every ? 1 : 0, alive.data(), kept.data(), &nk,
                                  ctx.stream),
                 "DefaultStrategy::prune");
        last_kept = nk;
        on_remove((char*)alive.data(), kept.data(), (int)nk);
    }

    tgs_pcg32 m_rng{0x853C49E6748FEA9Bull, 0xDA3E39CB94B95BDBull};   // pcg32's default state
};

inline std::unique_ptr<StrategyBase> create_strategy(const std::string& type, std::shared_ptr<GPUGaussian3d> g,
                                                     std::shared_ptr<GPUGaussian3d> gg, OptimizerBase* optimizer) {
    if (type == "default") return std::make_unique<DefaultStrategy>(std::move(g), std::move(gg), optimizer);
    if (type == "mcmc" || type == "improved")
        throw std::runtime_error("Strategy '" + type + "' is not built (only 'default')");
    throw std::runtime_error("Unknown strategy type: " + type);
}

// ---------------------------------------------------------------- metrics and files

// PsnrMetric::evaluate (tinygs/src/loss/psnr.cu:72-128).
class PsnrMetric {
public:
    float evaluate(const Image& pred, const Image& target, hipStream_t stream = nullptr) const {
        if (pred.shape.width != target.shape.width || pred.shape.height != target.shape.height ||
            pred.shape.channel != target.shape.channel)
            throw std::runtime_error("Prediction and target shapes must match");
        if (pred.data_type != target.data_type)
            throw std::runtime_error("PSNR: prediction and target data type must be the same");
        tgs_loss_context c{pred.data, target.data, nullptr, nullptr, pred.shape.width, pred.shape.height,
                           pred.shape.channel, c_dtype(pred.data_type)};
        float v = 0.0f;
        throw_on(tgs_psnr(&c, &v, stream), "PsnrMetric::evaluate");
        return v;
    }
};

// tinygs/include/tinygs/core/pointcloud.hpp:11-26
struct PointCloud {
    std::vector<float> points, colors;   // 3 floats per point each; colours in [0, 1]
    size_t size() const { return points.size() / 3; }
};
inline PointCloud load_point_cloud(const std::string& filename) {
    int64_t n = 0;
    throw_on(tgs_point_cloud_load(filename.c_str(), &n, nullptr, nullptr), "load_point_cloud");
    PointCloud pc;
    pc.points.resize(3 * (size_t)n);
    pc.colors.resize(3 * (size_t)n);
    if (n) throw_on(tgs_point_cloud_load(filename.c_str(), &n, pc.points.data(), pc.colors.data()), "load_point_cloud");
    return pc;
}
// save_ply (pointcloud.cpp:111-240) from the device arrays: byte for byte the reference's file.
inline void save_ply(const std::string& filename, const GPUGaussian3d& gs, bool full_features = false,
                     hipStream_t stream = nullptr) {
    const tgs_gaussians g = gs.to_c();
    throw_on(tgs_ply_save(filename.c_str(), &g, full_features ? 1 : 0, stream), "save_ply");
}
// The Gaussians of a full-feature PLY (the inverse of save_ply; no counterpart in the reference).
inline std::shared_ptr<GPUGaussian3d> load_gaussians_ply(const std::string& filename,
                                                         DataType sh_dtype = DataType::Float32) {
    tgs_ply_info info{};
    throw_on(tgs_ply_read_info(filename.c_str(), &info), "load_gaussians_ply");
    auto g = std::make_shared<GPUGaussian3d>((size_t)info.n_vertices, sh_dtype);
    const tgs_gaussians c = g->to_c();
    throw_on(tgs_ply_load_gaussians(filename.c_str(), &c, nullptr), "load_gaussians_ply");
    return g;
}

}  // namespace tinygs_amd
