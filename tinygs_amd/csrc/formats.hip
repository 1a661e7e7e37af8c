// On-disk and interchange formats: PLY files of Gaussians and point clouds,
// and the image layout converters.
//
// PLY. save_ply (tinygs/src/core/pointcloud.cpp:111-240) writes one binary
// little-endian "vertex" element through hapPLY (tinygs/src/core/happly.h:
// header text :1973-2010, element header :1084-1091, rows :1120-1126), which
// stores the element row by row, each row holding the properties in the
// order they were added:
//   x y z (float), red green blue (uchar: clamp(f_dc * C0 + 0.5, 0, 1) * 255
//   truncated), and with full features f_dc_r/g/b, f_rest_{r,g,b}_k for
//   k = 0..14 (so the 45 floats of a row are the sh_rest row in memory order),
//   opacity, scale_0..2, rot_w rot_x rot_y rot_z (float).
// Rows are 15 bytes (positions and colours) or 239 bytes. Here they are
// packed on the device straight from the SoA parameter arrays, one thread per
// 32-bit output word, so the host only copies finished bytes into the file.
//
// Reading accepts any vertex property order and scalar type, ascii or binary
// of either byte order, and two name sets for the Gaussian properties: the
// reference's (f_dc_r, f_rest_r_k, rot_w) and the common 3DGS one (f_dc_0,
// f_rest_i with i = channel * 15 + k, rot_0). The vertex rows are normalised
// to little-endian binary on the host and unpacked on the device.
// load_point_cloud (pointcloud.cpp:19-109): positions and uchar colours / 255
// from a PLY, or columns 1-6 of COLMAP's points3D.txt.
//
// Images. from_cv2 / to_cv2 (tinygs/src/utils/image_format.cu:68-114) move
// between interleaved HWC u8 (BGR for OpenCV) and the channel-planar 8x8-tiled
// layout; the data loader then widens u8 to float or half as (1 / 255) * v
// (tinygs/src/dataloader/dataloader.cu:18-95), and the image export narrows
// float to u8 as the truncation of clamp(255 v, 0, 255)
// (tinygs/src/orchestrator.cu:896-937). Here one kernel changes the layout
// and the type together: a workgroup stages an 8-row x 256-column strip in
// LDS, so the row reads and the tile writes are both contiguous runs.
#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <algorithm>
#include <cstdint>
#include <fstream>
#include <new>
#include <sstream>
#include <string>
#include <vector>

#include "common.h"
#include "status.h"

namespace tgs {
namespace {

// ---------------------------------------------------------------- PLY rows

constexpr uint32_t kPlyPartialRow = 15;
constexpr uint32_t kPlyFullRow = 239;
constexpr int kPlySlots = 59;   // means 3, opacity 1, scales 3, rotations 4, sh0 3, sh_rest 45

struct PlySrc {
    const float* means;
    const float* scales;
    const float* rotations;
    const float* opacities;
    const void* sh0;
    const void* sh_rest;
};

// Field of byte o of a row and the byte's index inside the field's value.
// Fields: 0-2 x y z, 3-5 red green blue, 6-8 f_dc, 9-53 f_rest, 54 opacity,
// 55-57 scale, 58-61 rot.
__device__ __forceinline__ void ply_field_of(uint32_t o, uint32_t& f, uint32_t& byte) {
    if (o < 12u) {
        f = o >> 2;
        byte = o & 3u;
    } else if (o < 15u) {
        f = o - 9u;
        byte = 0u;
    } else {
        f = 6u + ((o - 15u) >> 2);
        byte = (o - 15u) & 3u;
    }
}

// save_ply's colour byte: (unsigned char)(clamp(v * C0 + 0.5, 0, 1) * 255)
// with clamp(a, lo, hi) = a < lo ? lo : (hi < a ? hi : a) (tinygs/include/
// tinygs/cuda/vec.hpp:68); separate roundings (no contraction).
__device__ __forceinline__ uint32_t ply_colour(float v) {
    float t = v * 0.28209479177387814f;
    t = t + 0.5f;
    t = t < 0.f ? 0.f : (1.f < t ? 1.f : t);
    return (uint32_t)(t * 255.0f) & 0xffu;
}

template <typename ShT>
__device__ __forceinline__ uint32_t ply_field_bits(const PlySrc& g, int64_t r, uint32_t f) {
    const ShT* sh0 = (const ShT*)g.sh0;
    const ShT* shr = (const ShT*)g.sh_rest;
    if (f < 3u) return __float_as_uint(g.means[3 * r + f]);
    if (f < 6u) return ply_colour(load_as_float(sh0, 3 * r + (f - 3u)));
    if (f < 9u) return __float_as_uint(load_as_float(sh0, 3 * r + (f - 6u)));
    if (f < 54u) return __float_as_uint(load_as_float(shr, 45 * r + (f - 9u)));
    if (f == 54u) return __float_as_uint(g.opacities[r]);
    if (f < 58u) return __float_as_uint(g.scales[3 * r + (f - 55u)]);
    return __float_as_uint(g.rotations[4 * r + (f - 58u)]);
}

// One thread per 32-bit word of the n x row_bytes vertex block; bytes past
// the block (the last word's tail) are zero.
template <typename ShT>
__global__ void __launch_bounds__(256) ply_pack_kernel(PlySrc g, int64_t n, uint32_t row_bytes,
                                                       uint32_t* __restrict__ out, int64_t n_words) {
    const int64_t w = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (w >= n_words) return;
    const uint64_t total = (uint64_t)n * row_bytes;
    uint64_t b = 4ull * (uint64_t)w;
    int64_t r = (int64_t)(b / row_bytes);
    uint32_t o = (uint32_t)(b - (uint64_t)r * row_bytes);
    uint32_t word = 0u, cached = ~0u, bits = 0u;
    for (int q = 0; q < 4; ++q, ++b) {
        if (b >= total) break;
        uint32_t f, byte;
        ply_field_of(o, f, byte);
        if (f != cached) {
            bits = ply_field_bits<ShT>(g, r, f);
            cached = f;
        }
        word |= ((bits >> (8u * byte)) & 0xffu) << (8u * (uint32_t)q);
        if (++o == row_bytes) {
            o = 0u;
            ++r;
            cached = ~0u;
        }
    }
    out[w] = word;
}

enum PlyType { PT_CHAR = 0, PT_UCHAR, PT_SHORT, PT_USHORT, PT_INT, PT_UINT, PT_FLOAT, PT_DOUBLE };

int ply_type_size(int t) {
    static const int kSize[8] = {1, 1, 2, 2, 4, 4, 4, 8};
    return t >= 0 && t < 8 ? kSize[t] : 0;
}

struct PlyCol {
    uint32_t off;   // byte offset in the row
    int32_t type;   // PlyType
};

__device__ __forceinline__ float ply_read(const uint8_t* p, int type) {
    switch (type) {
        case PT_CHAR: return (float)(int8_t)p[0];
        case PT_UCHAR: return (float)p[0];
        case PT_SHORT: { int16_t v; __builtin_memcpy(&v, p, 2); return (float)v; }
        case PT_USHORT: { uint16_t v; __builtin_memcpy(&v, p, 2); return (float)v; }
        case PT_INT: { int32_t v; __builtin_memcpy(&v, p, 4); return (float)v; }
        case PT_UINT: { uint32_t v; __builtin_memcpy(&v, p, 4); return (float)v; }
        case PT_DOUBLE: { double v; __builtin_memcpy(&v, p, 8); return (float)v; }
        default: { float v; __builtin_memcpy(&v, p, 4); return v; }
    }
}

template <typename ShT>
__device__ __forceinline__ ShT sh_store(float v);
template <>
__device__ __forceinline__ float sh_store<float>(float v) { return v; }
template <>
__device__ __forceinline__ __half sh_store<__half>(float v) { return f2h_rn(v); }

struct PlyDst {
    float* means;
    float* scales;
    float* rotations;
    float* opacities;
    void* sh0;
    void* sh_rest;
};

// blockIdx.y selects the destination array (0 means, 1 opacities, 2 scales,
// 3 rotations, 4 sh0, 5 sh_rest); one thread per destination element, so
// the stores are contiguous. cols holds the 59 slots in that array order.
template <typename ShT>
__global__ void __launch_bounds__(256) ply_unpack_kernel(const uint8_t* __restrict__ rows, uint32_t stride,
                                                         int64_t n, const PlyCol* __restrict__ cols, PlyDst g) {
    const int a = (int)blockIdx.y;
    const uint32_t width = a == 0 ? 3u : a == 1 ? 1u : a == 2 ? 3u : a == 3 ? 4u : a == 4 ? 3u : 45u;
    const uint32_t slot0 = a == 0 ? 0u : a == 1 ? 3u : a == 2 ? 4u : a == 3 ? 7u : a == 4 ? 11u : 14u;
    const int64_t e = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (e >= n * (int64_t)width) return;
    const int64_t r = e / width;
    const uint32_t c = (uint32_t)(e - r * width);
    const PlyCol col = cols[slot0 + c];
    const float v = ply_read(rows + (size_t)r * stride + col.off, col.type);
    switch (a) {
        case 0: g.means[e] = v; break;
        case 1: g.opacities[e] = v; break;
        case 2: g.scales[e] = v; break;
        case 3: g.rotations[e] = v; break;
        case 4: ((ShT*)g.sh0)[e] = sh_store<ShT>(v); break;
        default: ((ShT*)g.sh_rest)[e] = sh_store<ShT>(v); break;
    }
}

// ---------------------------------------------------------------- images

constexpr int kStripTiles = 32;                 // tiles per workgroup strip
constexpr int kStripCols = kStripTiles * 8;     // 256 columns
constexpr float kCharToFloat = 1.0f / 255.0f;   // dataloader.cu:18

enum ImgType { IT_F32 = TGS_DTYPE_FLOAT32, IT_F16 = TGS_DTYPE_FLOAT16, IT_U8 = 2 };

__device__ __forceinline__ float u8_widen(uint32_t v) { return kCharToFloat * (float)v; }
// orchestrator.cu:932-934: static_cast<uint8_t>(clamp(255 v, 0, 255)); NaN gives 0
__device__ __forceinline__ uint32_t u8_narrow(float v) {
    return (uint32_t)__builtin_fminf(__builtin_fmaxf(v * 255.0f, 0.0f), 255.0f);
}

template <int T>
__device__ __forceinline__ void img_store(void* dst, size_t i, uint32_t v) {
    if constexpr (T == IT_F32) ((float*)dst)[i] = u8_widen(v);
    else if constexpr (T == IT_F16) ((__half*)dst)[i] = f2h_rn(u8_widen(v));
    else ((uint8_t*)dst)[i] = (uint8_t)v;
}
template <int T>
__device__ __forceinline__ uint32_t img_load(const void* src, size_t i) {
    if constexpr (T == IT_F32) return u8_narrow(((const float*)src)[i]);
    else if constexpr (T == IT_F16) return u8_narrow(__half2float(((const __half*)src)[i]));
    else return ((const uint8_t*)src)[i];
}

// HWC u8 (channel order reversed when bgr) -> tiled planar of type T; the
// padding is written as zero. Grid (ceil(tiled_w / 32), tiled_h).
template <int T>
__global__ void __launch_bounds__(256) hwc_to_tiled_kernel(const uint8_t* __restrict__ src, uint32_t W, uint32_t H,
                                                           uint32_t C, int bgr, void* __restrict__ dst,
                                                           uint32_t tiled_w, uint32_t channel_stride) {
    __shared__ uint8_t s[8][kStripCols * 4];
    const uint32_t t = threadIdx.x;
    const uint32_t tx0 = blockIdx.x * kStripTiles, y0 = blockIdx.y * 8u, x0 = tx0 * 8u;
    const uint32_t cols = x0 < W ? min((uint32_t)kStripCols, W - x0) : 0u;
    const uint32_t len = cols * C;
    for (uint32_t yy = 0; yy < 8u; ++yy) {
        const uint32_t y = y0 + yy;
        if (y >= H) break;
        const uint8_t* row = src + ((size_t)y * W + x0) * C;
        for (uint32_t i = t; i < len; i += 256u) s[yy][i] = row[i];
    }
    __syncthreads();
    const uint32_t tiles = min((uint32_t)kStripTiles, tiled_w - tx0);
    const size_t base = ((size_t)blockIdx.y * tiled_w + tx0) * 64u;
    for (uint32_t c = 0; c < C; ++c) {
        const uint32_t sc = bgr ? C - 1u - c : c;
        for (uint32_t e = t; e < tiles * 64u; e += 256u) {
            const uint32_t within = e & 63u, row = within >> 3, col = (e >> 6) * 8u + (within & 7u);
            const uint32_t v = (y0 + row < H && col < cols) ? (uint32_t)s[row][col * C + sc] : 0u;
            img_store<T>(dst, (size_t)c * channel_stride + base + e, v);
        }
    }
}

// tiled planar of type T -> HWC u8 (channel order reversed when bgr).
template <int T>
__global__ void __launch_bounds__(256) tiled_to_hwc_kernel(const void* __restrict__ src, uint32_t W, uint32_t H,
                                                           uint32_t C, int bgr, uint8_t* __restrict__ dst,
                                                           uint32_t tiled_w, uint32_t channel_stride) {
    __shared__ uint8_t s[8][kStripCols * 4];
    const uint32_t t = threadIdx.x;
    const uint32_t tx0 = blockIdx.x * kStripTiles, y0 = blockIdx.y * 8u, x0 = tx0 * 8u;
    const uint32_t cols = x0 < W ? min((uint32_t)kStripCols, W - x0) : 0u;
    const uint32_t tiles = min((uint32_t)kStripTiles, tiled_w - tx0);
    const size_t base = ((size_t)blockIdx.y * tiled_w + tx0) * 64u;
    for (uint32_t c = 0; c < C; ++c) {
        const uint32_t dc = bgr ? C - 1u - c : c;
        for (uint32_t e = t; e < tiles * 64u; e += 256u) {
            const uint32_t within = e & 63u, row = within >> 3, col = (e >> 6) * 8u + (within & 7u);
            if (y0 + row < H && col < cols) s[row][col * C + dc] = (uint8_t)img_load<T>(src, (size_t)c * channel_stride + base + e);
        }
    }
    __syncthreads();
    const uint32_t len = cols * C;
    for (uint32_t yy = 0; yy < 8u; ++yy) {
        const uint32_t y = y0 + yy;
        if (y >= H) break;
        uint8_t* row = dst + ((size_t)y * W + x0) * C;
        for (uint32_t i = t; i < len; i += 256u) row[i] = s[yy][i];
    }
}

// Elementwise type conversion (half_to_float_gpu / float_to_half_gpu,
// image_format.cu:117-139; convert_u8_float / convert_u8_half,
// dataloader.cu:26-95).
template <int S, int D>
__global__ void __launch_bounds__(256) convert_kernel(const void* __restrict__ src, void* __restrict__ dst, int64_t n) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= n) return;
    if constexpr (S == IT_U8) {
        img_store<D>(dst, (size_t)i, ((const uint8_t*)src)[i]);
    } else if constexpr (D == IT_U8) {
        ((uint8_t*)dst)[i] = (uint8_t)img_load<S>(src, (size_t)i);
    } else {
        const float v = S == IT_F32 ? ((const float*)src)[i] : __half2float(((const __half*)src)[i]);
        if constexpr (D == IT_F32) ((float*)dst)[i] = v;
        else ((__half*)dst)[i] = f2h_rn(v);
    }
}

// ---------------------------------------------------------------- PLY header (host)

bool ply_parse_type(const std::string& s, int& t) {
    static const char* const kNames[8][2] = {{"char", "int8"},   {"uchar", "uint8"},  {"short", "int16"},
                                             {"ushort", "uint16"}, {"int", "int32"},   {"uint", "uint32"},
                                             {"float", "float32"}, {"double", "float64"}};
    for (int k = 0; k < 8; ++k)
        if (s == kNames[k][0] || s == kNames[k][1]) {
            t = k;
            return true;
        }
    return false;
}

struct PlyProp {
    std::string name;
    int type = PT_FLOAT;
    bool is_list = false;
    int count_type = PT_UCHAR;
};
struct PlyElem {
    std::string name;
    int64_t count = 0;
    std::vector<PlyProp> props;
};
struct PlyHeader {
    int format = 1;   // 0 ascii, 1 binary little endian, 2 binary big endian
    std::vector<PlyElem> elems;
    std::streamoff data_start = 0;
};

int ply_read_header(std::ifstream& in, const char* filename, PlyHeader& h) {
    std::string line;
    auto next = [&](std::string& l) -> bool {
        if (!std::getline(in, l)) return false;
        if (!l.empty() && l.back() == '\r') l.pop_back();
        return true;
    };
    if (!next(line) || line != "ply") return fail(TGS_ERR_INVALID, "%s: not a PLY file", filename);
    bool have_format = false;
    while (true) {
        if (!next(line)) return fail(TGS_ERR_INVALID, "%s: PLY header has no end_header", filename);
        std::istringstream ls(line);
        std::string key;
        ls >> key;
        if (key.empty() || key == "comment" || key == "obj_info") continue;
        if (key == "end_header") break;
        if (key == "format") {
            std::string f, v;
            ls >> f >> v;
            if (f == "ascii") h.format = 0;
            else if (f == "binary_little_endian") h.format = 1;
            else if (f == "binary_big_endian") h.format = 2;
            else return fail(TGS_ERR_INVALID, "%s: unknown PLY format '%s'", filename, f.c_str());
            have_format = true;
        } else if (key == "element") {
            PlyElem e;
            long long cnt = -1;
            ls >> e.name >> cnt;
            if (e.name.empty() || cnt < 0) return fail(TGS_ERR_INVALID, "%s: bad PLY element line '%s'", filename, line.c_str());
            e.count = cnt;
            h.elems.push_back(e);
        } else if (key == "property") {
            if (h.elems.empty()) return fail(TGS_ERR_INVALID, "%s: PLY property before any element", filename);
            PlyProp p;
            std::string t;
            ls >> t;
            if (t == "list") {
                std::string ct, it;
                ls >> ct >> it >> p.name;
                p.is_list = true;
                if (!ply_parse_type(ct, p.count_type) || !ply_parse_type(it, p.type))
                    return fail(TGS_ERR_INVALID, "%s: bad PLY list property '%s'", filename, line.c_str());
            } else {
                ls >> p.name;
                if (!ply_parse_type(t, p.type)) return fail(TGS_ERR_INVALID, "%s: unknown PLY type '%s'", filename, t.c_str());
            }
            if (p.name.empty()) return fail(TGS_ERR_INVALID, "%s: bad PLY property line '%s'", filename, line.c_str());
            h.elems.back().props.push_back(p);
        } else {
            return fail(TGS_ERR_INVALID, "%s: unknown PLY header line '%s'", filename, line.c_str());
        }
    }
    if (!have_format) return fail(TGS_ERR_INVALID, "%s: PLY header has no format line", filename);
    h.data_start = in.tellg();
    return TGS_OK;
}

void ply_swap(uint8_t* p, int size) { std::reverse(p, p + size); }

// Writes the ascii token as a little-endian value of type t.
bool ply_put_ascii(const std::string& tok, int t, uint8_t* out) {
    char* end = nullptr;
    if (t == PT_FLOAT || t == PT_DOUBLE) {
        const double d = strtod(tok.c_str(), &end);
        if (end == tok.c_str()) return false;
        if (t == PT_FLOAT) {
            const float f = (float)d;
            memcpy(out, &f, 4);
        } else {
            memcpy(out, &d, 8);
        }
        return true;
    }
    const long long v = strtoll(tok.c_str(), &end, 10);
    if (end == tok.c_str()) return false;
    switch (t) {
        case PT_CHAR: { int8_t x = (int8_t)v; memcpy(out, &x, 1); break; }
        case PT_UCHAR: { uint8_t x = (uint8_t)v; memcpy(out, &x, 1); break; }
        case PT_SHORT: { int16_t x = (int16_t)v; memcpy(out, &x, 2); break; }
        case PT_USHORT: { uint16_t x = (uint16_t)v; memcpy(out, &x, 2); break; }
        case PT_INT: { int32_t x = (int32_t)v; memcpy(out, &x, 4); break; }
        default: { uint32_t x = (uint32_t)v; memcpy(out, &x, 4); break; }
    }
    return true;
}

int64_t ply_read_count(const uint8_t* p, int t, bool swap) {
    uint8_t b[8] = {};
    const int s = ply_type_size(t);
    memcpy(b, p, s);
    if (swap) ply_swap(b, s);
    switch (t) {
        case PT_CHAR: return (int8_t)b[0];
        case PT_UCHAR: return b[0];
        case PT_SHORT: { int16_t v; memcpy(&v, b, 2); return v; }
        case PT_USHORT: { uint16_t v; memcpy(&v, b, 2); return v; }
        case PT_INT: { int32_t v; memcpy(&v, b, 4); return v; }
        case PT_UINT: { uint32_t v; memcpy(&v, b, 4); return v; }
        default: return -1;
    }
}

// The vertex element of a PLY file as little-endian binary rows. offsets[k]
// is the byte offset of property k of the vertex element in a row.
struct PlyVertices {
    const PlyElem* elem = nullptr;
    std::vector<uint32_t> offsets;
    uint32_t stride = 0;
    std::vector<uint8_t> rows;
};

int ply_read_vertices(const char* filename, PlyHeader& h, PlyVertices& v, bool load_rows) {
    std::ifstream in(filename, std::ios::binary);
    if (!in) return fail(TGS_ERR_INVALID, "could not open %s", filename);
    TGS_TRY(ply_read_header(in, filename, h));
    size_t vi = h.elems.size();
    for (size_t k = 0; k < h.elems.size(); ++k)
        if (h.elems[k].name == "vertex") {
            vi = k;
            break;
        }
    if (vi == h.elems.size()) return fail(TGS_ERR_INVALID, "%s: PLY file has no vertex element", filename);
    v.elem = &h.elems[vi];
    v.offsets.clear();
    v.stride = 0;
    for (const PlyProp& p : v.elem->props) {
        if (p.is_list) return fail(TGS_ERR_UNSUPPORTED, "%s: list property '%s' in the vertex element", filename, p.name.c_str());
        v.offsets.push_back(v.stride);
        v.stride += (uint32_t)ply_type_size(p.type);
    }
    const int64_t n = v.elem->count;
    // counts come from the header: bound each by the bytes the file still
    // holds before allocating or stepping over anything (an ascii value takes
    // at least one character and one separator)
    in.seekg(0, std::ios::end);
    const int64_t file_end = (int64_t)in.tellg();
    in.seekg(h.data_start);
    if (file_end < 0 || !in) return fail(TGS_ERR_INVALID, "could not read %s", filename);
    auto left = [&]() -> int64_t { return file_end - (int64_t)in.tellg(); };
    if (n > 0 && v.stride == 0)
        return fail(TGS_ERR_INVALID, "%s: PLY vertex element has no properties", filename);
    const bool ascii = h.format == 0;
    if (n > 0 && n > (ascii ? ((left() + 1) / 2) / (int64_t)v.elem->props.size() : left() / (int64_t)v.stride))
        return fail(TGS_ERR_INVALID, "%s: PLY file truncated (%lld vertices declared)", filename, (long long)n);
    if (!load_rows) return TGS_OK;
    const bool swap = h.format == 2;
    if (ascii) {
        try {
            v.rows.assign((size_t)n * v.stride, 0);
        } catch (const std::bad_alloc&) {
            return fail(TGS_ERR_INVALID, "%s: no host memory for %lld PLY vertices", filename, (long long)n);
        }
        // ascii: whitespace-separated tokens, elements in header order
        auto token = [&](std::string& tok) -> bool { return (bool)(in >> tok); };
        std::string tok;
        for (size_t k = 0; k < vi; ++k)
            for (int64_t i = 0; i < h.elems[k].count && !h.elems[k].props.empty(); ++i)
                for (const PlyProp& p : h.elems[k].props) {
                    if (!token(tok)) return fail(TGS_ERR_INVALID, "%s: PLY file truncated", filename);
                    if (p.is_list) {
                        const long long c = strtoll(tok.c_str(), nullptr, 10);
                        for (long long j = 0; j < c; ++j)
                            if (!token(tok)) return fail(TGS_ERR_INVALID, "%s: PLY file truncated", filename);
                    }
                }
        for (int64_t i = 0; i < n; ++i) {
            uint8_t* row = v.rows.data() + (size_t)i * v.stride;
            for (size_t k = 0; k < v.elem->props.size(); ++k) {
                if (!token(tok)) return fail(TGS_ERR_INVALID, "%s: PLY file truncated", filename);
                if (!ply_put_ascii(tok, v.elem->props[k].type, row + v.offsets[k]))
                    return fail(TGS_ERR_INVALID, "%s: bad PLY value '%s'", filename, tok.c_str());
            }
        }
        return TGS_OK;
    }
    // binary: step over the elements before the vertex element (fixed-size
    // rows in one seek; rows with lists one by one, each read ends at EOF)
    for (size_t k = 0; k < vi; ++k) {
        bool has_list = false;
        int64_t row_bytes = 0;
        for (const PlyProp& p : h.elems[k].props) {
            has_list = has_list || p.is_list;
            row_bytes += ply_type_size(p.type);
        }
        if (!has_list) {
            if (row_bytes > 0 && h.elems[k].count > left() / row_bytes)
                return fail(TGS_ERR_INVALID, "%s: PLY file truncated", filename);
            in.seekg((std::streamoff)(h.elems[k].count * row_bytes), std::ios::cur);
            continue;
        }
        for (int64_t i = 0; i < h.elems[k].count; ++i)
            for (const PlyProp& p : h.elems[k].props) {
                if (p.is_list) {
                    uint8_t b[8];
                    const int cs = ply_type_size(p.count_type);
                    if (!in.read((char*)b, cs)) return fail(TGS_ERR_INVALID, "%s: PLY file truncated", filename);
                    const int64_t c = ply_read_count(b, p.count_type, swap);
                    if (c < 0) return fail(TGS_ERR_INVALID, "%s: bad PLY list count", filename);
                    in.seekg((std::streamoff)(c * ply_type_size(p.type)), std::ios::cur);
                } else {
                    in.seekg(ply_type_size(p.type), std::ios::cur);
                }
            }
    }
    if (!in || (n > 0 && n > left() / (int64_t)v.stride))
        return fail(TGS_ERR_INVALID, "%s: PLY file truncated (%lld vertices of %u bytes expected)", filename,
                    (long long)n, v.stride);
    try {
        v.rows.assign((size_t)n * v.stride, 0);
    } catch (const std::bad_alloc&) {
        return fail(TGS_ERR_INVALID, "%s: no host memory for %lld PLY vertices", filename, (long long)n);
    }
    if (n > 0 && !in.read((char*)v.rows.data(), (std::streamsize)v.rows.size()))
        return fail(TGS_ERR_INVALID, "%s: PLY file truncated (%lld vertices of %u bytes expected)", filename,
                    (long long)n, v.stride);
    if (swap)
        for (int64_t i = 0; i < n; ++i)
            for (size_t k = 0; k < v.elem->props.size(); ++k)
                ply_swap(v.rows.data() + (size_t)i * v.stride + v.offsets[k], ply_type_size(v.elem->props[k].type));
    return TGS_OK;
}

int ply_find(const PlyElem& e, const std::string& name) {
    for (size_t k = 0; k < e.props.size(); ++k)
        if (e.props[k].name == name) return (int)k;
    return -1;
}

// Property index of every Gaussian slot (means, opacity, scales, rotations,
// sh0, sh_rest order), from the reference's names or else the common 3DGS
// names; false if some slot has neither.
bool ply_gaussian_slots(const PlyElem& e, int idx[kPlySlots], std::string& missing) {
    const char* rgb = "rgb";
    auto ref_name = [&](int s) -> std::string {
        if (s < 3) return std::string(1, "xyz"[s]);
        if (s == 3) return "opacity";
        if (s < 7) return "scale_" + std::to_string(s - 4);
        if (s < 11) return std::string("rot_") + "wxyz"[s - 7];
        if (s < 14) return std::string("f_dc_") + rgb[s - 11];
        const int j = s - 14;   // sh_rest row element j = 3 k + c
        return std::string("f_rest_") + rgb[j % 3] + "_" + std::to_string(j / 3);
    };
    auto std_name = [&](int s) -> std::string {
        if (s < 7) return ref_name(s);
        if (s < 11) return "rot_" + std::to_string(s - 7);
        if (s < 14) return "f_dc_" + std::to_string(s - 11);
        const int j = s - 14;
        return "f_rest_" + std::to_string((j % 3) * 15 + j / 3);
    };
    for (int s = 0; s < kPlySlots; ++s) {
        int k = ply_find(e, ref_name(s));
        if (k < 0) k = ply_find(e, std_name(s));
        if (k < 0) {
            missing = ref_name(s);
            return false;
        }
        idx[s] = k;
    }
    return true;
}

double ply_host_value(const uint8_t* p, int t) {
    switch (t) {
        case PT_CHAR: return (int8_t)p[0];
        case PT_UCHAR: return p[0];
        case PT_SHORT: { int16_t v; memcpy(&v, p, 2); return v; }
        case PT_USHORT: { uint16_t v; memcpy(&v, p, 2); return v; }
        case PT_INT: { int32_t v; memcpy(&v, p, 4); return v; }
        case PT_UINT: { uint32_t v; memcpy(&v, p, 4); return v; }
        case PT_FLOAT: { float v; memcpy(&v, p, 4); return v; }
        default: { double v; memcpy(&v, p, 8); return v; }
    }
}

struct DeviceScratch {
    void* p = nullptr;
    ~DeviceScratch() {
        if (p) (void)hipFree(p);
    }
};
struct PinnedScratch {
    void* p = nullptr;
    ~PinnedScratch() {
        if (p) (void)hipHostFree(p);
    }
};

int check_ply_gaussians(const tgs_gaussians* g) {
    if (!g) return fail(TGS_ERR_INVALID, "gaussians is NULL");
    if (g->n < 0 || g->n > (int64_t)0xffffffffll) return fail(TGS_ERR_INVALID, "invalid gaussian count %lld", (long long)g->n);
    if (g->n > 0 && (!g->means || !g->scales || !g->rotations || !g->opacities || !g->sh0 || !g->sh_rest))
        return fail(TGS_ERR_INVALID, "a gaussian SoA pointer is NULL");
    if (g->sh_dtype != TGS_DTYPE_FLOAT32 && g->sh_dtype != TGS_DTYPE_FLOAT16)
        return fail(TGS_ERR_INVALID, "sh_dtype %d", g->sh_dtype);
    return TGS_OK;
}

bool img_dtype_ok(int32_t t) { return t == IT_F32 || t == IT_F16 || t == IT_U8; }

int check_image_args(const void* src, const void* dst, uint32_t W, uint32_t H, uint32_t C, int32_t bgr) {
    if (!src || !dst) return fail(TGS_ERR_INVALID, "image pointer is NULL");
    if (W == 0 || H == 0 || W > 65535u * 8u || H > 65535u * 8u) return fail(TGS_ERR_INVALID, "image size %ux%u", W, H);
    if (C < 1 || C > 4) return fail(TGS_ERR_INVALID, "channels %u (1 to 4 supported)", C);
    if (bgr && C != 3) return fail(TGS_ERR_INVALID, "BGR order expects 3 channels (RGB), got %u", C);
    return TGS_OK;
}

}  // namespace
}  // namespace tgs

using namespace tgs;

extern "C" {

int tgs_ply_save(const char* filename, const tgs_gaussians* g, int32_t full_features, void* stream) {
    if (!filename) return fail(TGS_ERR_INVALID, "filename is NULL");
    TGS_TRY(check_ply_gaussians(g));
    hipStream_t s = (hipStream_t)stream;
    const int64_t n = g->n;
    const uint32_t row = full_features ? kPlyFullRow : kPlyPartialRow;
    const uint64_t bytes = (uint64_t)n * row;
    const int64_t words = (int64_t)((bytes + 3) / 4);
    DeviceScratch dev;
    PinnedScratch host;
    if (words > 0) {
        TGS_HIP(hipMalloc(&dev.p, 4 * (size_t)words));
        TGS_HIP(hipHostMalloc(&host.p, 4 * (size_t)words, hipHostMallocDefault));
        const PlySrc src{(const float*)g->means, (const float*)g->scales, (const float*)g->rotations,
                         (const float*)g->opacities, g->sh0, g->sh_rest};
        const unsigned blocks = (unsigned)((words + 255) / 256);
        if (g->sh_dtype == TGS_DTYPE_FLOAT16)
            ply_pack_kernel<__half><<<blocks, 256, 0, s>>>(src, n, row, (uint32_t*)dev.p, words);
        else
            ply_pack_kernel<float><<<blocks, 256, 0, s>>>(src, n, row, (uint32_t*)dev.p, words);
        TGS_CHECK_LAUNCH();
        TGS_HIP(hipMemcpyAsync(host.p, dev.p, 4 * (size_t)words, hipMemcpyDeviceToHost, s));
        TGS_HIP(hipStreamSynchronize(s));
    }
    // hapPLY's header (happly.h:1973-2010): magic, format, its comment, the element and its properties
    std::string hdr = "ply\nformat binary_little_endian 1.0\ncomment Written with hapPLY (https://github.com/nmwsharp/happly)\n";
    hdr += "element vertex " + std::to_string(n) + "\n";
    static const char* const kHead[6] = {"float x", "float y", "float z", "uchar red", "uchar green", "uchar blue"};
    for (const char* p : kHead) hdr += std::string("property ") + p + "\n";
    if (full_features) {
        hdr += "property float f_dc_r\nproperty float f_dc_g\nproperty float f_dc_b\n";
        for (int k = 0; k < 15; ++k)
            for (const char* c : {"r", "g", "b"}) hdr += std::string("property float f_rest_") + c + "_" + std::to_string(k) + "\n";
        hdr += "property float opacity\nproperty float scale_0\nproperty float scale_1\nproperty float scale_2\n";
        hdr += "property float rot_w\nproperty float rot_x\nproperty float rot_y\nproperty float rot_z\n";
    }
    hdr += "end_header\n";
    FILE* f = fopen(filename, "wb");
    if (!f) return fail(TGS_ERR_INVALID, "could not open %s for writing", filename);
    bool ok = fwrite(hdr.data(), 1, hdr.size(), f) == hdr.size();
    if (ok && bytes > 0) ok = fwrite(host.p, 1, (size_t)bytes, f) == (size_t)bytes;
    ok = (fclose(f) == 0) && ok;
    if (!ok) return fail(TGS_ERR_INVALID, "writing %s failed", filename);
    return TGS_OK;
}

int tgs_ply_read_info(const char* filename, tgs_ply_info* info) {
    if (!filename || !info) return fail(TGS_ERR_INVALID, "filename / info is NULL");
    PlyHeader h;
    PlyVertices v;
    TGS_TRY(ply_read_vertices(filename, h, v, false));
    info->n_vertices = v.elem->count;
    info->format = h.format;
    int idx[kPlySlots];
    std::string missing;
    info->has_gaussians = ply_gaussian_slots(*v.elem, idx, missing) ? 1 : 0;
    info->has_colors = (ply_find(*v.elem, "red") >= 0 && ply_find(*v.elem, "green") >= 0 &&
                        ply_find(*v.elem, "blue") >= 0) ? 1 : 0;
    return TGS_OK;
}

int tgs_ply_load_gaussians(const char* filename, const tgs_gaussians* g, void* stream) {
    if (!filename) return fail(TGS_ERR_INVALID, "filename is NULL");
    TGS_TRY(check_ply_gaussians(g));
    hipStream_t s = (hipStream_t)stream;
    PlyHeader h;
    PlyVertices v;
    TGS_TRY(ply_read_vertices(filename, h, v, true));
    if (v.elem->count != g->n)
        return fail(TGS_ERR_INVALID, "%s holds %lld vertices, the arrays %lld rows", filename, (long long)v.elem->count,
                    (long long)g->n);
    int idx[kPlySlots];
    std::string missing;
    if (!ply_gaussian_slots(*v.elem, idx, missing))
        return fail(TGS_ERR_INVALID, "%s: vertex property '%s' missing (not a full-feature Gaussian PLY)", filename,
                    missing.c_str());
    if (g->n == 0) return TGS_OK;
    PlyCol cols[kPlySlots];
    for (int k = 0; k < kPlySlots; ++k) cols[k] = PlyCol{v.offsets[idx[k]], (int32_t)v.elem->props[idx[k]].type};
    const size_t rows_bytes = (v.rows.size() + 15) & ~(size_t)15;
    DeviceScratch dev;
    TGS_HIP(hipMalloc(&dev.p, rows_bytes + sizeof(cols)));
    uint8_t* d_rows = (uint8_t*)dev.p;
    PlyCol* d_cols = (PlyCol*)(d_rows + rows_bytes);
    TGS_HIP(hipMemcpyAsync(d_rows, v.rows.data(), v.rows.size(), hipMemcpyHostToDevice, s));
    TGS_HIP(hipMemcpyAsync(d_cols, cols, sizeof(cols), hipMemcpyHostToDevice, s));
    const PlyDst dst{(float*)g->means, (float*)g->scales, (float*)g->rotations, (float*)g->opacities, g->sh0,
                     g->sh_rest};
    const dim3 grid((unsigned)((45 * g->n + 255) / 256), 6);
    if (g->sh_dtype == TGS_DTYPE_FLOAT16)
        ply_unpack_kernel<__half><<<grid, 256, 0, s>>>(d_rows, v.stride, g->n, d_cols, dst);
    else
        ply_unpack_kernel<float><<<grid, 256, 0, s>>>(d_rows, v.stride, g->n, d_cols, dst);
    TGS_CHECK_LAUNCH();
    TGS_HIP(hipStreamSynchronize(s));
    return TGS_OK;
}

int tgs_point_cloud_load(const char* filename, int64_t* n, float* points, float* colors) {
    if (!filename || !n) return fail(TGS_ERR_INVALID, "filename / n is NULL");
    const std::string fn(filename);
    const std::string ext = fn.size() >= 4 ? fn.substr(fn.size() - 4) : std::string();
    if (ext == ".ply" || ext == ".PLY") {
        PlyHeader h;
        PlyVertices v;
        TGS_TRY(ply_read_vertices(filename, h, v, points != nullptr));
        const int kx = ply_find(*v.elem, "x"), ky = ply_find(*v.elem, "y"), kz = ply_find(*v.elem, "z");
        const int kr = ply_find(*v.elem, "red"), kg = ply_find(*v.elem, "green"), kb = ply_find(*v.elem, "blue");
        if (kx < 0 || ky < 0 || kz < 0) return fail(TGS_ERR_INVALID, "%s: vertex positions x, y, z missing", filename);
        if (kr < 0 || kg < 0 || kb < 0) return fail(TGS_ERR_INVALID, "%s: vertex colors red, green, blue missing", filename);
        for (int k : {kr, kg, kb})
            if (v.elem->props[k].type != PT_UCHAR)
                return fail(TGS_ERR_INVALID, "%s: vertex colors must be uchar", filename);
        if (!points) {
            *n = v.elem->count;
            return TGS_OK;
        }
        if (*n < v.elem->count) return fail(TGS_ERR_INVALID, "%s: %lld points do not fit in %lld", filename,
                                             (long long)v.elem->count, (long long)*n);
        if (!colors) return fail(TGS_ERR_INVALID, "colors is NULL");
        const int kp[3] = {kx, ky, kz}, kc[3] = {kr, kg, kb};
        for (int64_t i = 0; i < v.elem->count; ++i) {
            const uint8_t* row = v.rows.data() + (size_t)i * v.stride;
            for (int c = 0; c < 3; ++c) {
                // getVertexPositions reads doubles; the point is their float rounding
                points[3 * i + c] = (float)ply_host_value(row + v.offsets[kp[c]], v.elem->props[kp[c]].type);
                colors[3 * i + c] = (float)row[v.offsets[kc[c]]] / 255.0f;
            }
        }
        *n = v.elem->count;
        return TGS_OK;
    }
    if (ext == ".txt" || ext == ".TXT") {
        // load_from_colmap (pointcloud.cpp:19-73): lines that are empty or start
        // with '#' are skipped; a line with >= 7 numbers gives XYZ from columns
        // 1-3 and RGB / 255 from columns 4-6
        std::ifstream in(filename);
        if (!in) return fail(TGS_ERR_INVALID, "could not open %s", filename);
        std::string line;
        int64_t count = 0;
        const int64_t cap = *n;
        while (std::getline(in, line)) {
            if (line.empty() || line[0] == '#') continue;
            std::istringstream iss(line);
            std::vector<float> values;
            float value;
            while (iss >> value) values.push_back(value);
            if (values.size() < 7) continue;
            if (points) {
                if (count >= cap) return fail(TGS_ERR_INVALID, "%s: more points than %lld", filename, (long long)cap);
                if (!colors) return fail(TGS_ERR_INVALID, "colors is NULL");
                for (int c = 0; c < 3; ++c) {
                    points[3 * count + c] = values[1 + c];
                    colors[3 * count + c] = values[4 + c] / 255.0f;
                }
            }
            ++count;
        }
        *n = count;
        return TGS_OK;
    }
    return fail(TGS_ERR_UNSUPPORTED, "Unsupported point cloud file format: %s", ext.c_str());
}

int tgs_image_from_hwc_u8(const uint8_t* src, uint32_t width, uint32_t height, uint32_t channels, int32_t bgr,
                          void* dst, int32_t dst_dtype, void* stream) {
    TGS_TRY(check_image_args(src, dst, width, height, channels, bgr));
    if (!img_dtype_ok(dst_dtype)) return fail(TGS_ERR_INVALID, "image dtype %d", dst_dtype);
    hipStream_t s = (hipStream_t)stream;
    const uint32_t tw = (width + 7) / 8, th = (height + 7) / 8, cs = tw * th * 64u;
    const dim3 grid((tw + kStripTiles - 1) / kStripTiles, th);
    if (dst_dtype == IT_F32) hwc_to_tiled_kernel<IT_F32><<<grid, 256, 0, s>>>(src, width, height, channels, bgr, dst, tw, cs);
    else if (dst_dtype == IT_F16) hwc_to_tiled_kernel<IT_F16><<<grid, 256, 0, s>>>(src, width, height, channels, bgr, dst, tw, cs);
    else hwc_to_tiled_kernel<IT_U8><<<grid, 256, 0, s>>>(src, width, height, channels, bgr, dst, tw, cs);
    TGS_CHECK_LAUNCH();
    return TGS_OK;
}

int tgs_image_to_hwc_u8(const void* src, int32_t src_dtype, uint32_t width, uint32_t height, uint32_t channels,
                        int32_t bgr, uint8_t* dst, void* stream) {
    TGS_TRY(check_image_args(src, dst, width, height, channels, bgr));
    if (!img_dtype_ok(src_dtype)) return fail(TGS_ERR_INVALID, "image dtype %d", src_dtype);
    hipStream_t s = (hipStream_t)stream;
    const uint32_t tw = (width + 7) / 8, th = (height + 7) / 8, cs = tw * th * 64u;
    const dim3 grid((tw + kStripTiles - 1) / kStripTiles, th);
    if (src_dtype == IT_F32) tiled_to_hwc_kernel<IT_F32><<<grid, 256, 0, s>>>(src, width, height, channels, bgr, dst, tw, cs);
    else if (src_dtype == IT_F16) tiled_to_hwc_kernel<IT_F16><<<grid, 256, 0, s>>>(src, width, height, channels, bgr, dst, tw, cs);
    else tiled_to_hwc_kernel<IT_U8><<<grid, 256, 0, s>>>(src, width, height, channels, bgr, dst, tw, cs);
    TGS_CHECK_LAUNCH();
    return TGS_OK;
}

int tgs_convert(const void* src, int32_t src_dtype, void* dst, int32_t dst_dtype, int64_t n, void* stream) {
    if (n < 0) return fail(TGS_ERR_INVALID, "element count %lld", (long long)n);
    if (n == 0) return TGS_OK;
    if (!src || !dst) return fail(TGS_ERR_INVALID, "pointer is NULL");
    if (!img_dtype_ok(src_dtype) || !img_dtype_ok(dst_dtype))
        return fail(TGS_ERR_INVALID, "dtypes %d -> %d", src_dtype, dst_dtype);
    hipStream_t s = (hipStream_t)stream;
    const unsigned blocks = (unsigned)((n + 255) / 256);
#define TGS_CONV(S, D) convert_kernel<S, D><<<blocks, 256, 0, s>>>(src, dst, n)
    switch (src_dtype * 3 + dst_dtype) {
        case IT_F32 * 3 + IT_F32: TGS_CONV(IT_F32, IT_F32); break;
        case IT_F32 * 3 + IT_F16: TGS_CONV(IT_F32, IT_F16); break;
        case IT_F32 * 3 + IT_U8: TGS_CONV(IT_F32, IT_U8); break;
        case IT_F16 * 3 + IT_F32: TGS_CONV(IT_F16, IT_F32); break;
        case IT_F16 * 3 + IT_F16: TGS_CONV(IT_F16, IT_F16); break;
        case IT_F16 * 3 + IT_U8: TGS_CONV(IT_F16, IT_U8); break;
        case IT_U8 * 3 + IT_F32: TGS_CONV(IT_U8, IT_F32); break;
        case IT_U8 * 3 + IT_F16: TGS_CONV(IT_U8, IT_F16); break;
        default: TGS_CONV(IT_U8, IT_U8); break;
    }
#undef TGS_CONV
    TGS_CHECK_LAUNCH();
    return TGS_OK;
}

}  // extern "C"
