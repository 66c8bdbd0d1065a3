// vision.hip - the two gathers of the SigLIP vision tower around its
// transformer: patch extraction (src/hal/common/conv.cpp:179-190) and the
// connector's pixel shuffle (src/models/smolvla/siglip_vision.cpp:188-198).
// Both are pure data movement; each thread moves one float4.
#include "common.h"

namespace vla {
namespace hip {

namespace {

// out [grid*grid, 3*P*P], row = ph*grid + pw, column = ic*P*P + kh*P + kw,
// from pixels [3, img, img] (CHW). P % 4 == 0: four kw share a float4 on
// both sides.
__global__ __launch_bounds__(256) void extract_patches_kernel(float* __restrict__ out,
                                                              const float* __restrict__ pix, int img,
                                                              int P, int grid, int64_t n4) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= n4) return;
    const int64_t e = i * 4;  // first output element of this float4
    const int PD = 3 * P * P;
    const int p = (int)(e / PD), col = (int)(e % PD);
    const int ic = col / (P * P), r = col % (P * P);
    const int kh = r / P, kw = r % P;
    const int ph = p / grid, pw = p % grid;
    const float4 v = *reinterpret_cast<const float4*>(pix + ((size_t)ic * img + ph * P + kh) * img + pw * P + kw);
    *reinterpret_cast<float4*>(out + e) = v;
}

// dst [side*side, H] viewed as [n_tok, sf*sf*H]: row t*sf*sf + dh*sf + dw of
// dst is patch (h2*sf + dh)*side + (w2*sf + dw) of src, t = h2*g2 + w2.
__global__ __launch_bounds__(256) void pixel_shuffle_kernel(float* __restrict__ dst,
                                                            const float* __restrict__ src, int H, int sf,
                                                            int side) {
    const int row = blockIdx.y;
    const int c = (blockIdx.x * 256 + threadIdx.x) * 4;
    if (c >= H) return;
    const int g2 = side / sf, blk = sf * sf;
    const int t = row / blk, b = row % blk;
    const int h2 = t / g2, w2 = t % g2, dh = b / sf, dw = b % sf;
    const int sp = (h2 * sf + dh) * side + (w2 * sf + dw);
    *reinterpret_cast<float4*>(dst + (size_t)row * H + c) =
        *reinterpret_cast<const float4*>(src + (size_t)sp * H + c);
}

}  // namespace

void launch_extract_patches(float* out, const float* pixels, int img, int patch, hipStream_t st) {
    VLA_REQUIRE(img > 0 && patch > 0 && img % patch == 0, "extract_patches: img must be a multiple of patch");
    VLA_REQUIRE(patch % 4 == 0 && img % 4 == 0, "extract_patches: patch must be a multiple of 4");
    VLA_REQUIRE(aligned(out, 16) && aligned(pixels, 16), "extract_patches: buffers must be 16-byte aligned");
    const int grid = img / patch;
    const int64_t n4 = (int64_t)grid * grid * 3 * patch * patch / 4;
    VLA_REQUIRE((n4 + 255) / 256 < 2147483647LL, "extract_patches: image too large");
    extract_patches_kernel<<<(unsigned)((n4 + 255) / 256), 256, 0, st>>>(out, pixels, img, patch, grid, n4);
    VLA_LAUNCH_CHECK();
}

void launch_pixel_shuffle(float* dst, const float* src, int side, int hidden, int sf, hipStream_t st) {
    VLA_REQUIRE(side > 0 && sf > 0 && side % sf == 0, "pixel_shuffle: side must be a multiple of the scale factor");
    VLA_REQUIRE(hidden > 0 && hidden % 4 == 0, "pixel_shuffle: hidden must be a multiple of 4");
    VLA_REQUIRE(aligned(dst, 16) && aligned(src, 16), "pixel_shuffle: buffers must be 16-byte aligned");
    VLA_REQUIRE((int64_t)side * side < 65536, "pixel_shuffle: too many patches");
    pixel_shuffle_kernel<<<dim3((hidden / 4 + 255) / 256, side * side), 256, 0, st>>>(dst, src, hidden, sf, side);
    VLA_LAUNCH_CHECK();
}

}  // namespace hip
}  // namespace vla
