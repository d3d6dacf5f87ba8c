// I420 frame views and frame_padding (contract of the reference's
// core/src/yuv.cpp:19-31, 232-257, 266-270, 325-337).

#include "mlvc/core/yuv.hpp"

#include <stdexcept>

namespace mlvc {
namespace {

void check_dims(int width, int height)
{
    if (width <= 0 || height <= 0 || width % 2 != 0 || height % 2 != 0)
        throw std::runtime_error("YUV420 dimensions must be positive and even");
}

void check_planes(int width, int height, std::size_t y, std::size_t u, std::size_t v)
{
    check_dims(width, height);
    const std::size_t ysz = static_cast<std::size_t>(width) * static_cast<std::size_t>(height);
    if (y != ysz || u != ysz / 4 || v != ysz / 4) throw std::runtime_error("YUV420 plane sizes do not match dimensions");
}

}  // namespace

Yuv420FrameView::Yuv420FrameView(int width, int height, std::span<const std::uint8_t> y,
                                 std::span<const std::uint8_t> u, std::span<const std::uint8_t> v)
    : width_(width), height_(height), y_(y), u_(u), v_(v)
{
    check_planes(width, height, y.size(), u.size(), v.size());
}

MutableYuv420FrameView::MutableYuv420FrameView(int width, int height, std::span<std::uint8_t> y,
                                               std::span<std::uint8_t> u, std::span<std::uint8_t> v)
    : width_(width), height_(height), y_(y), u_(u), v_(v)
{
    check_planes(width, height, y.size(), u.size(), v.size());
}

std::size_t yuv420_frame_bytes(int width, int height)
{
    check_dims(width, height);
    const std::size_t ysz = static_cast<std::size_t>(width) * static_cast<std::size_t>(height);
    return ysz + 2 * (ysz / 4);
}

FramePadding frame_padding(int width, int height, int model_width, int model_height)
{
    check_dims(width, height);
    check_dims(model_width, model_height);
    const bool native = width <= model_width && height <= model_height;
    const bool transposed = height <= model_width && width <= model_height;
    if (!native && !transposed) throw std::runtime_error("input frame is larger than the model dimensions");
    const int active_w = native ? width : height;
    const int active_h = native ? height : width;
    return FramePadding{0, model_width - active_w, 0, model_height - active_h, !native};
}

}  // namespace mlvc
