#pragma once
// I420 frame views and the frame-to-model padding rule used at the codec I/O
// boundary of the buffered backends.
//
// Same contract as the reference's core/include/mlvc/core/yuv.hpp:23-86:
// Yuv420FrameView / MutableYuv420FrameView (plane sizes checked against the
// dimensions), FramePadding, frame_padding() and yuv420_frame_bytes(). The
// reference's CPU conversions (prepare_model_input / prepare_model_output)
// have no counterpart here: this backend converts on the GPU, inside the
// buffered submit path.

#include <cstddef>
#include <cstdint>
#include <span>

namespace mlvc {

class Yuv420FrameView {
public:
    Yuv420FrameView(int width, int height, std::span<const std::uint8_t> y, std::span<const std::uint8_t> u,
                    std::span<const std::uint8_t> v);

    int width() const noexcept { return width_; }
    int height() const noexcept { return height_; }
    std::span<const std::uint8_t> y() const noexcept { return y_; }
    std::span<const std::uint8_t> u() const noexcept { return u_; }
    std::span<const std::uint8_t> v() const noexcept { return v_; }

private:
    int width_;
    int height_;
    std::span<const std::uint8_t> y_, u_, v_;
};

class MutableYuv420FrameView {
public:
    MutableYuv420FrameView(int width, int height, std::span<std::uint8_t> y, std::span<std::uint8_t> u,
                           std::span<std::uint8_t> v);

    int width() const noexcept { return width_; }
    int height() const noexcept { return height_; }
    std::span<std::uint8_t> y() const noexcept { return y_; }
    std::span<std::uint8_t> u() const noexcept { return u_; }
    std::span<std::uint8_t> v() const noexcept { return v_; }

    operator Yuv420FrameView() const { return Yuv420FrameView(width_, height_, y_, u_, v_); }

private:
    int width_;
    int height_;
    std::span<std::uint8_t> y_, u_, v_;
};

// Where the frame sits in the model image: `rotated` frames are transposed
// into it; left/top offsets and right/bottom padding in model pixels.
struct FramePadding {
    int left = 0;
    int right = 0;
    int top = 0;
    int bottom = 0;
    bool rotated = false;
};

// The frame fits as is when width <= model_width and height <= model_height,
// else transposed; padding goes right and bottom (core/src/yuv.cpp:325-337).
FramePadding frame_padding(int width, int height, int model_width, int model_height);

// Bytes of one I420 frame: w*h + 2*(w/2)*(h/2); dimensions positive and even.
std::size_t yuv420_frame_bytes(int width, int height);

}  // namespace mlvc
