#pragma once
// Host tensor types crossing the backend boundary.
//
// Same contract as the reference's core/include/mlvc/core/tensor.hpp:19-120:
// FP16 values travel as raw binary16 bit patterns, tensors own their storage
// and carry an NCHW shape. Only the parts the inference path uses are kept.

#include <cstddef>
#include <cstdint>
#include <limits>
#include <span>
#include <stdexcept>
#include <string>
#include <string_view>
#include <type_traits>
#include <variant>
#include <vector>

namespace mlvc {

enum class TensorDataType { kFloat16, kInt32 };

using Float16Storage = std::uint16_t;
using TensorStorage =
    std::variant<std::vector<Float16Storage>, std::vector<std::int32_t>>;

inline std::size_t tensor_data_type_size(TensorDataType type)
{
    return type == TensorDataType::kFloat16 ? sizeof(Float16Storage)
                                            : sizeof(std::int32_t);
}

inline std::size_t checked_tensor_element_count(std::span<const std::int64_t> shape)
{
    std::size_t count = 1;
    for (const std::int64_t extent : shape) {
        if (extent <= 0)
            throw std::runtime_error("tensor dimensions must be positive");
        const auto e = static_cast<std::size_t>(extent);
        if (count > std::numeric_limits<std::size_t>::max() / e)
            throw std::runtime_error("tensor element count overflows size_t");
        count *= e;
    }
    return count;
}

struct Tensor {
    std::string name;
    std::vector<std::int64_t> shape;
    TensorStorage data;

    TensorDataType data_type() const noexcept
    {
        return std::holds_alternative<std::vector<Float16Storage>>(data)
                   ? TensorDataType::kFloat16
                   : TensorDataType::kInt32;
    }
    std::size_t element_count() const noexcept
    {
        return std::visit([](const auto& v) { return v.size(); }, data);
    }
    std::size_t byte_size() const noexcept
    {
        return std::visit(
            [](const auto& v) {
                return v.size() * sizeof(typename std::decay_t<decltype(v)>::value_type);
            },
            data);
    }
    const void* raw_data() const noexcept
    {
        return std::visit([](const auto& v) -> const void* { return v.data(); }, data);
    }
    void* raw_data() noexcept
    {
        return std::visit([](auto& v) -> void* { return v.data(); }, data);
    }
    void validate() const
    {
        if (checked_tensor_element_count(shape) != element_count())
            throw std::runtime_error("tensor shape does not match its storage");
    }
};

// Non-owning views over host tensor storage (shape span and data must
// outlive the view), as returned by the buffered codec slots. Contract of
// the reference's core/include/mlvc/core/tensor.hpp:104-200: the element
// count must match the shape, and from_raw checks the byte size.
template <bool Mutable>
class BasicTensorView {
public:
    using Pointer = std::conditional_t<Mutable, void*, const void*>;

    static BasicTensorView from_raw(std::string_view name, std::span<const std::int64_t> shape, TensorDataType type,
                                    Pointer data, std::size_t bytes)
    {
        const std::size_t count = checked_tensor_element_count(shape);
        if (data == nullptr || bytes != count * tensor_data_type_size(type))
            throw std::runtime_error("tensor view shape does not match its storage");
        return BasicTensorView(name, shape, type, data, count);
    }

    std::string_view name() const noexcept { return name_; }
    std::span<const std::int64_t> shape() const noexcept { return shape_; }
    TensorDataType data_type() const noexcept { return type_; }
    Pointer raw_data() const noexcept { return data_; }
    std::size_t element_count() const noexcept { return count_; }
    std::size_t byte_size() const noexcept { return count_ * tensor_data_type_size(type_); }

private:
    BasicTensorView(std::string_view name, std::span<const std::int64_t> shape, TensorDataType type, Pointer data,
                    std::size_t count)
        : name_(name), shape_(shape), type_(type), data_(data), count_(count)
    {
    }
    std::string_view name_;
    std::span<const std::int64_t> shape_;
    TensorDataType type_;
    Pointer data_;
    std::size_t count_;
};

using TensorView = BasicTensorView<false>;
using MutableTensorView = BasicTensorView<true>;

}  // namespace mlvc
