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

}  // namespace mlvc
