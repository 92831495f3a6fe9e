// Host tensor returned by HipBackend: shape + row-major f32 data, the same members and
// accessors as infvino::Tensor (include/infvino/Tensor.hpp:15-45 of the reference).
// Built inside the reference tree with INFVINO_HIP_USE_INFVINO_TENSOR defined, the
// reference's own infvino::Tensor is used instead, so decoders take the outputs unchanged.
#ifndef INFVINO_HIP_TENSOR_HPP_
#define INFVINO_HIP_TENSOR_HPP_

#include <cstddef>
#include <cstdint>
#include <vector>

#ifdef INFVINO_HIP_USE_INFVINO_TENSOR
#include "infvino/Tensor.hpp"
namespace infvino_hip { using Tensor = infvino::Tensor; }
#else
namespace infvino_hip
{
struct Tensor
{
  std::vector<int64_t> shape;
  std::vector<float> data;

  Tensor() = default;
  Tensor(std::vector<int64_t> s, std::vector<float> d) : shape(std::move(s)), data(std::move(d)) {}

  const std::vector<int64_t> & getShape() const { return shape; }
  size_t getSize() const { return data.size(); }
  const float * dataPtr() const { return data.data(); }
  float * dataPtr() { return data.data(); }
  size_t numel() const
  {
    size_t n = 1;
    for (auto d : shape) n *= static_cast<size_t>(d < 0 ? 0 : d);
    return n;
  }
};
}  // namespace infvino_hip
#endif

#endif  // INFVINO_HIP_TENSOR_HPP_
