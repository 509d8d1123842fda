#pragma once

// A non-owning, strided view of device or host memory. Interface of the
// reference's TensorView<T> (include/cuvit/tensor.hpp:15-262): rank 1 to
// kMaxTensorRank, extents and element strides, offsets of index tuples, and
// views derived without moving data (slice, select, transpose, reshape).
// Host-only; nothing here touches the memory it describes.
//
// The shape arithmetic lives in Layout, a plain value type; a TensorView is a
// pointer plus a Layout, and every derived view is a new Layout over an
// adjusted pointer.

#include <array>
#include <cstddef>
#include <cstdint>
#include <initializer_list>
#include <stdexcept>
#include <string>
#include <type_traits>
#include <utility>

namespace cuvit {

/// [batch, heads, tokens, head_dim] is the deepest shape a ViT needs.
inline constexpr int kMaxTensorRank = 4;

using Extent = std::int64_t;

namespace detail {

struct Layout {
    int rank = 0;
    std::array<Extent, kMaxTensorRank> extent{};
    std::array<Extent, kMaxTensorRank> stride{};

    /// A layout of the given extents, strides not yet set.
    static Layout with_extents(std::initializer_list<Extent> extents) {
        const std::size_t rank = extents.size();
        if (rank < 1 || rank > static_cast<std::size_t>(kMaxTensorRank)) {
            throw std::invalid_argument("A TensorView has rank 1 to " +
                                        std::to_string(kMaxTensorRank) + ", not " +
                                        std::to_string(rank));
        }
        Layout layout;
        layout.rank = static_cast<int>(rank);
        auto out = layout.extent.begin();
        for (const Extent e : extents) {
            if (e < 0) {
                throw std::invalid_argument("TensorView extents cannot be negative");
            }
            *out++ = e;
        }
        return layout;
    }

    /// Row-major strides: each axis steps over everything after it.
    Layout& packed() noexcept {
        Extent step = 1;
        for (int a = rank; a-- > 0;) {
            stride[static_cast<std::size_t>(a)] = step;
            step *= extent[static_cast<std::size_t>(a)];
        }
        return *this;
    }

    [[nodiscard]] Extent count() const noexcept {
        Extent total = 1;
        for (int a = 0; a < rank; ++a) {
            total *= extent[static_cast<std::size_t>(a)];
        }
        return total;
    }

    /// Row-major dense, where axes of extent one may have any stride.
    [[nodiscard]] bool dense() const noexcept {
        Layout reference = *this;
        reference.packed();
        for (std::size_t a = 0; a < static_cast<std::size_t>(rank); ++a) {
            if (extent[a] != 1 && stride[a] != reference.stride[a]) {
                return false;
            }
        }
        return true;
    }

    /// @p axis as an array index; out_of_range unless 0 <= axis < rank.
    [[nodiscard]] std::size_t at(int axis) const {
        if (axis >= 0 && axis < rank) {
            return static_cast<std::size_t>(axis);
        }
        throw std::out_of_range("Axis " + std::to_string(axis) + " does not exist in a rank-" +
                                std::to_string(rank) + " TensorView");
    }

    /// This layout with axis @p a removed.
    [[nodiscard]] Layout without(std::size_t a) const noexcept {
        Layout fewer;
        fewer.rank = rank - 1;
        for (std::size_t in = 0, out = 0; in < static_cast<std::size_t>(rank); ++in) {
            if (in == a) {
                continue;
            }
            fewer.extent[out] = extent[in];
            fewer.stride[out] = stride[in];
            ++out;
        }
        return fewer;
    }
};

} // namespace detail

template <typename T> class TensorView {
    static_assert(!std::is_reference<T>::value, "TensorView elements cannot be references");

  public:
    using value_type = T;

    TensorView() noexcept = default;

    /// A dense row-major view of @p data.
    TensorView(T* data, std::initializer_list<Extent> extents)
        : TensorView(data, detail::Layout::with_extents(extents).packed()) {}

    /// A view with the given element strides (non-negative, one per extent).
    static TensorView strided(T* data, std::initializer_list<Extent> extents,
                              std::initializer_list<Extent> strides) {
        detail::Layout layout = detail::Layout::with_extents(extents);
        if (strides.size() != extents.size()) {
            throw std::invalid_argument("A strided TensorView needs as many strides as extents");
        }
        auto out = layout.stride.begin();
        for (const Extent s : strides) {
            if (s < 0) {
                throw std::invalid_argument("TensorView strides cannot be negative");
            }
            *out++ = s;
        }
        return TensorView(data, layout);
    }

    [[nodiscard]] TensorView<const T> as_const() const noexcept {
        return TensorView<const T>(data_, layout_, typename TensorView<const T>::Unchecked{});
    }

    [[nodiscard]] int rank() const noexcept { return layout_.rank; }
    [[nodiscard]] bool empty() const noexcept { return layout_.count() == 0; }
    [[nodiscard]] T* data() const noexcept { return data_; }
    [[nodiscard]] Extent extent(int axis) const { return layout_.extent[layout_.at(axis)]; }
    [[nodiscard]] Extent stride(int axis) const { return layout_.stride[layout_.at(axis)]; }

    /// Elements the view addresses (not the size of the memory behind it).
    [[nodiscard]] Extent size() const noexcept { return layout_.count(); }
    [[nodiscard]] std::size_t bytes() const noexcept {
        return static_cast<std::size_t>(layout_.count()) * sizeof(T);
    }
    [[nodiscard]] bool is_contiguous() const noexcept { return layout_.dense(); }

    /// The element offset of an index tuple, one index per axis, each in range.
    [[nodiscard]] Extent offset_of(std::initializer_list<Extent> indices) const {
        if (static_cast<int>(indices.size()) != layout_.rank) {
            throw std::invalid_argument("A TensorView of rank " + std::to_string(layout_.rank) +
                                        " takes " + std::to_string(layout_.rank) + " indices, not " +
                                        std::to_string(indices.size()));
        }
        Extent offset = 0;
        std::size_t a = 0;
        for (const Extent i : indices) {
            if (i < 0 || i >= layout_.extent[a]) {
                throw std::out_of_range("Index " + std::to_string(i) + " is outside axis " +
                                        std::to_string(a) + " of extent " +
                                        std::to_string(layout_.extent[a]));
            }
            offset += i * layout_.stride[a++];
        }
        return offset;
    }

    /// Entries [start, start + count) of @p axis; the rank stays.
    [[nodiscard]] TensorView slice(int axis, Extent start, Extent count) const {
        const std::size_t a = layout_.at(axis);
        const Extent length = layout_.extent[a];
        if (!(start >= 0 && count >= 0 && start <= length && count <= length - start)) {
            throw std::out_of_range("Slice [" + std::to_string(start) + ", +" +
                                    std::to_string(count) + ") leaves axis " +
                                    std::to_string(axis) + " of extent " + std::to_string(length));
        }
        detail::Layout layout = layout_;
        layout.extent[a] = count;
        return TensorView(data_ + start * layout_.stride[a], layout, Unchecked{});
    }

    /// Entry @p position of @p axis, with that axis dropped.
    [[nodiscard]] TensorView select(int axis, Extent position) const {
        const std::size_t a = layout_.at(axis);
        if (position < 0 || position >= layout_.extent[a]) {
            throw std::out_of_range("Position " + std::to_string(position) + " is outside axis " +
                                    std::to_string(axis) + " of extent " +
                                    std::to_string(layout_.extent[a]));
        }
        return TensorView(data_ + position * layout_.stride[a], layout_.without(a), Unchecked{});
    }

    /// The view with two axes exchanged; no element moves.
    [[nodiscard]] TensorView transpose(int first, int second) const {
        const std::size_t a = layout_.at(first);
        const std::size_t b = layout_.at(second);
        detail::Layout layout = layout_;
        std::swap(layout.extent[a], layout.extent[b]);
        std::swap(layout.stride[a], layout.stride[b]);
        return TensorView(data_, layout, Unchecked{});
    }

    /// The same elements under new extents; the view must be dense.
    [[nodiscard]] TensorView reshape(std::initializer_list<Extent> extents) const {
        if (!layout_.dense()) {
            throw std::invalid_argument("A strided TensorView cannot be reshaped");
        }
        detail::Layout layout = detail::Layout::with_extents(extents);
        if (layout.count() != layout_.count()) {
            throw std::invalid_argument("Reshaping " + shape_string() + " to " +
                                        std::to_string(layout.count()) +
                                        " elements changes the element count");
        }
        return TensorView(data_, layout.packed(), Unchecked{});
    }

    /// "[e0, e1, ...]".
    [[nodiscard]] std::string shape_string() const {
        std::string text(1, '[');
        for (int a = 0; a < layout_.rank; ++a) {
            if (a != 0) {
                text += ", ";
            }
            text += std::to_string(layout_.extent[static_cast<std::size_t>(a)]);
        }
        text += ']';
        return text;
    }

  private:
    template <typename U> friend class TensorView;
    struct Unchecked {};

    /// A view of a layout built here or by the caller; a null pointer is only
    /// allowed when the view is empty.
    TensorView(T* data, const detail::Layout& layout) : data_(data), layout_(layout) {
        if (data == nullptr && layout.count() != 0) {
            throw std::invalid_argument("A TensorView with elements cannot view a null pointer");
        }
    }

    /// A view derived from a valid one: nothing to check.
    TensorView(T* data, const detail::Layout& layout, Unchecked) noexcept
        : data_(data), layout_(layout) {}

    T* data_ = nullptr;
    detail::Layout layout_{};
};

} // namespace cuvit
