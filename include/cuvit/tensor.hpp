#pragma once

// Non-owning strided view, the counterpart of the reference's TensorView<T>
// (include/cuvit/tensor.hpp:15-262). Host-only; no HIP include. Strides are in
// elements. Rank is 1..kMaxTensorRank. Views never own memory: slicing,
// selecting, transposing and reshaping only change the description.

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

template <typename T> class TensorView {
    static_assert(!std::is_reference<T>::value, "TensorView cannot view references");

  public:
    using value_type = T;

    TensorView() noexcept = default;

    /// Contiguous row-major view of @p data.
    TensorView(T* data, std::initializer_list<Extent> extents) {
        set_extents(extents);
        set_packed_strides();
        data_ = data;
        require_data();
    }

    /// View with explicit strides.
    static TensorView strided(T* data, std::initializer_list<Extent> extents,
                              std::initializer_list<Extent> strides) {
        if (extents.size() != strides.size()) {
            throw std::invalid_argument("TensorView needs one stride per extent");
        }
        TensorView view;
        view.set_extents(extents);
        int axis = 0;
        for (const Extent stride : strides) {
            if (stride < 0) {
                throw std::invalid_argument("TensorView strides cannot be negative");
            }
            view.strides_[static_cast<std::size_t>(axis++)] = stride;
        }
        view.data_ = data;
        view.require_data();
        return view;
    }

    [[nodiscard]] TensorView<const T> as_const() const noexcept {
        TensorView<const T> view;
        view.data_ = data_;
        view.extents_ = extents_;
        view.strides_ = strides_;
        view.rank_ = rank_;
        return view;
    }

    [[nodiscard]] int rank() const noexcept { return rank_; }
    [[nodiscard]] bool empty() const noexcept { return size() == 0; }
    [[nodiscard]] T* data() const noexcept { return data_; }
    [[nodiscard]] Extent extent(int axis) const { return extents_[index(axis)]; }
    [[nodiscard]] Extent stride(int axis) const { return strides_[index(axis)]; }

    /// Elements addressed by the view (not the size of the allocation).
    [[nodiscard]] Extent size() const noexcept {
        Extent total = 1;
        for (int axis = 0; axis < rank_; ++axis) {
            total *= extents_[static_cast<std::size_t>(axis)];
        }
        return total;
    }

    [[nodiscard]] std::size_t bytes() const noexcept {
        return static_cast<std::size_t>(size()) * sizeof(T);
    }

    /// Dense row-major layout; axes of extent one constrain nothing.
    [[nodiscard]] bool is_contiguous() const noexcept {
        Extent expected = 1;
        for (int axis = rank_ - 1; axis >= 0; --axis) {
            const auto a = static_cast<std::size_t>(axis);
            if (extents_[a] == 1) {
                continue;
            }
            if (strides_[a] != expected) {
                return false;
            }
            expected *= extents_[a];
        }
        return true;
    }

    [[nodiscard]] Extent offset_of(std::initializer_list<Extent> indices) const {
        if (static_cast<int>(indices.size()) != rank_) {
            throw std::invalid_argument("TensorView index has the wrong rank");
        }
        Extent offset = 0;
        std::size_t axis = 0;
        for (const Extent i : indices) {
            if (i < 0 || i >= extents_[axis]) {
                throw std::out_of_range("TensorView index is out of range on axis " +
                                        std::to_string(axis));
            }
            offset += i * strides_[axis];
            ++axis;
        }
        return offset;
    }

    /// Keeps @p count entries of @p axis starting at @p start; rank unchanged.
    [[nodiscard]] TensorView slice(int axis, Extent start, Extent count) const {
        const std::size_t a = index(axis);
        if (start < 0 || count < 0 || start > extents_[a] || count > extents_[a] - start) {
            throw std::out_of_range("TensorView slice exceeds the extent of axis " +
                                    std::to_string(axis));
        }
        TensorView view = *this;
        view.data_ = data_ + start * strides_[a];
        view.extents_[a] = count;
        return view;
    }

    /// Fixes @p axis at @p position and removes it.
    [[nodiscard]] TensorView select(int axis, Extent position) const {
        const std::size_t a = index(axis);
        if (position < 0 || position >= extents_[a]) {
            throw std::out_of_range("TensorView select is out of range on axis " +
                                    std::to_string(axis));
        }
        TensorView view;
        view.data_ = data_ + position * strides_[a];
        view.rank_ = rank_ - 1;
        std::size_t out = 0;
        for (std::size_t in = 0; in < static_cast<std::size_t>(rank_); ++in) {
            if (in != a) {
                view.extents_[out] = extents_[in];
                view.strides_[out] = strides_[in];
                ++out;
            }
        }
        return view;
    }

    /// Swaps two axes; no data moves.
    [[nodiscard]] TensorView transpose(int first, int second) const {
        const std::size_t a = index(first);
        const std::size_t b = index(second);
        TensorView view = *this;
        std::swap(view.extents_[a], view.extents_[b]);
        std::swap(view.strides_[a], view.strides_[b]);
        return view;
    }

    /// New shape over the same elements; only for contiguous views.
    [[nodiscard]] TensorView reshape(std::initializer_list<Extent> extents) const {
        if (!is_contiguous()) {
            throw std::invalid_argument("Only a contiguous TensorView can be reshaped");
        }
        TensorView view;
        view.set_extents(extents);
        if (view.size() != size()) {
            throw std::invalid_argument("TensorView reshape changes the element count");
        }
        view.set_packed_strides();
        view.data_ = data_;
        return view;
    }

    [[nodiscard]] std::string shape_string() const {
        std::string text = "[";
        for (int axis = 0; axis < rank_; ++axis) {
            text += (axis == 0 ? "" : ", ") + std::to_string(extents_[static_cast<std::size_t>(axis)]);
        }
        return text + ']';
    }

  private:
    template <typename U> friend class TensorView;

    void set_extents(std::initializer_list<Extent> extents) {
        if (extents.size() == 0 || extents.size() > static_cast<std::size_t>(kMaxTensorRank)) {
            throw std::invalid_argument("TensorView rank must be between 1 and " +
                                        std::to_string(kMaxTensorRank));
        }
        rank_ = static_cast<int>(extents.size());
        std::size_t axis = 0;
        for (const Extent e : extents) {
            if (e < 0) {
                throw std::invalid_argument("TensorView extents cannot be negative");
            }
            extents_[axis++] = e;
        }
    }

    void set_packed_strides() noexcept {
        Extent stride = 1;
        for (int axis = rank_ - 1; axis >= 0; --axis) {
            strides_[static_cast<std::size_t>(axis)] = stride;
            stride *= extents_[static_cast<std::size_t>(axis)];
        }
    }

    void require_data() const {
        if (data_ == nullptr && size() != 0) {
            throw std::invalid_argument("A non-empty TensorView cannot view a null pointer");
        }
    }

    [[nodiscard]] std::size_t index(int axis) const {
        if (axis < 0 || axis >= rank_) {
            throw std::out_of_range("TensorView axis " + std::to_string(axis) +
                                    " is outside a rank-" + std::to_string(rank_) + " tensor");
        }
        return static_cast<std::size_t>(axis);
    }

    T* data_ = nullptr;
    std::array<Extent, kMaxTensorRank> extents_{};
    std::array<Extent, kMaxTensorRank> strides_{};
    int rank_ = 0;
};

} // namespace cuvit
