// type_dispatch.h -- element type identity and typed dispatch, as in the
// reference (include/onnx/type_dispatch.h:17-20, 104-122): a type index is a
// hash of the type's name, and visit_type_index<List> calls a templated
// lambda with the C++ type whose index matches.
#pragma once

#include <cstdint>
#include <string_view>
#include <tuple>
#include <type_traits>

#include "onnx/error.h"

namespace lcml::onnx {

// Element types of the FP8 linear path.  The fp8 and bf16 structs are type
// tags over dense device bytes (one byte per fp8 element, two per bf16).
struct FP8E4M3FN {
    uint8_t bits;
};
struct FP8E5M2 {
    uint8_t bits;
};
struct BFloat16 {
    uint16_t bits;
};

template <typename T>
struct TypeName;
template <> struct TypeName<float> { static constexpr std::string_view value = "float"; };
template <> struct TypeName<FP8E4M3FN> { static constexpr std::string_view value = "FP8E4M3FN"; };
template <> struct TypeName<FP8E5M2> { static constexpr std::string_view value = "FP8E5M2"; };
template <> struct TypeName<BFloat16> { static constexpr std::string_view value = "bfloat16"; };
template <> struct TypeName<int64_t> { static constexpr std::string_view value = "int64"; };
template <typename T>
inline constexpr std::string_view type_name_v = TypeName<T>::value;

namespace refl {

using TypeIndex = uint64_t;

constexpr TypeIndex fnv1a(std::string_view s) {
    uint64_t h = 1469598103934665603ull;
    for (char c : s) {
        h ^= (uint8_t)c;
        h *= 1099511628211ull;
    }
    return h;
}

template <typename T>
constexpr TypeIndex type_index_of() noexcept {
    return fnv1a(type_name_v<T>);
}

}  // namespace refl

using NNTypeList = std::tuple<float, FP8E4M3FN, FP8E5M2, BFloat16, int64_t>;

namespace detail {
template <typename Tuple, size_t I = 0, typename F>
void visit_impl(refl::TypeIndex idx, F &&f) {
    if constexpr (I < std::tuple_size_v<Tuple>) {
        using T = std::tuple_element_t<I, Tuple>;
        if (refl::type_index_of<T>() == idx) {
            f.template operator()<T>();
            return;
        }
        visit_impl<Tuple, I + 1>(idx, std::forward<F>(f));
    } else {
        LCML_ASSERT(false, "unsupported element type index %llu", (unsigned long long)idx);
    }
}
}  // namespace detail

template <typename TypeList, typename F>
void visit_type_index(refl::TypeIndex idx, F &&f) {
    detail::visit_impl<TypeList>(idx, std::forward<F>(f));
}

}  // namespace lcml::onnx
