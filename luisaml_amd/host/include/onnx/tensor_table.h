// tensor_table.h -- name -> tensor map with the reference's ownership
// convention and lookup API (include/onnx/tensor_table.h:22-214):
// intermediates, weights and packed weights are owned (unique_ptr); external
// inputs and outputs are borrowed (reference_wrapper).  Lookups fall back to
// a parent table (set_parent), as a subgraph's table does to its graph's.
// Operators only ever receive references.
#pragma once

#include <functional>
#include <memory>
#include <string>
#include <unordered_map>
#include <variant>

#include "onnx/tensor.h"

namespace lcml::onnx {

// One table entry: an owned tensor or a borrowed reference, read the same way.
class TensorEntry {
public:
    using OwnedPtr = std::unique_ptr<ITensor>;
    using BorrowedRef = std::reference_wrapper<ITensor>;

private:
    std::variant<OwnedPtr, BorrowedRef> storage_;

public:
    explicit TensorEntry(OwnedPtr p) : storage_(std::move(p)) {}
    explicit TensorEntry(BorrowedRef r) : storage_(r) {}
    explicit TensorEntry(ITensor &t) : storage_(std::ref(t)) {}
    TensorEntry(TensorEntry &&) noexcept = default;
    TensorEntry &operator=(TensorEntry &&) noexcept = default;
    TensorEntry(const TensorEntry &) = delete;
    TensorEntry &operator=(const TensorEntry &) = delete;

    bool is_owned() const noexcept { return std::holds_alternative<OwnedPtr>(storage_); }
    bool is_borrowed() const noexcept { return std::holds_alternative<BorrowedRef>(storage_); }
    ITensor &get() {
        if (auto *p = std::get_if<OwnedPtr>(&storage_)) return **p;
        return std::get<BorrowedRef>(storage_).get();
    }
    const ITensor &get() const {
        if (auto *p = std::get_if<OwnedPtr>(&storage_)) return **p;
        return std::get<BorrowedRef>(storage_).get();
    }
    operator ITensor &() { return get(); }
    operator const ITensor &() const { return get(); }
    // moves the owned tensor out (nullptr for a borrowed entry); the entry
    // is then empty and should be erased
    OwnedPtr release_owned() {
        auto *p = std::get_if<OwnedPtr>(&storage_);
        return p ? std::move(*p) : nullptr;
    }
};

class TensorTable {
public:
    using MapType = std::unordered_map<std::string, TensorEntry>;
    using iterator = MapType::iterator;
    using const_iterator = MapType::const_iterator;

private:
    MapType map_;
    TensorTable *parent_ = nullptr;

    const TensorEntry *find(std::string_view name) const {
        auto it = map_.find(std::string(name));
        if (it != map_.end()) return &it->second;
        return parent_ ? parent_->find(name) : nullptr;
    }

public:
    TensorTable() = default;
    TensorTable(TensorTable &&) noexcept = default;
    TensorTable &operator=(TensorTable &&) noexcept = default;
    TensorTable(const TensorTable &) = delete;
    TensorTable &operator=(const TensorTable &) = delete;

    // ---- parent (fallback for lookups) ----
    void set_parent(TensorTable *parent) noexcept { parent_ = parent; }
    TensorTable *parent() const noexcept { return parent_; }

    // ---- insertion (replaces an entry of the same name) ----
    void bind(std::string name, ITensor &t) { map_.insert_or_assign(std::move(name), TensorEntry{std::ref(t)}); }
    void own(std::string name, std::unique_ptr<ITensor> t) {
        map_.insert_or_assign(std::move(name), TensorEntry{std::move(t)});
    }

    // ---- lookup: local entries first, then the parent chain ----
    ITensor &at(std::string_view name) {
        const TensorEntry *e = find(name);
        LCML_ASSERT(e != nullptr, "TensorTable: key not found: %.*s", (int)name.size(), name.data());
        return const_cast<TensorEntry *>(e)->get();
    }
    const ITensor &at(std::string_view name) const {
        const TensorEntry *e = find(name);
        LCML_ASSERT(e != nullptr, "TensorTable: key not found: %.*s", (int)name.size(), name.data());
        return e->get();
    }
    bool contains(std::string_view name) const { return find(name) != nullptr; }
    bool contains_local(std::string_view name) const { return map_.find(std::string(name)) != map_.end(); }
    // the local entry (ownership inspection); asserts when absent
    TensorEntry &entry(std::string_view name) {
        auto it = map_.find(std::string(name));
        LCML_ASSERT(it != map_.end(), "TensorTable: key not found: %.*s", (int)name.size(), name.data());
        return it->second;
    }
    const TensorEntry &entry(std::string_view name) const {
        auto it = map_.find(std::string(name));
        LCML_ASSERT(it != map_.end(), "TensorTable: key not found: %.*s", (int)name.size(), name.data());
        return it->second;
    }
    bool is_owned(std::string_view name) const {
        auto it = map_.find(std::string(name));
        return it != map_.end() && it->second.is_owned();
    }

    // ---- capacity and removal ----
    size_t size() const noexcept { return map_.size(); }
    bool empty() const noexcept { return map_.empty(); }
    void clear() noexcept { map_.clear(); }
    void erase(std::string_view name) { map_.erase(std::string(name)); }
    // removes a local owned entry and hands its tensor to the caller;
    // nullptr (and the table unchanged) when absent or borrowed
    std::unique_ptr<ITensor> release_owned(std::string_view name) {
        auto it = map_.find(std::string(name));
        if (it == map_.end() || !it->second.is_owned()) return nullptr;
        auto t = it->second.release_owned();
        map_.erase(it);
        return t;
    }

    // ---- iteration over the local entries ----
    iterator begin() noexcept { return map_.begin(); }
    iterator end() noexcept { return map_.end(); }
    const_iterator begin() const noexcept { return map_.begin(); }
    const_iterator end() const noexcept { return map_.end(); }
    const_iterator cbegin() const noexcept { return map_.cbegin(); }
    const_iterator cend() const noexcept { return map_.cend(); }
};

}  // namespace lcml::onnx
