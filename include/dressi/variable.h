/* dressi/variable.h -- Variable: a node of the computational graph holding
 * one image (the reference's include/dressi/variable.h:18-72: a shared
 * handle to its node; copies name the same node). Node ids come from one
 * counter, so creation order is a topological order. */
#ifndef DRESSI_VARIABLE_H
#define DRESSI_VARIABLE_H

#include <cstddef>
#include <cstdint>
#include <functional>
#include <memory>
#include <vector>

#include "dressi/types.h"

namespace dressi {

struct VariableNode;
class Function;

class Variable {
public:
    Variable(VType vtype = FLOAT, ImgSize img_size = {1, 1});
    Variable(std::nullptr_t) {}  // null handle: "no gradient"

    explicit operator bool() const { return m_node != nullptr; }
    bool operator==(const Variable& o) const { return m_node == o.m_node; }
    bool operator!=(const Variable& o) const { return m_node != o.m_node; }
    uint64_t id() const;

    VType getVType() const;
    void setVType(VType vtype);
    ImgSize getImgSize() const;
    void setImgSize(ImgSize img_size);
    Function getCreator() const;
    void setCreator(const Function& creator);
    std::vector<Function> getUsers() const;
    void addUser(const Function& user);
    bool getRequiresGrad() const;
    void setRequiresGrad(bool req_grad);
    // this variable and everything computed from it
    void setRequiresGradRecursively(bool req_grad = true);
    // "changed since the last execStep": set by sendImg, cleared (with
    // everything downstream) once an execStep has consumed it
    bool IsDirty() const;
    void setDirty(bool is_dirty);
    void setDirtyRecursively(bool is_dirty);

private:
    friend struct NodeAccess;
    explicit Variable(std::shared_ptr<VariableNode> node) : m_node(std::move(node)) {}
    std::shared_ptr<VariableNode> m_node;
};

using Variables = std::vector<Variable>;

}  // namespace dressi

template <>
struct std::hash<dressi::Variable> {
    size_t operator()(const dressi::Variable& v) const {
        return v ? std::hash<uint64_t>()(v.id()) : 0;
    }
};

// Maps keyed by Variable order them by creation id (operator< itself builds
// a comparison node, see dressi/f.h)
template <>
struct std::less<dressi::Variable> {
    bool operator()(const dressi::Variable& a, const dressi::Variable& b) const {
        return (a ? a.id() : 0) < (b ? b.id() : 0);
    }
};

#endif  // DRESSI_VARIABLE_H
