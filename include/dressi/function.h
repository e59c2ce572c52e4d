/* dressi/function.h -- Function: an operation of the computational graph
 * with its backward generator (the reference's include/dressi/function.h:
 * 20-74). Graphs are normally built with the F:: catalogue (dressi/f.h);
 * a Function made from the public constructor carries the reference's
 * GLSL snippet as text and connects into graphs (buildFwd infers the
 * output like an elementwise op), but the HIP executor has no GLSL
 * compiler: executing it raises DressiError. */
#ifndef DRESSI_FUNCTION_H
#define DRESSI_FUNCTION_H

#include <cstddef>
#include <cstdint>
#include <functional>
#include <memory>
#include <string>

#include "dressi/types.h"
#include "dressi/variable.h"

namespace dressi {

struct FunctionNode;

// The gradient graph of input xs[bwd_idx] given the output y and its
// incoming gradient gy; a null Variable means "no gradient"
using BwdFunc = std::function<Variable(const Variables& xs, const Variable& y,
                                       const Variable& gy, uint32_t bwd_idx)>;

class Function {
public:
    Function() = default;
    Function(std::nullptr_t) {}
    Function(const std::string& code, ShaderType type, const BwdFunc& bwd_func);

    explicit operator bool() const { return m_node != nullptr; }
    bool operator==(const Function& o) const { return m_node == o.m_node; }
    bool operator!=(const Function& o) const { return m_node != o.m_node; }
    uint64_t id() const;

    std::string getFwdCode() const;  // GLSL text or the op's name
    ShaderType getShaderType() const;
    Variables getInputVars() const;
    Variable getOutputVar() const;

    Variable buildFwd(const Variables& xs);
    Variable buildBwd(const Variable& gy, uint32_t bwd_idx) const;

private:
    friend struct NodeAccess;
    explicit Function(std::shared_ptr<FunctionNode> node) : m_node(std::move(node)) {}
    std::shared_ptr<FunctionNode> m_node;
};

using Functions = std::vector<Function>;

}  // namespace dressi

template <>
struct std::hash<dressi::Function> {
    size_t operator()(const dressi::Function& f) const {
        return f ? std::hash<uint64_t>()(f.id()) : 0;
    }
};

template <>
struct std::less<dressi::Function> {
    bool operator()(const dressi::Function& a, const dressi::Function& b) const {
        return (a ? a.id() : 0) < (b ? b.id() : 0);
    }
};

#endif  // DRESSI_FUNCTION_H
