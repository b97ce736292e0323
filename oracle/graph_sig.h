// graph_sig.h — a text signature of a built mg::Graph (TEST INFRASTRUCTURE ONLY).
//
// Compiled into both oracle/ref_harness.cpp (against the reference's include/mg-tensor.hpp)
// and tests/graph_harness.cpp (against this project's include/mg-tensor.hpp, which mirrors
// it field for field), so the same graph-building call on both sides can be compared node
// by node: one line per node with its op, type, shape, byte strides, integer parameters,
// float parameters as bit patterns, and each source as a named leaf ("L:<name>"), an unnamed
// leaf ("L:?") or an earlier node ("N:<index>").
#pragma once

#include <algorithm>
#include <cstdint>
#include <cstring>
#include <sstream>
#include <string>
#include <unordered_map>

namespace graph_sig {

inline std::string describe(const mg::Graph& g) {
    std::unordered_map<const mg::Tensor*, size_t> index;
    for (size_t i = 0; i < g.nodes.size(); i++) index[g.nodes[i]] = i;
    std::ostringstream os;
    for (size_t i = 0; i < g.nodes.size(); i++) {
        const mg::Tensor* t = g.nodes[i];
        os << i << " op=" << (int)t->op << " type=" << (int)t->type << " ne=";
        for (int d = 0; d < 4; d++) os << t->ne[d] << (d < 3 ? "," : "");
        os << " nb=";
        for (int d = 0; d < 4; d++) os << t->nb[d] << (d < 3 ? "," : "");
        os << " ip=";
        for (int d = 0; d < 4; d++) os << t->iparam[d] << (d < 3 ? "," : "");
        os << " fp=";
        for (int d = 0; d < 4; d++) {
            uint32_t u;
            std::memcpy(&u, &t->fparam[d], 4);
            os << std::hex << u << std::dec << (d < 3 ? "," : "");
        }
        os << " src=";
        for (const mg::Tensor* s : t->src) {
            if (!s) continue;
            const auto it = index.find(s);
            if (it != index.end()) os << "N:" << it->second << ";";
            else os << "L:" << (s->name.empty() ? "?" : s->name) << ";";
        }
        os << "\n";
    }
    return os.str();
}

// copies the signature into buf (NUL-terminated when it fits) and returns its length
inline int64_t copy_out(const std::string& s, char* buf, int64_t cap) {
    if (buf && cap > 0) {
        const size_t n = std::min((size_t)cap - 1, s.size());
        std::memcpy(buf, s.data(), n);
        buf[n] = 0;
    }
    return (int64_t)s.size();
}

}  // namespace graph_sig
