// planner.hpp — static memory plan of a compute_graph: liveness and arena
// offsets. The algorithm is the reference's (S/graph/planner.hpp:52-150):
// tensor t lives over the node interval [first, last] (inputs from node 0,
// outputs to the last node, a node's operands and results live together);
// tensors are placed largest first, each at the lowest aligned offset clear
// of every placed tensor whose interval intersects its own (greedy by size).
// Invariants checked by plan_is_valid:
//   P1 offset % plan_alignment == 0;   P2 offset + bytes <= arena_bytes;
//   P3 tensors with intersecting intervals occupy disjoint bytes.
// Only the alignment differs (plan_alignment, 256 bytes on the device).
#pragma once

#include "graph.hpp"

#include <algorithm>
#include <numeric>

namespace syn::graph {

struct live_interval {
    std::size_t first = 0;
    std::size_t last = 0;
};

inline bool intersects(live_interval a, live_interval b) noexcept {
    return a.first <= b.last && b.first <= a.last;
}

inline std::vector<live_interval> liveness(const compute_graph& g) {
    const std::size_t n = g.nodes().size();
    const std::size_t end = n == 0 ? 0 : n - 1;
    std::vector<live_interval> live(g.tensors().size());
    for (std::size_t i = 0; i < n; ++i) {
        for (tensor_id t : results(g.nodes()[i])) {
            live[t] = {i, i};
        }
    }
    for (tensor_id t : g.inputs()) {
        live[t] = {0, 0};
    }
    for (std::size_t i = 0; i < n; ++i) {
        for (tensor_id t : operands(g.nodes()[i])) {
            live[t].last = std::max(live[t].last, i);
        }
    }
    for (tensor_id t : g.outputs()) {
        live[t].last = end;
    }
    return live;
}

struct memory_plan {
    std::vector<std::size_t> offset;
    std::size_t arena_bytes = 0;
    std::size_t naive_bytes = 0;  // no aliasing at all
};

constexpr std::size_t align_up(std::size_t n) noexcept {
    return (n + plan_alignment - 1) / plan_alignment * plan_alignment;
}

// The plan for given live intervals (at least liveness(g)'s): a caller that
// runs some nodes' work later than the graph says extends its tensors'
// intervals first.
inline memory_plan plan(const compute_graph& g, const std::vector<live_interval>& live) {
    const auto& tensors = g.tensors();
    std::vector<tensor_id> order(tensors.size());
    std::iota(order.begin(), order.end(), tensor_id{0});
    std::stable_sort(order.begin(), order.end(),
                     [&](tensor_id a, tensor_id b) { return tensors[a].bytes > tensors[b].bytes; });
    memory_plan p;
    p.offset.assign(tensors.size(), 0);
    std::vector<tensor_id> placed, clash;
    for (tensor_id t : order) {
        p.naive_bytes += align_up(tensors[t].bytes);
        clash.clear();
        for (tensor_id u : placed) {
            if (intersects(live[t], live[u])) {
                clash.push_back(u);
            }
        }
        std::sort(clash.begin(), clash.end(), [&](tensor_id a, tensor_id b) { return p.offset[a] < p.offset[b]; });
        std::size_t at = 0;
        for (tensor_id u : clash) {
            if (at + tensors[t].bytes <= p.offset[u]) {
                break;  // fits in the gap below u
            }
            at = std::max(at, align_up(p.offset[u] + tensors[u].bytes));
        }
        p.offset[t] = at;
        p.arena_bytes = std::max(p.arena_bytes, align_up(at + tensors[t].bytes));
        placed.push_back(t);
    }
    return p;
}

inline memory_plan plan(const compute_graph& g) {
    return plan(g, liveness(g));
}

inline bool plan_is_valid(const compute_graph& g, const memory_plan& p, const std::vector<live_interval>& live) {
    const auto& tensors = g.tensors();
    if (p.offset.size() != tensors.size()) {
        return false;
    }
    for (std::size_t t = 0; t < tensors.size(); ++t) {
        if (p.offset[t] % plan_alignment != 0 || p.offset[t] + tensors[t].bytes > p.arena_bytes) {
            return false;  // P1, P2
        }
        for (std::size_t u = t + 1; u < tensors.size(); ++u) {
            const bool apart =
                p.offset[t] + tensors[t].bytes <= p.offset[u] || p.offset[u] + tensors[u].bytes <= p.offset[t];
            if (intersects(live[t], live[u]) && !apart && tensors[t].bytes > 0 && tensors[u].bytes > 0) {
                return false;  // P3
            }
        }
    }
    return true;
}

inline bool plan_is_valid(const compute_graph& g, const memory_plan& p) {
    return plan_is_valid(g, p, liveness(g));
}

}  // namespace syn::graph
