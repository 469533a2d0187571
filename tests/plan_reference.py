"""Python statement of the dense plan's processing order, kept as the test reference for the
library's native builder (cl_plan_locality_order, compactlogic_amd/csrc/plan.hip): same
traversal, same tie-breaking, so the two orders must be identical."""
import numpy as np
import torch


def dfs_forest(ra: torch.Tensor, rb: torch.Tensor, degree: torch.Tensor, in_dim: int):
    """Depth-first spanning forest of the graph whose edges are the runs (a, b): returns
    (roots, parent, children) as Python lists, parent[v] = -1 for a root and -2 for an input of
    degree 0.  Each search starts from the highest-degree unvisited input (lowest index on
    ties) and follows the neighbours in entry order; children are listed in discovery order."""
    a = ra.cpu().numpy().astype(np.int64)
    b = rb.cpu().numpy().astype(np.int64)
    deg = degree.cpu().numpy().astype(np.int64)
    src = np.concatenate((a, b))
    dst = np.concatenate((b, a))
    nbr = dst[np.argsort(src, kind="stable")].tolist()
    ptr = np.zeros(in_dim + 1, dtype=np.int64)
    np.cumsum(np.bincount(src, minlength=in_dim), out=ptr[1:])
    ptr = ptr.tolist()
    parent = [-2] * in_dim
    children = [[] for _ in range(in_dim)]
    roots = []
    for s in np.argsort(-deg, kind="stable").tolist():
        if parent[s] != -2 or deg[s] == 0:
            continue
        parent[s] = -1
        roots.append(s)
        stack = [[s, ptr[s]]]
        while stack:
            top = stack[-1]
            u, i = top
            if i < ptr[u + 1]:
                top[1] = i + 1
                v = nbr[i]
                if parent[v] == -2:
                    parent[v] = u
                    children[u].append(v)
                    stack.append([v, ptr[v]])
            else:
                stack.pop()
    return roots, parent, children


def locality_order(ra: torch.Tensor, rb: torch.Tensor, degree: torch.Tensor,
                   in_dim: int) -> torch.Tensor:
    """Processing order of the inputs for the input-gradient pass: preorder of the depth-first
    spanning forest of the run graph (dfs_forest), in which the children of every input are
    visited in increasing order of their subtree sizes (equal sizes in discovery order);
    inputs of degree 0 last.

    A subtree occupies consecutive positions, so a run between a parent and its child spans
    only the subtrees of the child's smaller siblings; visiting the small subtrees first keeps
    that span short for every child, and with it the time between the two reads of the
    run's grad_y row and of the shared input rows.  Deterministic."""
    dev = ra.device
    roots, parent, children = dfs_forest(ra, rb, degree, in_dim)
    size = [1] * in_dim
    # a parent is discovered before its children, so reversed discovery (preorder) order
    # visits every child before its parent
    pre = []
    for r in roots:
        stack = [r]
        while stack:
            u = stack.pop()
            pre.append(u)
            stack.extend(children[u])
    for u in reversed(pre):
        if parent[u] >= 0:
            size[parent[u]] += size[u]
    out = []
    for r in roots:
        stack = [r]
        while stack:
            u = stack.pop()
            out.append(u)
            ch = sorted(children[u], key=lambda v: size[v])   # stable: discovery order on ties
            stack.extend(reversed(ch))
    deg = degree.cpu().numpy()
    out.extend(np.nonzero(deg == 0)[0].tolist())
    return torch.as_tensor(np.asarray(out, dtype=np.int64), dtype=torch.int64, device=dev)
