"""Chain-rule programs used by the fixpoint tests (plan arrays in the layout of
include/xlog_hip.h: [n_rules, per rule: head, hv0, hv1, n_body, (pred, v0, v1) * n_body]).

Each is a recursive program over binary relations whose rule bodies form a
path between the head variables, in the style of the reference's recursion
tests (crates/xlog-integration-tests/tests/real_world_tests.rs) and its
example programs (examples/xlog/); the cyclic plans at the end have an atom
whose two variables are both bound when it is joined (the reference's
left-deep lowering then joins on both keys, lower.rs build_join_tree)."""

X, Y, Z, P, Q, V, W = 0, 1, 2, 3, 4, 5, 6


def left_tc_plan(edge=0, reach=1):
    """reach(X,Y) :- edge(X,Y).  reach(X,Z) :- edge(X,Y), reach(Y,Z)."""
    return [2, reach, X, Y, 1, edge, X, Y, reach, X, Z, 2, edge, X, Y, reach, Y, Z]


def nonlinear_tc_plan(edge=0, path=1):
    """path(X,Y) :- edge(X,Y).  path(X,Z) :- path(X,Y), path(Y,Z)."""
    return [2, path, X, Y, 1, edge, X, Y, path, X, Z, 2, path, X, Y, path, Y, Z]


def same_generation_plan(flat=0, up=1, down=2, sg=3):
    """sg(X,Y) :- flat(X,Y).  sg(X,Y) :- up(X,P), sg(P,Q), down(Q,Y)."""
    return [2, sg, X, Y, 1, flat, X, Y, sg, X, Y, 3, up, X, P, sg, P, Q, down, Q, Y]


def same_generation_par_plan(flat=0, par=1, sg=2):
    """sg(X,Y) :- flat(X,Y).  sg(X,Y) :- par(X,P), sg(P,Q), par(Y,Q)   (par read backward)."""
    return [2, sg, X, Y, 1, flat, X, Y, sg, X, Y, 3, par, X, P, sg, P, Q, par, Y, Q]


def parity_plan(edge=0, odd=1, even=2):
    """Walks of odd / even length (mutual recursion over two IDB predicates):
    odd(X,Y) :- edge(X,Y).  even(X,Z) :- odd(X,Y), edge(Y,Z).  odd(X,Z) :- even(X,Y), edge(Y,Z)."""
    return [3, odd, X, Y, 1, edge, X, Y,
            even, X, Z, 2, odd, X, Y, edge, Y, Z,
            odd, X, Z, 2, even, X, Y, edge, Y, Z]


def parity_left_plan(edge=0, odd=1, even=2):
    """The same walks with the IDB atom last: odd(X,Y) :- edge(X,Y).  even(X,Z) :- edge(X,Y), odd(Y,Z).
    odd(X,Z) :- edge(X,Y), even(Y,Z).  Every variant is a CSR-left product and each head has one, so every
    iteration is fused; the two deltas alternate between empty and non-empty."""
    return [3, odd, X, Y, 1, edge, X, Y,
            even, X, Z, 2, edge, X, Y, odd, Y, Z,
            odd, X, Z, 2, edge, X, Y, even, Y, Z]


def symmetric_plan(edge=0, sym=1):
    """sym(X,Y) :- edge(Y,X).  sym(X,Y) :- sym(Y,X).  sym(X,Z) :- sym(X,Y), edge(Y,Z)."""
    return [3, sym, X, Y, 1, edge, Y, X,
            sym, X, Y, 1, sym, Y, X,
            sym, X, Z, 2, sym, X, Y, edge, Y, Z]


def quad_plan(a=0, b=1, p=2):
    """p(X,Y) :- a(X,Y).  p(X,W) :- a(X,Y), p(Y,Z), b(Z,V), p(V,W)   (four atoms, two IDB)."""
    return [2, p, X, Y, 1, a, X, Y, p, X, W, 4, a, X, Y, p, Y, Z, b, Z, V, p, V, W]


def scrambled_chain_plan(a=0, b=1, p=2):
    """p(X,Y) :- a(X,Y).  p(X,W) :- a(X,Y), b(Z,W), p(Y,Z): a chain whose second atom
    shares no variable with the first (left-deep evaluation cannot take it)."""
    return [2, p, X, Y, 1, a, X, Y, p, X, W, 3, a, X, Y, b, Z, W, p, Y, Z]


def ordered_chain_plan(a=0, b=1, p=2):
    """The same program as scrambled_chain_plan with the body in path order."""
    return [2, p, X, Y, 1, a, X, Y, p, X, W, 3, a, X, Y, p, Y, Z, b, Z, W]


def triangle_closure_plan(edge=0, r=1):
    """r(X,Y) :- edge(X,Y).  r(X,Z) :- r(X,Y), edge(Y,Z), edge(Z,X)   (the last atom closes a triangle:
    both of its variables are bound)."""
    return [2, r, X, Y, 1, edge, X, Y, r, X, Z, 3, r, X, Y, edge, Y, Z, edge, Z, X]


def triangles_plan(edge=0, tri=1):
    """tri(X,Z) :- edge(X,Y), edge(Y,Z), edge(Z,X)   (non-recursive: one iteration derives nothing)."""
    return [1, tri, X, Z, 3, edge, X, Y, edge, Y, Z, edge, Z, X]


def filtered_tc_plan(a=0, keep=1, b=2, p=3):
    """p(X,Y) :- a(X,Y).  p(X,Z) :- p(X,Y), keep(Y,X), b(Y,Z)   (a two-key step in the middle, its atom's
    columns in the reverse of the binding's order)."""
    return [2, p, X, Y, 1, a, X, Y, p, X, Z, 3, p, X, Y, keep, Y, X, b, Y, Z]


def flat_sg_plan(flat=0, par=1, sg=2):
    """sg(X,Y) :- flat(X,Y).  sg(X,Y) :- par(X,P), sg(P,Q), par(Y,Q), flat(X,Y)   (four atoms, the last a
    two-key step)."""
    return [2, sg, X, Y, 1, flat, X, Y, sg, X, Y, 4, par, X, P, sg, P, Q, par, Y, Q, flat, X, Y]
