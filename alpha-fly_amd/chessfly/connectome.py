"""The wiring the recurrent core runs on, in the reference's own layout.

A `Connectome` is an edge list in CSR order of W[post, pre]: `pre` and `post` are int64 and sorted by
(post, pre), so the edge arrays double as the CSR column and value order.  `sign` is +1/-1 per edge and
always follows the presynaptic neuron (Dale's law).  `neurons` is a table with at least the columns
`flow` ("afferent" / "intrinsic" / "efferent") and `super_class`.

Reference: chessfly/connectome.py:54-95.  Reading the MaleCNS release itself (connectome.py:97-165) is not part
of this package: it needs a network download, and the evaluator takes any graph in this layout.  Synthetic graphs
of the MaleCNS size come from chessfly.synthetic.
"""

from __future__ import annotations

import dataclasses

import numpy as np
import pandas as pd
import torch


@dataclasses.dataclass
class Connectome:
    neurons: pd.DataFrame     # index 0..N-1; columns include super_class and flow
    pre: torch.Tensor         # (E,) int64  presynaptic node index
    post: torch.Tensor        # (E,) int64  postsynaptic node index, non-decreasing
    syn_count: torch.Tensor   # (E,) float32
    sign: torch.Tensor        # (E,) float32 +1 / -1, the sign of the presynaptic neuron

    @property
    def n_neurons(self) -> int:
        return len(self.neurons)

    @property
    def n_edges(self) -> int:
        return int(self.pre.numel())

    @property
    def weight(self) -> torch.Tensor:
        """Each edge's synapse count over its postsynaptic neuron's total input (connectome.py:70-74):
        the inputs of every neuron sum to 1 (a neuron without inputs divides by 1)."""
        total = torch.zeros(self.n_neurons, dtype=self.syn_count.dtype).index_add_(0, self.post, self.syn_count)
        return self.syn_count / total[self.post].clamp_min(1.0)

    def nodes(self, flow: str) -> torch.Tensor:
        """Sorted indices of the neurons whose flow is `flow` (connectome.py:76-77)."""
        return torch.as_tensor(np.flatnonzero((self.neurons["flow"] == flow).to_numpy()), dtype=torch.long)

    def nodes_of_superclass(self, *names: str) -> torch.Tensor:
        """Sorted indices of the neurons in any of the given super classes (connectome.py:79-80)."""
        return torch.as_tensor(np.flatnonzero(self.neurons["super_class"].isin(names).to_numpy()), dtype=torch.long)

    def shuffled(self, seed: int = 0) -> "Connectome":
        """Degree-preserving control graph (connectome.py:82-89).

        The presynaptic column is permuted over all edges with torch's seeded `randperm`, so every neuron keeps
        its in-degree and its out-degree, and the edges are re-sorted into (post, pre) order with a stable
        lexicographic sort.  Signs are re-derived from the new presynaptic neuron.  The permutation can create
        self-loops and repeated (post, pre) pairs; both stay as separate edges, which the sparse products sum.
        """
        gen = torch.Generator().manual_seed(seed)
        new_pre = self.pre[torch.randperm(self.n_edges, generator=gen)]
        order = torch.as_tensor(np.lexsort((new_pre.numpy(), self.post.numpy())))
        sign_of = torch.ones(self.n_neurons, dtype=self.sign.dtype)
        sign_of[self.pre] = self.sign
        pre = new_pre[order]
        return Connectome(self.neurons, pre, self.post[order], self.syn_count[order], sign_of[pre])
