"""The wiring the recurrent core runs on, in the reference's own layout.

A `Connectome` is an edge list in CSR order of W[post, pre]: `pre` and `post` are int64 and sorted by
(post, pre), so the edge arrays double as the CSR column and value order.  `sign` is +1/-1 per edge and
always follows the presynaptic neuron (Dale's law).  `neurons` is a table with at least the columns
`flow` ("afferent" / "intrinsic" / "efferent") and `super_class`.

Reference: chessfly/connectome.py:54-95.  `load_malecns` parses a local copy of the MaleCNS v1.0 release
(connectome.py:97-165) into the same graph; it never downloads (fetch the three feather files named in
MALECNS_FILES from MALECNS_URL yourself).  Synthetic graphs of the same size come from chessfly.synthetic.
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

    def summary(self) -> str:
        flows = self.neurons["flow"].value_counts().to_dict()
        return (f"{self.n_neurons:,} neurons, {self.n_edges:,} edges, "
                f"{float((self.sign > 0).float().mean()):.1%} excitatory, flow={flows}")


# ---- the MaleCNS v1.0 release, from local files ------------------------------------------------------------
MALECNS_URL = "https://storage.googleapis.com/flyem-male-cns/v1.0/connectome-data/flat-connectome"
MALECNS_FILES = {                               # local name -> released name (connectome.py:34-38)
    "body-annotations.feather": "body-annotations-male-cns-v1.0-minconf-0.5.feather",
    "body-neurotransmitters.feather": "body-neurotransmitters-male-cns-v1.0.feather",
    "connectome-weights.feather": "connectome-weights-male-cns-v1.0-minconf-0.5.feather",
}
# Dale's-law sign of the presynaptic transmitter; histamine and glutamate act through chloride channels in the
# fly, so both inhibit.  Anything else counts as excitatory (connectome.py:42-43, 153).
TRANSMITTER_SIGN = {"acetylcholine": 1.0, "dopamine": 1.0, "serotonin": 1.0, "octopamine": 1.0,
                    "gaba": -1.0, "glutamate": -1.0, "histamine": -1.0}
# super class -> flow: sensory classes are the inputs, motor / efferent / endocrine the outputs (connectome.py:46-51)
AFFERENT_CLASSES = frozenset({"ol_sensory", "cb_sensory", "vnc_sensory", "sensory_ascending", "sensory_descending",
                              "cb_sensory_tbc", "vnc_sensory_tbc", "sensory_ascending_tbc"})
EFFERENT_CLASSES = frozenset({"vnc_motor", "cb_motor", "vnc_efferent", "cb_efferent", "vnc_endocrine",
                              "cb_endocrine", "efferent_ascending", "efferent_descending"})
CACHE_VERSION = 2


def _malecns_neurons(data_dir: str) -> pd.DataFrame:
    """Bodies with a super class, sorted by body id: root_id, super_class, cell_type, nt, flow
    (connectome.py:106-119)."""
    import os
    import pyarrow.feather as feather
    ann = feather.read_feather(os.path.join(data_dir, "body-annotations.feather"),
                               columns=["bodyId", "superclass", "type"])
    ann = ann[ann["superclass"].notna()]
    nt = feather.read_feather(os.path.join(data_dir, "body-neurotransmitters.feather"), columns=["body", "consensus_nt"])
    nt = nt.rename(columns={"body": "root_id", "consensus_nt": "nt"})
    df = pd.DataFrame({"root_id": ann["bodyId"].astype(np.int64).to_numpy(),
                       "super_class": ann["superclass"].astype(str).to_numpy(),
                       "cell_type": ann["type"].astype(object).where(ann["type"].notna(), "").astype(str).to_numpy()})
    df = df.merge(nt, on="root_id", how="left")
    df["nt"] = df["nt"].astype(object).where(df["nt"].notna(), "unclear").astype(str)
    df["flow"] = np.where(df["super_class"].isin(AFFERENT_CLASSES), "afferent",
                          np.where(df["super_class"].isin(EFFERENT_CLASSES), "efferent", "intrinsic"))
    return df.sort_values("root_id").reset_index(drop=True)


def _malecns_pairs(data_dir: str, ids: np.ndarray, min_syn: int) -> pd.DataFrame:
    """Synapse counts between annotated bodies, pairs below min_syn dropped and repeated pairs summed,
    filtered batch by batch so the 152M-row table is never materialised whole (connectome.py:122-140)."""
    import os
    import pyarrow as pa
    import pyarrow.compute as pc
    reader = pa.ipc.open_file(os.path.join(data_dir, "connectome-weights.feather"))
    names = reader.schema.names
    cols = [next(c for c in cands if c in names)
            for cands in (("body_pre", "pre"), ("body_post", "post"), ("weight", "syn_count"))]
    keep = pa.array(ids)
    parts = []
    for i in range(reader.num_record_batches):
        batch = reader.get_batch(i).select(cols)
        mask = pc.and_(pc.and_(pc.is_in(batch.column(0), value_set=keep), pc.is_in(batch.column(1), value_set=keep)),
                       pc.greater_equal(batch.column(2), min_syn))
        batch = batch.filter(mask)
        if batch.num_rows:
            parts.append(batch)
    if not parts:
        return pd.DataFrame({"pre": np.zeros(0, np.int64), "post": np.zeros(0, np.int64), "syn": np.zeros(0)})
    table = pa.Table.from_batches(parts).rename_columns(["pre", "post", "syn"]).to_pandas()
    return table.groupby(["pre", "post"], sort=False, as_index=False)["syn"].sum()


def load_malecns(data_dir: str = "data", min_syn: int = 3, cache: bool = True) -> Connectome:
    """The MaleCNS v1.0 connectome from the three release files in data_dir (connectome.py:143-165): neurons
    are the bodies with a super class, in body-id order; edges the pairs with >= min_syn synapses in (post,
    pre) order; signs from the presynaptic transmitter.  The parsed graph is cached as
    data_dir/cache/malecns_min{min_syn}_v2.npz (plain arrays, read without pickle)."""
    import os
    cache_path = os.path.join(data_dir, "cache", f"malecns_min{min_syn}_v{CACHE_VERSION}.npz")
    if cache and os.path.exists(cache_path):
        with np.load(cache_path, allow_pickle=False) as z:
            neurons = pd.DataFrame({k[2:]: z[k] for k in z.files if k.startswith("n_")})
            return Connectome(neurons, torch.as_tensor(z["pre"]), torch.as_tensor(z["post"]),
                              torch.as_tensor(z["syn"]), torch.as_tensor(z["sign"]))
    missing = [f for f in MALECNS_FILES if not os.path.exists(os.path.join(data_dir, f))]
    if missing:
        raise FileNotFoundError(f"MaleCNS files missing in {data_dir}: {missing}; download "
                                f"{[MALECNS_FILES[f] for f in missing]} from {MALECNS_URL} and save them under "
                                "those local names")
    neurons = _malecns_neurons(data_dir)
    pairs = _malecns_pairs(data_dir, neurons["root_id"].to_numpy(), min_syn)
    node_of = pd.Series(np.arange(len(neurons)), index=neurons["root_id"].to_numpy())
    pre = node_of.loc[pairs["pre"].to_numpy()].to_numpy().astype(np.int64)
    post = node_of.loc[pairs["post"].to_numpy()].to_numpy().astype(np.int64)
    node_sign = neurons["nt"].map(TRANSMITTER_SIGN).fillna(1.0).to_numpy(dtype=np.float32)
    order = np.lexsort((pre, post))
    pre, post = pre[order], post[order]
    syn = pairs["syn"].to_numpy(dtype=np.float32)[order]
    sign = node_sign[pre]
    if cache:
        os.makedirs(os.path.dirname(cache_path), exist_ok=True)
        np.savez(cache_path, pre=pre, post=post, syn=syn, sign=sign,
                 **{f"n_{c}": neurons[c].to_numpy(dtype=np.int64 if c == "root_id" else str) for c in neurons.columns})
    return Connectome(neurons, torch.as_tensor(pre), torch.as_tensor(post), torch.as_tensor(syn), torch.as_tensor(sign))
