"""MI355X-native forward evaluator of the alpha-fly connectome chess network.

Modules mirror the reference package `chessfly`: `brain` (ConnectomeRNN, LightCone), `model`
(FlyChessNet, Evaluator, RunningNorm, ModelConfig, load_weights), `connectome` (Connectome), `encoding`
(feature and move-index constants).  `synthetic` draws MaleCNS-sized graphs, weights and boards from a seed.
The compute runs in libflyeval.so (gfx950 HIP kernels behind a C ABI, include/flyeval.h), loaded by `_hip`.
"""
