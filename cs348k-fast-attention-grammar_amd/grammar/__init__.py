"""MI355X-native kernel grammar: IR, analysis, rewrites, stochastic rewrite
descent and a HIP (gfx950) renderer, plus the C-ABI runtime binding and the
hand-written CDNA4 baselines. Submodules import lazily; nothing here needs a
GPU or torch at import time."""
