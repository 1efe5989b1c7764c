"""Spectral/hash large-tensor route (host orchestration of the HIP pipeline)."""


class SpectralEngine:
    def step(self, param, grad, state, group):
        raise NotImplementedError("spectral route: HIP pipeline not built yet")

    def reset(self):
        pass
