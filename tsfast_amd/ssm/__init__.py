"""NeuralStateSpace backward: the sequence-parallel adjoint scan (``adjoint_hip``)."""
