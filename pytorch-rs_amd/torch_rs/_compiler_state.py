"""Process-wide state of torch_rs.compiler, kept in its own module so that it
survives a reload of torch_rs.compiler (python/torch_rs/_compiler_state.py)."""

default_backend = "inductor"
