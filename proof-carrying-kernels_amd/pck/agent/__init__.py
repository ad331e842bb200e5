"""Parameter types of the agent's GEMV templates (reference `src/pck/agent/config.py`,
`src/pck/agent/column.py`): the knobs the row-major, INT8 and column-major template kernels
of libpck_hip.so are instantiated with.  The agent environment itself (episodes, regimes,
sandbox) is not part of this package."""
