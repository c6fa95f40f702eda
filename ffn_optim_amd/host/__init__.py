"""Host side of the FFN operator: input contract, tiling plan, implementation selection."""
