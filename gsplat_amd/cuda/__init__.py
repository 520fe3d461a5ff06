"""Op layer: torch.ops.gsplat registration (_backend), host-side op
implementations (_ops) and the autograd-facing wrappers (_wrapper)."""
