"""CPU oracle for the routed-expert MoE path (test infrastructure only)."""
