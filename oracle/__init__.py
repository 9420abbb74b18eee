"""CPU oracle of soso-llm-core's decode path -- test infrastructure only."""
