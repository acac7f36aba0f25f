"""CPU oracle of the reference training step -- test infrastructure only."""
