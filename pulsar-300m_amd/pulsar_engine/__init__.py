"""Host side of the MI355X-native Pulsar self-speculative decode path."""
